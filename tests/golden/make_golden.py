"""Write the golden vectors from the reference operator itself.

Runs only in a container that holds the reference checkout (it imports
``reference moe/ref_moe.py`` by path). For every workload of
``flashinfer_mlsys_amd.workloads`` it regenerates the seeded inputs, calls the
reference ``run`` once, and records:

* sha256 of each input (the weights once, in ``weights.json``)
* the selected expert ids per token, ascending (captured from the reference's
  third ``torch.topk`` call, ``ref_moe.py:119``)
* per-local-expert token lists (captured from its ``torch.nonzero`` calls,
  ``ref_moe.py:144``), concatenated, with counts
* the bf16 output: in full for T <= 16, otherwise selected rows plus the sha256
  of the whole output
* the selection margins and the torch build / CPU capability used

The fixtures are data (inputs are regenerated from seeds; expected outputs are
stored). Usage: ``python tests/golden/make_golden.py [workload ...]``.

``python tests/golden/make_golden.py ties`` writes ``ties_<case>.npz`` for the
exact-tie routing cases of ``tests/tie_cases.py`` (selections that
torch.topk(sorted=False)'s nth_element order decides): the logits and bias
themselves (small), the reference's selection in its own order and sorted, and
its bf16 output rows, with hidden states from a seeded generator.
"""
from __future__ import annotations

import gc
import importlib.util
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from flashinfer_mlsys_amd import workloads as wl  # noqa: E402
from oracle import cpu_ref  # noqa: E402

REF_PATH = "/root/reference/reference moe/ref_moe.py"
OUT_DIR = os.path.join(ROOT, "tests", "golden")
FULL_OUTPUT_MAX_T = 16
N_SAMPLE_ROWS = 8


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_moe", REF_PATH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


class Capture:
    """Records the reference's own topk / nonzero results during one call."""

    def __init__(self):
        self.topk = []
        self.nonzero = []

    def __enter__(self):
        self._topk, self._nonzero = torch.topk, torch.nonzero
        cap = self

        def topk(*a, **k):
            r = cap._topk(*a, **k)
            cap.topk.append(r.indices.clone())
            return r

        def nonzero(*a, **k):
            r = cap._nonzero(*a, **k)
            cap.nonzero.append(r.clone())
            return r

        torch.topk, torch.nonzero = topk, nonzero
        return self

    def __exit__(self, *exc):
        torch.topk, torch.nonzero = self._topk, self._nonzero
        return False


def sample_rows(T, lists, seed):
    """Rows with 0, 1 and >= 2 local pairs where they exist, then random ones."""
    npairs = np.zeros(T, dtype=np.int64)
    for l in lists:
        npairs[l.numpy()] += 1
    rng = np.random.default_rng(seed)
    picks = []
    for cond in (npairs == 0, npairs == 1, npairs >= 2, npairs == npairs.max()):
        idx = np.nonzero(cond)[0]
        if len(idx):
            picks.append(int(rng.choice(idx)))
    while len(set(picks)) < min(N_SAMPLE_ROWS, T):
        picks.append(int(rng.integers(T)))
    return sorted(set(picks))[:N_SAMPLE_ROWS]


def main(names):
    ref = load_reference()
    os.makedirs(OUT_DIR, exist_ok=True)
    w13, s13, w2, s2 = wl.make_weights()
    weights_meta = {
        "weight_seed": wl.WEIGHT_SEED,
        "gemm1_weights": wl.fingerprint(w13), "gemm1_weights_scale": wl.fingerprint(s13),
        "gemm2_weights": wl.fingerprint(w2), "gemm2_weights_scale": wl.fingerprint(s2),
    }
    with open(os.path.join(OUT_DIR, "weights.json"), "w") as f:
        json.dump(weights_meta, f, indent=1)
    for name in names:
        w = wl.WORKLOADS[name]
        args = wl.make_inputs(name)
        t0 = time.time()
        with Capture() as cap:
            out = ref.run(*args)
        dt = time.time() - t0
        topk_idx = cap.topk[2]
        assert topk_idx.shape == (w.T, 8)
        sel = torch.sort(topk_idx, dim=1).values
        # token lists: one nonzero call per local expert that has at least one token
        lists, it = [], iter(cap.nonzero)
        for le in range(32):
            ge = w.local_expert_offset + le
            if 0 <= ge < 256 and bool((topk_idx == ge).any()):
                lists.append(next(it).squeeze(1))
            else:
                lists.append(torch.empty(0, dtype=torch.int64))
        assert next(it, None) is None
        counts = np.array([len(l) for l in lists], dtype=np.int32)
        g_margin, e_margin = cpu_ref.selection_margins(args[0], args[1])
        out_u16 = out.view(torch.int16).numpy().view(np.uint16)
        rows = np.arange(w.T) if w.T <= FULL_OUTPUT_MAX_T else np.array(sample_rows(w.T, lists, w.seed))
        np.savez_compressed(
            os.path.join(OUT_DIR, f"{name}.npz"),
            T=w.T, local_expert_offset=w.local_expert_offset, seed=w.seed,
            routed_scaling_factor=w.routed_scaling_factor,
            sel_ids=sel.numpy().astype(np.uint8),
            counts=counts,
            token_lists=np.concatenate([l.numpy() for l in lists]).astype(np.int32)
            if counts.sum() else np.zeros(0, np.int32),
            out_rows=rows.astype(np.int32),
            out_bf16=out_u16[rows],
            out_sha256=wl.fingerprint(out),
            in_sha256=np.array([wl.fingerprint(a) for a in args[:4]]),
            margins_ulp=np.array([g_margin, e_margin]),
            torch_version=torch.__version__,
            cpu_capability=torch.backends.cpu.get_cpu_capability(),
            num_threads=torch.get_num_threads(),
        )
        print(f"{name}: T={w.T} P={counts.sum()} E_act={(counts > 0).sum()} "
              f"margins={g_margin:.1f}/{e_margin:.1f} ulp ref_run={dt:.1f}s", flush=True)
        del args, out, cap
        gc.collect()


TIE_HIDDEN_SEED = 7000
TIE_ROWS = 16


def main_ties():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import tie_cases as tc
    ref = load_reference()
    w13, s13, w2, s2 = wl.make_weights()
    for i, name in enumerate(tc.CASES):
        logits, bias, offset, rsf = tc.case_tensors(name)
        T = logits.shape[0]
        _, _, hidden, hscale = wl.make_activations(T, TIE_HIDDEN_SEED + i)
        t0 = time.time()
        with Capture() as cap:
            out = ref.run(logits, bias, hidden, hscale, w13, s13, w2, s2, offset, rsf)
        topk_idx = cap.topk[2]
        rows = np.arange(T) if T <= TIE_ROWS else np.sort(
            np.random.default_rng(TIE_HIDDEN_SEED + i).choice(T, TIE_ROWS, replace=False))
        out_u16 = out.view(torch.int16).numpy().view(np.uint16)
        np.savez_compressed(
            os.path.join(OUT_DIR, f"ties_{name}.npz"),
            T=T, local_expert_offset=offset, routed_scaling_factor=rsf, hidden_seed=TIE_HIDDEN_SEED + i,
            logits=logits.numpy(), bias_bf16=bias.view(torch.int16).numpy().view(np.uint16),
            topk_idx=topk_idx.numpy().astype(np.int16),
            sel_ids=torch.sort(topk_idx, dim=1).values.numpy().astype(np.uint8),
            out_rows=rows.astype(np.int32), out_bf16=out_u16[rows], out_sha256=wl.fingerprint(out),
            in_sha256=np.array([wl.fingerprint(a) for a in (logits, bias, hidden, hscale)]),
            torch_version=torch.__version__,
            cpu_capability=torch.backends.cpu.get_cpu_capability(),
        )
        print(f"ties_{name}: T={T} offset={offset} ref_run={time.time() - t0:.1f}s", flush=True)
        del out, cap
        gc.collect()


if __name__ == "__main__":
    if sys.argv[1:] == ["ties"]:
        main_ties()
    else:
        main(sys.argv[1:] or list(wl.WORKLOADS))
