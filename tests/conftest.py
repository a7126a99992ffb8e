import os
import sys

import numpy as np
import torch
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

# Bar for the bf16 output against the reference (torch.allclose semantics).
ATOL = 1e-2
RTOL = 2e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU with ROCm")


def load_golden(name):
    path = os.path.join(GOLDEN_DIR, f"{name}.npz")
    if not os.path.exists(path):
        pytest.skip(f"golden fixture {name} not generated")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_lists(g):
    """Per-local-expert token lists from a golden fixture."""
    out, pos = [], 0
    for c in g["counts"].tolist():
        out.append(g["token_lists"][pos:pos + c].astype(np.int64))
        pos += c
    return out


def bf16_bits_to_f32(u16):
    u16 = np.asarray(u16, dtype=np.uint16)
    return (u16.astype(np.uint32) << 16).view(np.float32)


def assert_close_bf16(actual_f32, expected_f32, what=""):
    a = np.asarray(actual_f32, dtype=np.float64)
    e = np.asarray(expected_f32, dtype=np.float64)
    bad = np.abs(a - e) > ATOL + RTOL * np.abs(e)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements outside atol={ATOL} rtol={RTOL}; "
            f"first at {tuple(i)}: got {a[tuple(i)]!r} want {e[tuple(i)]!r}; "
            f"max abs err {np.abs(a - e).max():.4g}")

from oracle import np_ref  # noqa: E402  (test infrastructure)


# --- GPU fixtures shared by the GPU test files (one weight upload per session) ---
@pytest.fixture(scope="session")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def weights(dev):
    """Expert weights (cpu, gpu), checked against the fingerprints the fixtures were made with."""
    import json
    from flashinfer_mlsys_amd import workloads as wl
    print("generating expert weights", flush=True)
    cpu = wl.make_weights()
    with open(os.path.join(GOLDEN_DIR, "weights.json")) as f:
        meta = json.load(f)
    for t, k in zip(cpu, ["gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale"]):
        assert wl.fingerprint(t) == meta[k], f"{k} does not regenerate identically on this host"
    gpu = [t.to(dev) for t in cpu]
    torch.cuda.synchronize()
    return cpu, gpu


# --- Trace-replay cases -----------------------------------------------------
from flashinfer_mlsys_amd import workloads as wl  # noqa: E402

# Token counts and local-expert offsets of the official FlashInfer-Trace
# workloads for this operator (input_analysis/input_check.ipynb cell 7: T from
# 1 to 14107, offsets 0..224), with their routing-bias profile (every bias
# 4.9375 or 4.96875, two adjacent bf16 values, cell 5). The uuids are the first
# of "mi355x-trace-<T>-<offset>-<k>" whose routing has at least one local pair
# and selection margins of at least 8 fp32 ulps (test_trace checks both).
# Together with the two largest (T = 11,948 at offset 128 and T = 14,107 at
# offset 32, the workloads trace_t11948 / trace_t14107) these are all 19 official
# (T, offset) pairs, in the notebook's order.
TRACE_CASES = [c for c in wl.OFFICIAL_TRACE if c[1] < 4096]
# The official (T, offset) pairs (input_analysis/input_check.ipynb cell 7).
OFFICIAL_PAIRS = [(7, 192), (1, 32), (32, 32), (80, 96), (901, 96), (16, 224), (15, 32), (14, 0), (14107, 32),
                  (11948, 128), (62, 96), (59, 160), (58, 64), (57, 96), (56, 64), (55, 128), (54, 128),
                  (53, 32), (52, 160)]


def trace_case_tensors(uuid, T):
    """Recorded inputs of a trace case: fp32 N(0,1) logits and the two-level bf16 bias."""
    from flashinfer_mlsys_amd import trace, workloads as wl
    seed = trace.TraceWorkload(uuid, T, {}).seed
    return wl._normal((seed, 10), (T, 256), 1.0), wl.official_bias(seed)


def write_trace_cases(root, cases=TRACE_CASES):
    from flashinfer_mlsys_amd import trace
    rows = []
    for uuid, T, offset in cases:
        lg, b = trace_case_tensors(uuid, T)
        rows.append((uuid, T, offset, 2.5, {"routing_logits": lg, "routing_bias": b}))
    return trace.write_trace_set(str(root), rows)


def quant_edge_rows():
    """bf16 rows whose blocks have closed-form quantisations: a power-of-two scale
    (amax 448 * 2^-3) with every e4m3 value and every midpoint between two (ties);
    an all-zero block; -0.0; bf16 subnormals; the largest bf16 values."""
    vals = np_ref.e4m3_table()
    fin = np.unique(vals[np.isfinite(vals) & (vals >= 0)])
    mids = (fin[:-1] + fin[1:]) / 2
    rows = np.zeros((3, 7168), dtype=np.float32)
    scale = 2.0 ** -3
    block = np.concatenate([[448.0], fin[:63], -mids[:64]])[:128] * scale  # exact in bf16
    rows[0, :128] = block
    rows[0, 128:256] = -block[::-1]
    rows[1, 256:384] = np.float32(2.0 ** -130) * np.arange(1, 129, dtype=np.float32)  # bf16 subnormals
    rows[1, 384] = -0.0
    rows[2, 512:640] = np.linspace(-3.3e38, 3.3e38, 128, dtype=np.float32)
    x = torch.from_numpy(rows).to(torch.bfloat16)
    assert torch.equal(x[0, :128].float(), torch.from_numpy(block.astype(np.float32)))
    return x
