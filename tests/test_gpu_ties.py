"""Exact-tie routing on the GPU against the reference (tests/golden/ties_*.npz,
written by running reference moe/ref_moe.py on tests/tie_cases.py inputs).

Where equal scores straddle the group or expert cut, the reference keeps the
entries torch.topk(sorted=False) -- std::nth_element -- leaves in front; the
kernels detect such tokens and replay that order. Bars: selection bit-exact;
weights within 8 fp32 ulps of the oracle's; output within atol=1e-2, rtol=2e-2
of the reference's rows and of the oracle in full.
"""
import os

import numpy as np
import pytest
import torch

import flashinfer_mlsys_amd as fm
from flashinfer_mlsys_amd import workloads as wl
from oracle import cpu_ref

from conftest import GOLDEN_DIR, assert_close_bf16, bf16_bits_to_f32

import tie_cases as tc

pytestmark = pytest.mark.gpu

SHAPES = [fm.SHAPE_AUTO, fm.SHAPE_PREFILL]
TOPK_IDS_OFFSET = 512  # workspace: the 512-byte dispatch header, then topk_ids int32 [T, 8]


def _say(msg):
    print(msg, flush=True)


def _fixture(name):
    path = os.path.join(GOLDEN_DIR, f"ties_{name}.npz")
    if not os.path.exists(path):
        pytest.skip(f"tie fixture {name} not generated")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _routing_inputs(z):
    lg = torch.from_numpy(z["logits"])
    b = torch.from_numpy(z["bias_bf16"].view(np.int16)).view(torch.bfloat16)
    return lg, b


@pytest.mark.parametrize("name", tc.CASES)
def test_route_ties_match_reference(dev, name):
    z = _fixture(name)
    lg, b = _routing_inputs(z)
    rsf = float(z["routed_scaling_factor"])
    _say(f"ties route {name} T={lg.shape[0]}")
    ids, w, _ = fm.route(lg.to(dev), b.to(dev), rsf)
    ids = ids.cpu().numpy()
    np.testing.assert_array_equal(ids, z["sel_ids"].astype(np.int32))
    _, dense, _, _, _ = cpu_ref.route(lg, b, rsf)
    ref_w = torch.gather(dense, 1, torch.from_numpy(ids).long()).numpy()
    np.testing.assert_allclose(w.cpu().numpy(), ref_w, rtol=4e-7 * 8, atol=0)


@pytest.mark.parametrize("name", tc.CASES)
@pytest.mark.parametrize("shape", SHAPES, ids=["auto", "prefill"])
def test_route_dispatch_ties_match_reference(dev, name, shape):
    z = _fixture(name)
    lg, b = _routing_inputs(z)
    off = int(z["local_expert_offset"])
    _say(f"ties route_dispatch {name} shape={shape}")
    ids, _, header, perm_tok, _, _ = fm.route_dispatch(lg.to(dev), b.to(dev), off,
                                                       float(z["routed_scaling_factor"]), shape=shape)
    np.testing.assert_array_equal(ids.cpu().numpy(), z["sel_ids"].astype(np.int32))
    sel = z["sel_ids"].astype(np.int64)
    counts = np.array([(sel == off + le).any(1).sum() if 0 <= off + le < 256 else 0 for le in range(32)])
    np.testing.assert_array_equal(header.cpu().numpy()[:32], counts)
    pt = perm_tok.cpu().numpy()
    pos = 0
    for le in range(32):
        want = np.nonzero((sel == off + le).any(1))[0] if 0 <= off + le < 256 else np.zeros(0, np.int64)
        np.testing.assert_array_equal(pt[pos:pos + len(want)], want)
        pos += len(want)


@pytest.mark.parametrize("name", tc.CASES)
@pytest.mark.parametrize("shape", SHAPES, ids=["auto", "prefill"])
def test_forward_ties_match_reference(weights, dev, name, shape):
    """The whole operator on the tie inputs (in the decode shape the cases of at
    most 8 tokens are routed inside GEMM1, whose workgroup 0 also stores the ids
    in the workspace, checked here)."""
    z = _fixture(name)
    lg, b = _routing_inputs(z)
    T, off, rsf = int(z["T"]), int(z["local_expert_offset"]), float(z["routed_scaling_factor"])
    _, _, hs, hss = wl.make_activations(T, int(z["hidden_seed"]))
    for t, h in zip((lg, b, hs, hss), z["in_sha256"]):
        assert wl.fingerprint(t) == str(h), f"{name}: inputs do not regenerate identically"
    _say(f"ties forward {name} T={T} shape={shape}")
    gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
    ws = torch.zeros(fm.workspace_size(T), dtype=torch.uint8, device=dev)
    out = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    fm._forward(shape, *gpu, off, rsf, out, ws)
    torch.cuda.synchronize()
    ids = ws[TOPK_IDS_OFFSET:TOPK_IDS_OFFSET + T * 32].view(torch.int32).reshape(T, 8).cpu().numpy()
    np.testing.assert_array_equal(ids, z["sel_ids"].astype(np.int32))
    got = out.float().cpu().numpy()
    assert_close_bf16(got[z["out_rows"]], bf16_bits_to_f32(z["out_bf16"]), f"{name}: reference rows")
    ref = cpu_ref.run(lg, b, hs, hss, *weights[0], off, rsf).float().numpy()
    assert_close_bf16(got, ref, f"{name}: oracle")
