"""moe_fp8_forward_noalloc, the allocation-free entry point (its workspace is a
library-owned device array), against moe_fp8_forward with a caller workspace:
bit-identical outputs on consecutive calls, each smaller or different from the
one before (the array keeps the previous call's contents), and a clear error
beyond its token limit. Calls go through the C ABI."""
import numpy as np
import pytest
import torch

import flashinfer_mlsys_amd as fm
from flashinfer_mlsys_amd import _lib, workloads as wl

pytestmark = pytest.mark.gpu

# (T, offset, activation seed): T=64 then smaller calls; T <= 8 routes inside GEMM1
CALLS = [(64, 0, 8101), (5, 0, 8102), (37, 96, 8103), (1, 0, 1102)]


def _noalloc(lib, gpu, T, offset, rsf, out, dev):
    return lib.moe_fp8_forward_noalloc(*[t.data_ptr() for t in gpu], T, offset, rsf, out.data_ptr(),
                                       torch.cuda.current_stream(dev).cuda_stream)


def test_noalloc_matches_forward(weights, dev):
    lib = _lib.load()
    for T, offset, seed in CALLS:
        print(f"noalloc T={T} offset={offset} seed={seed}", flush=True)
        lg, b, hs, hss = wl.make_activations(T, seed, offset)
        gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
        ref = fm.run(*gpu, offset, 2.5)  # moe_fp8_forward with its own workspace
        out = torch.full((T, 7168), -7.0, dtype=torch.bfloat16, device=dev)
        _lib.check(_noalloc(lib, gpu, T, offset, 2.5, out, dev), "moe_fp8_forward_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"T={T} offset={offset}"
        assert out.float().abs().sum().item() > 0, "the call must route some pairs locally"


def test_noalloc_limits(weights, dev):
    lib = _lib.load()
    assert _lib.MOE_FP8_NOALLOC_MAX_TOKENS == 64
    lg, b, hs, hss = wl.make_activations(65, 8104)
    gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
    out = torch.zeros((65, 7168), dtype=torch.bfloat16, device=dev)
    assert _noalloc(lib, gpu, 65, 0, 2.5, out, dev) == _lib.MOE_ERR_NOALLOC_SIZE
    assert b"MOE_FP8_NOALLOC_MAX_TOKENS" in lib.moe_fp8_strerror(_lib.MOE_ERR_NOALLOC_SIZE)
    assert _noalloc(lib, gpu, -1, 0, 2.5, out, dev) == _lib.MOE_ERR_SIZE
    assert _noalloc(lib, gpu, 0, 0, 2.5, out, dev) == _lib.MOE_OK
    torch.cuda.synchronize()
    assert (out.view(torch.int16) == 0).all(), "rejected and empty calls write nothing"
    np.testing.assert_equal(int(lib.moe_fp8_forward_noalloc(None, *[0] * 7, 3, 0, 2.5, None, None)),
                            _lib.MOE_ERR_NULL)
