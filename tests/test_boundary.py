"""The C-ABI library and the Python entry points, without a GPU: the library
loads, exports every symbol the header declares, and rejects bad arguments on
the host before any GPU call; the Python layer validates like ref_moe.py."""
import ctypes
import os
import re

import pytest
import torch

import flashinfer_mlsys_amd as fm
from flashinfer_mlsys_amd import _lib

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "moe_fp8.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(moe_fp8_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmoe_mi355x.so is not built: run python -m flashinfer_mlsys_amd.build")
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 8
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must cover the header exactly"


def test_header_constants_match_binding():
    """Every plain numeric #define and enum value of the header equals the binding's constant."""
    text = open(HEADER).read()
    found = {}
    for name, shift, num in re.findall(r"#define\s+(MOE_\w+)\s+(?:\(1 << (\d+)\)|(\d+))\s*$", text, re.M):
        found[name] = 1 << int(shift) if shift else int(num)
    for name, val in re.findall(r"\b(MOE_(?:ERR|OK|SHAPE)\w*)\s*=\s*(-?\d+)", text):
        found[name] = int(val)
    assert {"MOE_FP8_DECODE_MAX_TOKENS", "MOE_FP8_NOALLOC_MAX_TOKENS", "MOE_FP8_CHUNK_TOKENS",
            "MOE_SHAPE_PREFILL", "MOE_ERR_NOALLOC_SIZE"} <= set(found)
    for name, val in found.items():
        assert getattr(_lib, name) == val, name
    assert _lib.MOE_FP8_NOALLOC_MAX_TOKENS <= _lib.MOE_FP8_DECODE_MAX_TOKENS


def test_abi_version_and_strings(lib):
    assert lib.moe_fp8_abi_version() == 3
    for code in (0, -1, -2, -3, -4, -5, -6, -7):
        assert lib.moe_fp8_strerror(code)
    assert lib.moe_fp8_strerror(-99) == b"unknown error"


def test_workspace_size(lib):
    assert lib.moe_fp8_workspace_size(-1) == 0
    assert lib.moe_fp8_workspace_size(_lib.MOE_FP8_MAX_TOKENS + 1) == 0
    # calls above the chunk size run chunk by chunk in one chunk's workspace
    chunk = lib.moe_fp8_workspace_size(_lib.MOE_FP8_CHUNK_TOKENS)
    assert chunk < 5e9
    for T in (_lib.MOE_FP8_CHUNK_TOKENS + 1, 20000, _lib.MOE_FP8_MAX_TOKENS):
        assert lib.moe_fp8_workspace_size(T) == chunk
    assert lib.moe_fp8_workspace_size(_lib.MOE_FP8_CHUNK_TOKENS - 1) < chunk
    assert lib.moe_fp8_workspace_size(0) > 0
    prev = 0
    for T in (1, 2, 16, 1024, 8192):
        n = lib.moe_fp8_workspace_size(T)
        assert n > prev
        # at least the per-pair fp16 C rows and fp16 pair rows
        assert n >= 8 * T * (2048 * 2 + 7168 * 2)
        assert n % 256 == 0
        prev = n


FAKE = 0x10000  # aligned, never dereferenced: every call below fails validation first


def _fwd(lib, T=1, ptrs=None, ws_bytes=1 << 40):
    p = ptrs or [FAKE] * 8
    return lib.moe_fp8_forward(*p, T, 0, 2.5, FAKE, FAKE, ws_bytes, None)


def test_forward_argument_errors(lib):
    assert _fwd(lib, T=-1) == _lib.MOE_ERR_SIZE
    assert _fwd(lib, T=_lib.MOE_FP8_MAX_TOKENS + 1) == _lib.MOE_ERR_SIZE
    # the forward runs long calls chunk by chunk: beyond the other entry points' limit is fine
    assert _fwd(lib, T=_lib.MOE_FP8_MAX_TAP_TOKENS + 1, ws_bytes=1) == _lib.MOE_ERR_WORKSPACE
    assert _fwd(lib, T=0) == _lib.MOE_OK
    ptrs = [FAKE] * 8
    ptrs[3] = None
    assert _fwd(lib, ptrs=ptrs) == _lib.MOE_ERR_NULL
    ptrs = [FAKE] * 8
    ptrs[4] = FAKE + 4
    assert _fwd(lib, ptrs=ptrs) == _lib.MOE_ERR_ALIGN
    # the prefill kernels need the whole moe_fp8_workspace_size(T)
    T = _lib.MOE_FP8_DECODE_MAX_TOKENS + 1
    assert _fwd(lib, T=T, ws_bytes=lib.moe_fp8_workspace_size(T) - 1) == _lib.MOE_ERR_WORKSPACE
    assert lib.moe_fp8_forward_shape(_lib.MOE_SHAPE_PREFILL, *[FAKE] * 8, 16, 0, 2.5, FAKE, FAKE,
                                     lib.moe_fp8_workspace_size(16) - 1, None) == _lib.MOE_ERR_WORKSPACE
    # the decode kernels (T <= MOE_FP8_DECODE_MAX_TOKENS) use no pair rows: less is enough, but not a
    # few bytes
    assert _fwd(lib, T=16, ws_bytes=4096) == _lib.MOE_ERR_WORKSPACE


def test_noalloc_argument_errors(lib):
    """Rejected on the host before any GPU call: beyond its 64-token limit, T < 0."""
    f = lib.moe_fp8_forward_noalloc
    assert f(*[FAKE] * 8, 65, 0, 2.5, FAKE, None) == _lib.MOE_ERR_NOALLOC_SIZE
    assert f(*[FAKE] * 8, _lib.MOE_FP8_MAX_TOKENS, 0, 2.5, FAKE, None) == _lib.MOE_ERR_NOALLOC_SIZE
    assert f(*[FAKE] * 8, -1, 0, 2.5, FAKE, None) == _lib.MOE_ERR_SIZE
    assert f(*[FAKE] * 8, 0, 0, 2.5, FAKE, None) == _lib.MOE_OK
    assert lib.moe_fp8_strerror(_lib.MOE_ERR_NOALLOC_SIZE).startswith(b"token count beyond")


def test_route_and_dispatch_argument_errors(lib):
    assert lib.moe_fp8_route(FAKE, FAKE, 0, 2.5, FAKE, FAKE, None, None) == _lib.MOE_OK
    assert lib.moe_fp8_route(None, FAKE, 4, 2.5, FAKE, FAKE, None, None) == _lib.MOE_ERR_NULL
    assert lib.moe_fp8_route(FAKE + 8, FAKE, 4, 2.5, FAKE, FAKE, None, None) == _lib.MOE_ERR_ALIGN
    assert lib.moe_fp8_route(FAKE, FAKE, -3, 2.5, FAKE, FAKE, None, None) == _lib.MOE_ERR_SIZE
    hw = _lib.MOE_FP8_HEADER_WORDS + 32
    assert lib.moe_fp8_dispatch(FAKE, FAKE, 4, 0, None, hw, FAKE, FAKE, FAKE, None) == _lib.MOE_ERR_NULL
    assert lib.moe_fp8_dispatch(FAKE, FAKE, 4, 0, FAKE + 4, hw, FAKE, FAKE, FAKE, None) == _lib.MOE_ERR_ALIGN
    assert lib.moe_fp8_route(FAKE, FAKE, _lib.MOE_FP8_MAX_TAP_TOKENS + 1, 2.5, FAKE, FAKE, None, None) == \
        _lib.MOE_ERR_SIZE


def test_dispatch_header_size_checked(lib):
    """The dispatch taps take the header's size: the header words, then 32 counts per
    group of 16 tokens; one word short is rejected before any GPU call."""
    for T in (1, 16, 17, 300, 4097):
        need = _lib.MOE_FP8_HEADER_WORDS + 32 * ((T + 15) // 16)
        assert lib.moe_fp8_dispatch(FAKE, FAKE, T, 0, FAKE, need - 1, FAKE, FAKE, FAKE, None) == \
            _lib.MOE_ERR_WORKSPACE
        for shape in (_lib.MOE_SHAPE_AUTO, _lib.MOE_SHAPE_PREFILL):
            assert lib.moe_fp8_route_dispatch(shape, FAKE, FAKE, T, 0, 2.5, FAKE, FAKE, FAKE, need - 1, FAKE, FAKE,
                                              FAKE, None) == _lib.MOE_ERR_WORKSPACE


def test_quantize_argument_errors(lib):
    q = lib.moe_fp8_quantize_activations
    assert q(FAKE, 0, FAKE, FAKE, None) == _lib.MOE_OK
    assert q(FAKE, -1, FAKE, FAKE, None) == _lib.MOE_ERR_SIZE
    assert q(FAKE, _lib.MOE_FP8_MAX_TAP_TOKENS + 1, FAKE, FAKE, None) == _lib.MOE_ERR_SIZE
    assert q(None, 4, FAKE, FAKE, None) == _lib.MOE_ERR_NULL
    assert q(FAKE, 4, FAKE, None, None) == _lib.MOE_ERR_NULL
    assert q(FAKE, 4, FAKE + 8, FAKE, None) == _lib.MOE_ERR_ALIGN


def test_router_argument_errors(lib):
    r = lib.moe_fp8_router_logits
    assert r(FAKE, FAKE, 0, None, None) == _lib.MOE_OK  # nothing to do, nothing read
    assert r(FAKE, FAKE, -1, FAKE, None) == _lib.MOE_ERR_SIZE
    assert r(FAKE, FAKE, _lib.MOE_FP8_MAX_TAP_TOKENS + 1, FAKE, None) == _lib.MOE_ERR_SIZE
    assert r(None, FAKE, 4, FAKE, None) == _lib.MOE_ERR_NULL
    assert r(FAKE, None, 4, FAKE, None) == _lib.MOE_ERR_NULL
    assert r(FAKE, FAKE, 4, None, None) == _lib.MOE_ERR_NULL
    assert r(FAKE, FAKE + 8, 4, FAKE, None) == _lib.MOE_ERR_ALIGN
    assert r(FAKE, FAKE, 4, FAKE + 4, None) == _lib.MOE_ERR_ALIGN


def test_router_quantize_argument_errors(lib):
    r = lib.moe_fp8_router_quantize
    assert r(FAKE, FAKE, 0, None, None, None, None) == _lib.MOE_OK  # nothing to do, nothing read
    assert r(FAKE, FAKE, -1, FAKE, FAKE, FAKE, None) == _lib.MOE_ERR_SIZE
    assert r(FAKE, FAKE, _lib.MOE_FP8_MAX_TAP_TOKENS + 1, FAKE, FAKE, FAKE, None) == _lib.MOE_ERR_SIZE
    for i in range(5):
        args = [FAKE] * 5
        args[i] = None
        assert r(args[0], args[1], 4, args[2], args[3], args[4], None) == _lib.MOE_ERR_NULL, i
        args[i] = FAKE + 4
        assert r(args[0], args[1], 4, args[2], args[3], args[4], None) == _lib.MOE_ERR_ALIGN, i


def test_shape_argument(lib):
    """The kernel shape is a per-call argument of the test and bench entry points
    (there is no process-global switch); out-of-range values are rejected first."""
    assert not hasattr(_lib.SIGNATURES, "moe_fp8_set_path") and "moe_fp8_set_path" not in _lib.SIGNATURES
    args = [FAKE] * 8 + [1, 0, 2.5, FAKE, FAKE, 1 << 40, None]
    for bad in (-1, 2, 7):
        assert lib.moe_fp8_forward_shape(bad, *args) == _lib.MOE_ERR_ARG
        assert lib.moe_fp8_run_stage(0, bad, *args) == _lib.MOE_ERR_ARG
        assert lib.moe_fp8_route_dispatch(bad, FAKE, FAKE, 4, 0, 2.5, FAKE, FAKE, FAKE, 1 << 20, *[FAKE] * 3,
                                          None) == _lib.MOE_ERR_ARG
    for stage in (-1, 4):
        assert lib.moe_fp8_run_stage(stage, 0, *args) == _lib.MOE_ERR_ARG
    for shape in (_lib.MOE_SHAPE_AUTO, _lib.MOE_SHAPE_PREFILL):  # valid shape: the usual checks follow
        assert lib.moe_fp8_forward_shape(shape, *[FAKE] * 8, -1, 0, 2.5, FAKE, FAKE, 1 << 40, None) == \
            _lib.MOE_ERR_SIZE
        assert lib.moe_fp8_forward_shape(shape, *[FAKE] * 8, 0, 0, 2.5, FAKE, FAKE, 1 << 40, None) == _lib.MOE_OK


def _cpu_inputs(T=2):
    return [
        torch.zeros((T, 256), dtype=torch.float32),
        torch.zeros(256, dtype=torch.bfloat16),
        torch.zeros((T, 7168), dtype=torch.float8_e4m3fn),
        torch.zeros((56, T), dtype=torch.float32),
        torch.zeros((32, 4096, 7168), dtype=torch.float8_e4m3fn),
        torch.zeros((32, 32, 56), dtype=torch.float32),
        torch.zeros((32, 7168, 2048), dtype=torch.float8_e4m3fn),
        torch.zeros((32, 56, 16), dtype=torch.float32),
    ]


def test_python_entry_rejects_cpu_tensors():
    args = _cpu_inputs()
    with pytest.raises(fm.MoEInputError, match="GPU"):
        fm.run(*args, 0, 2.5)
    with pytest.raises(AssertionError):  # same exception family as ref_moe.py's asserts
        fm.kernel(*args, 0, 2.5, torch.empty((2, 7168), dtype=torch.bfloat16))


def test_python_validation_messages(monkeypatch):
    """Shape and dtype checks run before any GPU work (device check stubbed out)."""
    monkeypatch.setattr(fm, "_on_gpu", lambda t, n: t)
    good = _cpu_inputs()
    assert fm._validate(*good) == 2
    bad = list(good)
    bad[0] = torch.zeros((2, 128), dtype=torch.float32)
    with pytest.raises(fm.MoEInputError, match="num_experts must be 256"):
        fm._validate(*bad)
    bad = list(good)
    bad[3] = torch.zeros((2, 56), dtype=torch.float32)
    with pytest.raises(fm.MoEInputError, match="hidden_states_scale"):
        fm._validate(*bad)
    bad = list(good)
    bad[1] = torch.zeros(256, dtype=torch.float32)
    with pytest.raises(fm.MoEInputError, match="bfloat16"):
        fm._validate(*bad)
    bad = list(good)
    bad[4] = torch.zeros((16, 4096, 7168), dtype=torch.float8_e4m3fn)
    with pytest.raises(fm.MoEInputError, match="num_local_experts must be 32"):
        fm._validate(*bad)


def test_no_oracle_in_product_path():
    """The shipped package never imports the oracle."""
    pkg = os.path.join(ROOT, "flashinfer_mlsys_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle\b", src, re.M), f
