"""Parity of the HIP operator with the reference (golden vectors) and the CPU oracle.

Bars: expert selection and the per-expert permutation bit-exact; the bf16 output
within atol=1e-2, rtol=2e-2 (torch.allclose semantics) of the reference.
Everything goes through libmoe_mi355x.so's C ABI via flashinfer_mlsys_amd.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

import flashinfer_mlsys_amd as fm
from flashinfer_mlsys_amd import workloads as wl
from oracle import cpu_ref, np_ref

from conftest import ATOL, RTOL, assert_close_bf16, bf16_bits_to_f32, golden_lists, load_golden, quant_edge_rows

pytestmark = pytest.mark.gpu

ALL = list(wl.WORKLOADS)
SMALL = [n for n in ALL if wl.WORKLOADS[n].T <= 1024]


def _say(msg):
    print(msg, flush=True)


class Case:
    def __init__(self, name, weights, dev):
        self.name = name
        self.w = wl.WORKLOADS[name]
        self.g = load_golden(name)
        acts = wl.workload_activations(self.w)
        for a, h in zip(acts, self.g["in_sha256"]):
            assert wl.fingerprint(a) == str(h), f"{name}: inputs do not regenerate identically"
        self.cpu = list(acts) + list(weights[0])
        self.gpu = [a.to(dev) for a in acts] + list(weights[1])
        self.offset = self.w.local_expert_offset
        self.rsf = self.w.routed_scaling_factor

    def forward(self, offset=None, shape=fm.SHAPE_AUTO):
        return fm.run_shape(shape, *self.gpu, self.offset if offset is None else offset, self.rsf)


_cases = {}


@pytest.fixture
def case(request, weights, dev):
    name = request.param
    if name not in _cases:
        _say(f"case {name}")
        _cases.clear()
        _cases[name] = Case(name, weights, dev)
    return _cases[name]


# logits whose float32 sigmoid is the same whether exp(-x) is correctly rounded
# (the kernel) or torch's (the oracle), so both sides see identical keys
TIE_LOGITS = np.array([-0.5, 0.0, 0.25, 0.5, 0.75, 1.0, 2.0, 3.0], dtype=np.float32)
TIE_BIAS = np.array([0.0, 0.25, 0.5], dtype=np.float32)


@pytest.mark.parametrize("T", [1, 8, 64, 300])
def test_route_ties_follow_torch_topk(dev, T):
    """Logits and bias from a few values, so equal keys meet at the group cut and
    at the 8th expert everywhere: the selection must be the oracle's
    (torch.topk(sorted=False), i.e. std::nth_element's order), bit for bit, and
    the tie-resolving brute-force search's."""
    lg_t = torch.from_numpy(TIE_LOGITS)
    s_torch = (1.0 / (1.0 + torch.exp(-lg_t))).numpy()
    one = np.float32(1.0)
    s_cr = one / (one + np.exp(-TIE_LOGITS.astype(np.float64)).astype(np.float32))
    if not (s_torch == s_cr).all():
        pytest.skip("this host's torch exp rounds a tie logit differently from the kernel's")
    rng = np.random.default_rng(4242 + T)
    lg = TIE_LOGITS[rng.integers(0, len(TIE_LOGITS), size=(T, 256))]
    b = TIE_BIAS[rng.integers(0, len(TIE_BIAS), size=256)]
    bias = torch.from_numpy(b).to(torch.bfloat16)
    ids, w, _ = fm.route(torch.from_numpy(lg).to(dev), bias.to(dev), 2.5)
    ref_idx, dense, _, _, _ = cpu_ref.route(torch.from_numpy(lg), bias, 2.5)
    ids = ids.cpu().numpy()
    np.testing.assert_array_equal(ids, cpu_ref.sorted_selection(ref_idx).numpy().astype(np.int32))
    bf_ids, _ = np_ref.brute_force_route(lg[:16], b, 2.5)
    np.testing.assert_array_equal(ids[:16], bf_ids.astype(np.int32))
    np.testing.assert_allclose(w.cpu().numpy(), torch.gather(dense, 1, torch.from_numpy(ids).long()).numpy(),
                               rtol=4e-7 * 8, atol=0)
    # every key equal: the reference keeps groups 4-7 and experts 168-175
    eq, _, _ = fm.route(torch.ones((T, 256), device=dev), torch.zeros(256, dtype=torch.bfloat16, device=dev), 2.5)
    assert (eq.cpu().numpy() == np.arange(168, 176, dtype=np.int32)).all()


def _near_tie_tokens(T, seed):
    """Token families that put the group and expert cuts anywhere from exact ties to
    far apart: N(0,1) logits; logits on a grid c + k*2^-e (e in 12..24, so sigmoid
    gaps of 0 to a few thousand fp32 ulps, around the fast path's certification
    bound); the tie set; huge magnitudes (exp overflows / underflows, s = 0 or 1)."""
    rng = np.random.default_rng(seed)
    lg = rng.standard_normal((T, 256)).astype(np.float32)
    fam = rng.integers(0, 4, size=T)
    for t in np.nonzero(fam == 1)[0]:
        e = int(rng.integers(12, 25))
        c = np.float32(rng.uniform(-1.5, 1.5))
        lg[t] = c + rng.integers(0, 64, size=256).astype(np.float32) * np.float32(2.0 ** -e)
    tie = fam == 2
    lg[tie] = TIE_LOGITS[rng.integers(0, len(TIE_LOGITS), size=(int(tie.sum()), 256))]
    big = fam == 3
    lg[big] = rng.choice(np.array([-200.0, -90.0, -30.0, 30.0, 90.0, 200.0], dtype=np.float32),
                         size=(int(big.sum()), 256)) + lg[big]
    return lg


TEST_SUPPORT_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "libmoe_test_support.so")


def test_fast_sigmoid_error_bound():
    """The routing fast path certifies its cuts assuming |fast_sigmoid(x) -
    exact_sigmoid(x)| <= 2^-20; the kernel here measures the largest difference over
    every finite fp32 x with the routing kernels' own device functions."""
    if not os.path.exists(TEST_SUPPORT_LIB):
        raise FileNotFoundError(f"{TEST_SUPPORT_LIB} is not built (build() compiles it)")
    lib = ctypes.CDLL(TEST_SUPPORT_LIB)
    lib.moe_test_fast_sigmoid_max_error.argtypes = [ctypes.POINTER(ctypes.c_double)]
    lib.moe_test_fast_sigmoid_max_error.restype = ctypes.c_int
    out = ctypes.c_double(-1.0)
    assert lib.moe_test_fast_sigmoid_max_error(ctypes.byref(out)) == 0
    _say(f"max |fast_sigmoid - exact_sigmoid| = {out.value:.3e} = {out.value / 2.0 ** -23:.2f} * 2^-23")
    assert 0.0 < out.value <= 2.0 ** -20


@pytest.mark.parametrize("T,bias_kind", [(6144, "normal"), (6144, "tie"), (9000, "normal")])
def test_route_fast_path_certification(dev, T, bias_kind):
    """From 6,144 tokens the routing kernel tries the fast scores first and keeps
    their selection only when both cuts clear the error bound; every other token
    takes the exact path. Either way the selection must be the oracle's bit for bit
    (exp correctly rounded, as the exact path) and the weights within a few ulps."""
    lg = _near_tie_tokens(T, 97 + T)
    rng = np.random.default_rng(T)
    if bias_kind == "tie":
        b = TIE_BIAS[rng.integers(0, len(TIE_BIAS), size=256)]
    else:
        b = (rng.standard_normal(256) * 0.1).astype(np.float32)
    bias = torch.from_numpy(b).to(torch.bfloat16)
    ids, w, _ = fm.route(torch.from_numpy(lg).to(dev), bias.to(dev), 2.5)
    ref_idx, dense, _, _, _ = cpu_ref.route(torch.from_numpy(lg), bias, 2.5, exp="correctly_rounded")
    ids = ids.cpu().numpy()
    np.testing.assert_array_equal(ids, cpu_ref.sorted_selection(ref_idx).numpy().astype(np.int32))
    np.testing.assert_allclose(w.cpu().numpy(), torch.gather(dense, 1, torch.from_numpy(ids).long()).numpy(),
                               rtol=4e-7 * 8, atol=0)


def test_route_weights_do_not_depend_on_the_path(dev):
    """A token's routing weights are the same bits whether the fast path (calls of
    6,144 tokens or more) or the exact path (smaller calls) routed it: both sum the 8
    selected scores, in ascending id order, by the same tree. The first 300 rows of a
    6,144-token call are routed again as a call of their own."""
    rng = np.random.default_rng(6144)
    lg = torch.from_numpy(rng.standard_normal((6144, 256), dtype=np.float32)).to(dev)
    bias = torch.from_numpy((rng.standard_normal(256) * 0.1).astype(np.float32)).to(torch.bfloat16).to(dev)
    ids_big, w_big, _ = fm.route(lg, bias, 2.5)
    ids_small, w_small, _ = fm.route(lg[:300].contiguous(), bias, 2.5)
    assert torch.equal(ids_big[:300], ids_small)
    assert torch.equal(w_big[:300].view(torch.int32), w_small.view(torch.int32))


@pytest.mark.parametrize("case", ALL, indirect=True)
def test_route_selection_bit_exact(case):
    ids, w, _ = fm.route(case.gpu[0], case.gpu[1], case.rsf)
    ids = ids.cpu().numpy()
    assert (np.diff(ids, axis=1) > 0).all(), "ids must be ascending and distinct per token"
    np.testing.assert_array_equal(ids, case.g["sel_ids"].astype(np.int32))
    # weights: the oracle's dense weights at the selected ids, to a few fp32 ulps (the
    # oracle's sigmoid rounded as the kernel's, so that this host's exp bits cannot move
    # a near-tie; the selection itself is pinned to the reference's above)
    _, dense, _, _, _ = cpu_ref.route(case.cpu[0], case.cpu[1], case.rsf, exp="correctly_rounded")
    ref_w = torch.gather(dense, 1, torch.from_numpy(ids).long()).numpy()
    np.testing.assert_allclose(w.cpu().numpy(), ref_w, rtol=4e-7 * 8, atol=0)


def _check_dispatch(case, ids, w, header, perm_tok, perm_w, pair):
    h = header.cpu().numpy()
    counts, seg = h[:32], h[32:65]
    np.testing.assert_array_equal(counts, case.g["counts"])
    assert seg[0] == 0 and (np.diff(seg) == counts).all()
    P = int(seg[32])
    np.testing.assert_array_equal(perm_tok.cpu().numpy()[:P], case.g["token_lists"])
    n_act = h[65]
    np.testing.assert_array_equal(h[66:66 + n_act], np.nonzero(counts)[0])
    # perm_w is the routing weight of each pair; tok_pair points back at it
    ids_c, w_c, pair_c = ids.cpu().numpy(), w.cpu().numpy(), pair.cpu().numpy()
    np.testing.assert_array_equal(ids_c, case.g["sel_ids"].astype(np.int32))
    pt, pw = perm_tok.cpu().numpy()[:P], perm_w.cpu().numpy()[:P]
    local = (ids_c >= case.offset) & (ids_c < case.offset + 32)
    assert ((pair_c >= 0) == local).all()
    assert (pair_c[~local] == -1).all()
    t_idx, j_idx = np.nonzero(local)
    p_idx = pair_c[t_idx, j_idx]
    assert sorted(p_idx.tolist()) == list(range(P))
    np.testing.assert_array_equal(pt[p_idx], t_idx)
    np.testing.assert_array_equal(pw[p_idx], w_c[t_idx, j_idx])


@pytest.mark.parametrize("case", ALL, indirect=True)
def test_dispatch_bit_exact(case):
    """The two separate stage kernels (route_kernel, dispatch_kernel)."""
    ids, w, pair = fm.route(case.gpu[0], case.gpu[1], case.rsf)
    header, perm_tok, perm_w, pair = fm.dispatch(ids, w, pair, case.offset)
    _check_dispatch(case, ids, w, header, perm_tok, perm_w, pair)


def _synthetic_ids(T, offset, seed):
    """8 distinct ascending ids per token ((a + k s) mod 256 with s odd), plus
    tokens with all 8 ids local and tokens with none."""
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, T)
    s = 2 * rng.integers(0, 128, T) + 1
    ids = np.sort((a[:, None] + np.arange(8)[None, :] * s[:, None]) % 256, axis=1).astype(np.int32)
    ids[::97] = offset + np.arange(8, dtype=np.int32) * 3          # all 8 local
    far = (offset + 128) % 256
    ids[5::89] = np.sort((far + np.arange(8, dtype=np.int32)) % 256)  # none local (the window is 32 wide)
    w = rng.random((T, 8), dtype=np.float32)
    return ids, w


@pytest.mark.parametrize("T,offset", [(20000, 64), (131072, 0), (777, 200)])
def test_dispatch_large_synthetic(dev, T, offset):
    """Dispatch bit-exact at sizes past the benchmark's: many 256-token chunks
    (T=20000), the largest token count the library accepts (T=131072: 512
    chunks) and a ragged last chunk (T=777), against a numpy restatement of
    ref_moe.py:131-145."""
    _say(f"dispatch synthetic T={T} offset={offset}")
    ids, w = _synthetic_ids(T, offset, seed=T)
    ids_d = torch.from_numpy(ids).to(dev)
    w_d = torch.from_numpy(w).to(dev)
    pair = torch.full((T, 8), -1, dtype=torch.int32, device=dev)
    header, perm_tok, perm_w, pair = fm.dispatch(ids_d, w_d, pair, offset)
    torch.cuda.synchronize()
    h = header.cpu().numpy()
    lists = [np.nonzero((ids == offset + e).any(axis=1))[0] for e in range(32)]
    counts = np.array([len(x) for x in lists])
    np.testing.assert_array_equal(h[:32], counts)
    P = int(counts.sum())
    assert h[32] == 0 and h[64] == P
    np.testing.assert_array_equal(perm_tok.cpu().numpy()[:P], np.concatenate(lists))
    pair_c, pw = pair.cpu().numpy(), perm_w.cpu().numpy()[:P]
    local = (ids >= offset) & (ids < offset + 32)
    assert ((pair_c >= 0) == local).all()
    t_idx, j_idx = np.nonzero(local)
    p_idx = pair_c[t_idx, j_idx]
    np.testing.assert_array_equal(perm_tok.cpu().numpy()[p_idx], t_idx)
    np.testing.assert_array_equal(pw[p_idx], w[t_idx, j_idx])


@pytest.mark.parametrize("case", ALL, indirect=True)
def test_route_dispatch_as_forward_runs_it(case):
    """Routing + dispatch exactly as the forward runs them (for T <= 96 the routing kernel and the
    decode GEMM1's in-workgroup dispatch)."""
    ids, w, header, perm_tok, perm_w, pair = fm.route_dispatch(case.gpu[0], case.gpu[1], case.offset, case.rsf)
    _check_dispatch(case, ids, w, header, perm_tok, perm_w, pair)
    ids2, w2, _ = fm.route(case.gpu[0], case.gpu[1], case.rsf)
    assert torch.equal(ids, ids2) and torch.equal(w, w2)


@pytest.mark.parametrize("case", ALL, indirect=True)
def test_forward_matches_reference(case):
    out = case.forward()
    torch.cuda.synchronize()
    out_np = out.view(torch.int16).cpu().numpy().view(np.uint16)
    rows = case.g["out_rows"]
    assert_close_bf16(bf16_bits_to_f32(out_np[rows]), bf16_bits_to_f32(case.g["out_bf16"]),
                      f"{case.name} vs reference rows")
    # the whole output against the oracle (its sigmoid rounded as the kernel's: the same
    # selection as the reference's, checked above, on any host)
    ref = cpu_ref.run(*case.cpu, case.offset, case.rsf, exp="correctly_rounded").float().numpy()
    got = bf16_bits_to_f32(out_np).astype(np.float64)
    ratio = np.abs(got - ref) / (ATOL + RTOL * np.abs(ref))
    _say(f"{case.name}: worst |err| / (atol + rtol |ref|) over the whole output {ratio.max():.4f}, "
         f"max |err| {np.abs(got - ref).max():.4g}")
    assert_close_bf16(got, ref, f"{case.name} vs oracle")
    # tokens without a local expert are exact zeros
    lists = golden_lists(case.g)
    has = np.zeros(case.w.T, dtype=bool)
    for l in lists:
        has[l] = True
    assert (out_np[~has] == 0).all()


@pytest.mark.parametrize("case", ["decode_t1", "decode_t8", "t16", "decode_t64"], indirect=True)
def test_decode_and_prefill_shapes_agree(case):
    """T <= 96 runs the decode kernels by default; SHAPE_PREFILL forces the prefill kernels."""
    a = case.forward().float()
    b = case.forward(shape=fm.SHAPE_PREFILL).float()
    ref = bf16_bits_to_f32(case.g["out_bf16"])
    rows = case.g["out_rows"]
    assert_close_bf16(a.cpu().numpy()[rows], ref, "decode shape")
    assert_close_bf16(b.cpu().numpy()[rows], ref, "prefill shape")
    # both shapes compute the same sums in different order: they agree far inside the bar
    d = (a - b).abs().max().item()
    assert d <= 2e-2, d


@pytest.mark.parametrize("case", ["decode_t8", "prefill_t1024", "skew_t4096"], indirect=True)
def test_deterministic(case):
    a = case.forward()
    b = case.forward()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("case", ["decode_t64", "prefill_t8192"], indirect=True)
def test_token_permutation_equivariance(case):
    """Each token's output depends only on its own row: permuting tokens permutes rows, bit for bit."""
    T = case.w.T
    perm = torch.from_numpy(np.random.default_rng(5).permutation(T)).to(case.gpu[0].device)
    lg, b, h, hs = case.gpu[:4]
    out = case.forward()
    out_p = fm.run(lg[perm].contiguous(), b, h[perm].contiguous(), hs[:, perm].contiguous(), *case.gpu[4:],
                   case.offset, case.rsf)
    assert torch.equal(out_p.view(torch.int16), out[perm].view(torch.int16))


@pytest.mark.parametrize("case", ["t16"], indirect=True)
@pytest.mark.parametrize("offset", [256, -32, 1000, -1000])
def test_no_local_expert_gives_zeros(case, offset):
    out = case.forward(offset)
    assert (out.view(torch.int16) == 0).all()


@pytest.mark.parametrize("case", ["t16", "prefill_t1024"], indirect=True)
@pytest.mark.parametrize("offset", [256, -1000])
def test_no_local_expert_gives_zeros_prefill_kernels(case, offset):
    """No pair for the local experts through the prefill kernels (zero row tiles:
    every GEMM workgroup has no item), whatever T: exact zeros."""
    out = case.forward(offset, shape=fm.SHAPE_PREFILL)
    torch.cuda.synchronize()
    assert (out.view(torch.int16) == 0).all()


@pytest.mark.parametrize("case", ["t16"], indirect=True)
@pytest.mark.parametrize("offset", [224, 240, -16, 32])
def test_other_offsets_match_oracle(case, offset):
    """Offsets whose 32-expert window is partly outside [0, 256) skip those experts (ref_moe.py:134-137)."""
    out = case.forward(offset).float().cpu().numpy()
    ref = cpu_ref.run(*case.cpu, offset, case.rsf).float().numpy()
    assert_close_bf16(out, ref, f"offset {offset}")


def test_chunked_forward_equals_separate_calls(weights, dev):
    """A call above MOE_FP8_CHUNK_TOKENS runs chunk by chunk in one chunk's
    workspace: its output equals, bit for bit, separate calls over the token chunks
    (each with its own columns of hidden_states_scale, which the chunked call reads
    with the whole call's row stride), and rows on both sides of the chunk edge
    match the oracle run on those tokens alone."""
    from flashinfer_mlsys_amd import _lib
    C = _lib.MOE_FP8_CHUNK_TOKENS
    T = C + 1000
    lg, b, hs, hss = wl.make_activations(T, 4242)
    offset, rsf = 64, 2.5
    _say(f"chunked forward T={T}")
    g = [t.to(dev) for t in (lg, b, hs, hss)]
    out = fm.run(*g, *weights[1], offset, rsf)
    parts = []
    for a, e in ((0, C), (C, T)):
        parts.append(fm.run(g[0][a:e].contiguous(), g[1], g[2][a:e].contiguous(), g[3][:, a:e].contiguous(),
                            *weights[1], offset, rsf))
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), torch.cat(parts).view(torch.int16))
    rows = torch.tensor([0, 1, C - 2, C - 1, C, C + 1, T - 2, T - 1])
    ref = cpu_ref.run(lg[rows], b, hs[rows], hss[:, rows].contiguous(), *weights[0], offset, rsf).float().numpy()
    assert_close_bf16(out.float().cpu().numpy()[rows.numpy()], ref, "rows at the chunk edge")


def test_zero_tokens(weights, dev):
    w13, s13, w2, s2 = weights[1]
    lg = torch.empty((0, 256), dtype=torch.float32, device=dev)
    b = torch.zeros(256, dtype=torch.bfloat16, device=dev)
    h = torch.empty((0, 7168), dtype=torch.float8_e4m3fn, device=dev)
    hs = torch.empty((56, 0), dtype=torch.float32, device=dev)
    out = fm.run(lg, b, h, hs, w13, s13, w2, s2, 0, 2.5)
    assert out.shape == (0, 7168)


# (T, local_expert_offset, seed, routed_scaling_factor): token counts between the
# benchmark's (3 and 9 around the in-GEMM1 routing limit of 8; 65 in the decode
# kernels' second half of 64 tokens, 96 their limit, 97 and 100 prefill counts;
# 257 a partial row tile, 513 one past a dispatch chunk of 512), other offsets and
# a scaling factor of 1. Each seed is the first from 7000 + T whose selection
# margins are at least 8 fp32 ulps and that routes a local pair.
ODD_CASES = [(3, 0, 7003, 2.5), (9, 96, 7009, 2.5), (65, 224, 7065, 2.5), (96, 64, 7096, 2.5),
             (97, 128, 7097, 2.5), (100, 32, 7100, 1.0), (257, 0, 7257, 2.5), (513, 160, 7513, 2.5)]


# Rows per local expert at the prefill kernels' edges: 16-row fragments (GEMM1),
# 32-row blocks (GEMM2), 128-row tiles, and an empty expert among full ones.
EDGE_COUNTS = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 95, 96, 97, 127, 128, 129, 0, 255, 256, 257]


def _routing_for_counts(counts, offset, seed):
    """Logits that send exactly counts[e] tokens to local expert offset + e: each
    token's top-8 is its one local expert plus 3 + 2 + 2 experts of three other
    groups (every chosen logit in [6, 7), every other -8), in shuffled token order."""
    rng = np.random.default_rng(seed)
    assign = np.repeat(np.arange(len(counts)), counts)
    rng.shuffle(assign)
    T = len(assign)
    logits = np.full((T, 256), -8.0, dtype=np.float32)
    others = [g for g in range(8) if g != offset // 32]
    for t in range(T):
        logits[t, offset + assign[t]] = 6.0 + rng.random()
        for g, n in zip(rng.choice(others, 3, replace=False), (3, 2, 2)):
            logits[t, g * 32 + rng.choice(32, n, replace=False)] = 6.0 + rng.random(n)
    return torch.from_numpy(logits), torch.zeros(256, dtype=torch.bfloat16)


@pytest.mark.parametrize("offset", [0, 96])
def test_expert_row_counts_at_tile_edges_match_oracle(weights, dev, offset):
    """Experts with 1, 15, 16, 17, ..., 127, 128, 129, 255, 256, 257 rows: the
    prefill GEMMs skip row groups past each tile's valid rows, so every fragment,
    block and tile boundary is exercised; the dispatch counts are exactly those,
    and the output is within the bar of the CPU oracle."""
    lg, b = _routing_for_counts(EDGE_COUNTS, offset, 4242 + offset)
    T = lg.shape[0]
    _say(f"edge counts T={T} offset={offset}")
    g, e = cpu_ref.selection_margins(lg, b)
    assert min(g, e) >= 8
    hs, hss = wl.quantize_1x128(wl.hidden_bf16(T, 4343 + offset).to(torch.float32))
    gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
    ids, w, pair = fm.route(gpu[0], gpu[1], 2.5)
    header = fm.dispatch(ids, w, pair, offset)[0].cpu().numpy()
    want = np.zeros(32, dtype=np.int64)
    want[:len(EDGE_COUNTS)] = EDGE_COUNTS
    np.testing.assert_array_equal(header[:32], want)
    out = fm.run(*gpu, offset, 2.5).float().cpu().numpy()
    ref = cpu_ref.run(lg, b, hs, hss, *weights[0], offset, 2.5).float().numpy()
    assert_close_bf16(out, ref, f"edge counts offset={offset}")


@pytest.mark.parametrize("counts", [[64, 33, 64, 1, 0, 17], [65, 64, 2]], ids=["max64", "max65"])
def test_gemm2_item_heights_match_oracle(weights, dev, counts):
    """The prefill GEMM2 takes 64-row items when no expert has more than 64 rows
    (experts of exactly 64 rows fill one item) and 128-row items otherwise (an
    expert of 65 rows): both match the CPU oracle."""
    offset = 64
    lg, b = _routing_for_counts(counts, offset, 6161 + sum(counts))
    T = lg.shape[0]
    _say(f"GEMM2 item heights T={T} {counts}")
    hs, hss = wl.quantize_1x128(wl.hidden_bf16(T, 6262 + T).to(torch.float32))
    gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
    out = fm.run_shape(fm.SHAPE_PREFILL, *gpu, offset, 2.5).float().cpu().numpy()
    ref = cpu_ref.run(lg, b, hs, hss, *weights[0], offset, 2.5).float().numpy()
    assert_close_bf16(out, ref, f"counts={counts}")


DECODE_EDGE_COUNTS = [[64], [33, 31], [17, 16, 15, 1, 0, 15], [1] * 32, [0] * 31 + [48], [2, 3, 4, 5, 6, 7, 8, 9],
                      [96], [65, 31], [3] * 32, [0] * 31 + [90], [30, 0, 31, 35]]


@pytest.mark.parametrize("counts", DECODE_EDGE_COUNTS,
                         ids=["64", "33-31", "17-16-15-1-0-15", "1x32", "last48", "2-to-9", "96", "65-31", "3x32",
                              "last90", "30-0-31-35"])
@pytest.mark.parametrize("path", [fm.SHAPE_AUTO, fm.SHAPE_PREFILL], ids=["auto", "prefill"])
def test_decode_row_counts_at_pass_edges_match_oracle(weights, dev, counts, path):
    """At most 96 tokens with the local rows packed on few experts (a 64-row or
    96-row expert, 16 / 17 / 31 / 33 rows, every expert with one or three rows,
    only the last expert, 2 to 9 rows: the decode GEMM2's activation loads in
    one, two or three steps; experts whose tokens fall in both halves of 64
    tokens): the decode kernels' 16-row passes and the prefill kernels (forced)
    both match the CPU oracle."""
    offset = 32
    lg, b = _routing_for_counts(counts, offset, 5151 + len(counts))
    T = lg.shape[0]
    _say(f"decode edge counts T={T} {counts} path={path}")
    hs, hss = wl.quantize_1x128(wl.hidden_bf16(T, 5252 + T).to(torch.float32))
    gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
    out = fm.run_shape(path, *gpu, offset, 2.5).float().cpu().numpy()
    ref = cpu_ref.run(lg, b, hs, hss, *weights[0], offset, 2.5).float().numpy()
    assert_close_bf16(out, ref, f"counts={counts} path={path}")


@pytest.mark.parametrize("T,offset,seed,rsf", ODD_CASES)
def test_odd_token_counts_match_oracle(weights, dev, T, offset, seed, rsf):
    """Selection bit-exact, the dispatch of both kernel shapes identical (the decode
    shape's in-workgroup dispatch against the prefill shape's count and scatter
    kernels), and the whole output within the bar of the CPU oracle."""
    _say(f"odd T={T} offset={offset} seed={seed} rsf={rsf}")
    lg, b, hs, hss = wl.make_activations(T, seed, offset)
    g, e = cpu_ref.selection_margins(lg, b)
    assert min(g, e) >= 8, "the seed must keep the selection away from fp32 near-ties"
    gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
    ids, _, _ = fm.route(gpu[0], gpu[1], rsf)
    ref_ids = cpu_ref.sorted_selection(cpu_ref.route(lg, b, rsf)[0])
    assert torch.equal(ids.cpu().long(), ref_ids)
    da = fm.route_dispatch(gpu[0], gpu[1], offset, rsf, shape=fm.SHAPE_AUTO)
    dp = fm.route_dispatch(gpu[0], gpu[1], offset, rsf, shape=fm.SHAPE_PREFILL)
    P = int(da[2][:32].sum().item())
    for k, (x, y) in enumerate(zip(da, dp)):
        if k == 2:  # header: counts, segment starts, active count and list (the chunk counts differ)
            x, y = x[:fm._lib.MOE_FP8_HEADER_WORDS], y[:fm._lib.MOE_FP8_HEADER_WORDS]
        elif k in (3, 4):  # perm_tok, perm_w: the P pairs
            x, y = x[:P], y[:P]
        assert torch.equal(x.view(torch.int32), y.view(torch.int32)), k
    out = fm.run(*gpu, offset, rsf).float().cpu().numpy()
    ref = cpu_ref.run(lg, b, hs, hss, *weights[0], offset, rsf).float().numpy()
    assert_close_bf16(out, ref, f"T={T} offset={offset}")


@pytest.mark.parametrize("case", ["t16"], indirect=True)
def test_dps_writes_into_output(case):
    out = torch.full((case.w.T, 7168), 7.0, dtype=torch.bfloat16, device=case.gpu[0].device)
    ret = fm.kernel(*case.gpu, case.offset, case.rsf, out)
    assert ret is None
    ref = bf16_bits_to_f32(case.g["out_bf16"])
    assert_close_bf16(out.float().cpu().numpy()[case.g["out_rows"]], ref, "dps")


@pytest.mark.parametrize("case", ["decode_t1", "decode_t8", "t16", "decode_t32", "prefill_t1024"], indirect=True)
def test_graph_replay_matches_eager(case):
    """The forward captured in a HIP graph: every replay, with eager work and
    synchronisations between replays, gives the eager output bit for bit."""
    out = torch.empty((case.w.T, 7168), dtype=torch.bfloat16, device=case.gpu[0].device)
    ws = torch.empty(fm.workspace_size(case.w.T), dtype=torch.uint8, device=out.device)
    fm.kernel(*case.gpu, case.offset, case.rsf, out, workspace=ws)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fm.kernel(*case.gpu, case.offset, case.rsf, out, workspace=ws)
    for i in range(3):
        out.fill_(3.0)
        other = case.forward()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {i}"
        assert torch.equal(other.view(torch.int16), eager.view(torch.int16))


@pytest.mark.parametrize("T,offset,seed", [(80, 96, 8080), (96, 0, 8096)])
def test_graph_replay_matches_eager_second_half(weights, dev, T, offset, seed):
    """The decode kernels built for 128 tokens (calls of 65 to 96 tokens) captured in
    a HIP graph: every replay, with eager work between replays, gives the eager
    output bit for bit, and the eager output is the oracle's within the bar."""
    lg, b, hs, hss = wl.make_activations(T, seed, offset)
    gpu = [t.to(dev) for t in (lg, b, hs, hss)] + list(weights[1])
    out = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(fm.workspace_size(T), dtype=torch.uint8, device=dev)
    fm.kernel(*gpu, offset, 2.5, out, workspace=ws)
    torch.cuda.synchronize()
    eager = out.clone()
    ref = cpu_ref.run(lg, b, hs, hss, *weights[0], offset, 2.5).float().numpy()
    assert_close_bf16(eager.float().cpu().numpy(), ref, f"T={T} eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fm.kernel(*gpu, offset, 2.5, out, workspace=ws)
    for i in range(3):
        out.fill_(3.0)
        other = fm.run(*gpu, offset, 2.5)  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {i}"
        assert torch.equal(other.view(torch.int16), eager.view(torch.int16))


@pytest.mark.parametrize("case", ["prefill_t1024", "skew_t4096"], indirect=True)
def test_prefill_stages_rerun_alone(case):
    """The GEMM stages launched again on their own (no routing or dispatch in
    between, as a per-stage replay or a profiler does), GEMM2 twice in a row,
    recompute the same output, bit for bit, every time: the kernels keep no
    state in the workspace between launches beyond the dispatch they read."""
    from flashinfer_mlsys_amd import _lib
    lib = _lib.load()
    dev = case.gpu[0].device
    out = torch.empty((case.w.T, 7168), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(fm.workspace_size(case.w.T), dtype=torch.uint8, device=dev)
    fm.kernel(*case.gpu, case.offset, case.rsf, out, workspace=ws)
    torch.cuda.synchronize()
    ref = out.clone()
    args = ([t.data_ptr() for t in case.gpu] + [case.w.T, case.offset, case.rsf, out.data_ptr(), ws.data_ptr(),
                                                 ws.numel(), torch.cuda.current_stream(dev).cuda_stream])
    for rep in range(3):
        out.fill_(3.0)
        for stage in (1, 2, 2, 3):
            _lib.check(lib.moe_fp8_run_stage(stage, fm.SHAPE_AUTO, *args), "moe_fp8_run_stage")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"rerun {rep}"


@pytest.mark.parametrize("case", ["t16", "prefill_t1024", "skew_t4096"], indirect=True)
def test_stale_workspace_is_never_read_as_data(case):
    """The workspace arrives filled with 0xFF bytes (every stale token index reads
    -1): the prefill kernels' partial row tiles read token entries past an expert's
    segment and must replace them with a valid row, never load through them. The
    output equals the one from a zeroed workspace, bit for bit."""
    out = []
    for fill in (0x00, 0xFF):
        ws = torch.full((fm.workspace_size(case.w.T),), fill, dtype=torch.uint8, device=case.gpu[0].device)
        o = torch.empty((case.w.T, 7168), dtype=torch.bfloat16, device=ws.device)
        # the prefill kernels, whatever T
        fm._forward(fm.SHAPE_PREFILL, *case.gpu, case.offset, case.rsf, o, ws)
        torch.cuda.synchronize()
        out.append(o)
    assert torch.equal(out[0].view(torch.int16), out[1].view(torch.int16))


def test_concurrent_streams_own_workspaces(weights, dev):
    """Two callers on two streams (default priority), each with its own
    workspace, interleaved: each output equals its single-stream eager output
    bit for bit (the ABI is reentrant per workspace)."""
    names = ["decode_t8", "prefill_t1024"]
    ins, eager, outs, wss = [], [], [], []
    for n in names:
        w = wl.WORKLOADS[n]
        acts = [a.to(dev) for a in wl.workload_activations(w)]
        ins.append((acts, w))
        e = fm.run(*acts, *weights[1], w.local_expert_offset, w.routed_scaling_factor)
        torch.cuda.synchronize()
        eager.append(e)
        outs.append(torch.empty_like(e))
        wss.append(torch.empty(fm.workspace_size(w.T), dtype=torch.uint8, device=dev))
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream(dev))
    for _ in range(3):
        for k in (0, 1):
            acts, w = ins[k]
            with torch.cuda.stream(streams[k]):
                fm.kernel(*acts, *weights[1], w.local_expert_offset, w.routed_scaling_factor, outs[k],
                          workspace=wss[k])
    torch.cuda.synchronize()
    for k in (0, 1):
        assert torch.equal(outs[k].view(torch.int16), eager[k].view(torch.int16)), names[k]


# --- producer-side activation quantiser ---------------------------------------

@pytest.mark.parametrize("name", ["decode_t1", "t16", "decode_t64", "prefill_t1024", "prefill_t8192", "skew_t4096"])
def test_quantize_activations_reproduces_reference_inputs(dev, name):
    """The HIP quantiser turns a workload's bf16 hidden states into exactly the
    e4m3 hidden_states / scales the reference was run on (sha256 in the fixture)."""
    w = wl.WORKLOADS[name]
    g = load_golden(name)
    _say(f"quantize {name} T={w.T}")
    q, s = fm.quantize_activations(wl.hidden_bf16(w.T, w.seed).to(dev))
    torch.cuda.synchronize()
    assert wl.fingerprint(q) == str(g["in_sha256"][2])
    assert wl.fingerprint(s) == str(g["in_sha256"][3])


def test_quantize_activations_edge_cases(dev):
    """Bit-exact with the oracle on closed-form blocks (power-of-two scales with
    every e4m3 value and every tie, zeros, -0.0, bf16 subnormals, the largest
    bf16 values) and on a token count that is not a multiple of 16."""
    gen = torch.Generator().manual_seed(9)
    rnd = (torch.randn(37, 7168, generator=gen) * torch.logspace(-8, 8, 37).unsqueeze(1)).to(torch.bfloat16)
    for x in (quant_edge_rows(), rnd):
        q, s = fm.quantize_activations(x.to(dev))
        torch.cuda.synchronize()
        rq, rs = cpu_ref.quantize_activations(x)
        np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), rq.view(torch.uint8).numpy())
        np.testing.assert_array_equal(s.cpu().numpy(), rs.numpy())


def test_quantize_activations_graph_replay(dev):
    """The quantiser captured in a HIP graph: each replay, with eager work in
    between, reproduces the eager result."""
    x = wl.hidden_bf16(37, 4).to(dev)
    q = torch.empty((37, 7168), dtype=torch.float8_e4m3fn, device=dev)
    s = torch.empty((56, 37), dtype=torch.float32, device=dev)
    fm.quantize_activations(x, out=(q, s))
    torch.cuda.synchronize()
    q0, s0 = q.clone(), s.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fm.quantize_activations(x, out=(q, s))
    for i in range(3):
        q.view(torch.uint8).fill_(0x55)
        s.fill_(-1.0)
        fm.quantize_activations(wl.hidden_bf16(16, 5).to(dev))  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(q.view(torch.uint8), q0.view(torch.uint8)) and torch.equal(s, s0), f"replay {i}"

