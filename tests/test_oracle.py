"""Pins the CPU oracle (no GPU): against the reference's own golden vectors,
the OCP e4m3 spec, a brute-force routing search and a float64 recomputation;
planted mistakes in the oracle must be caught by those same checks."""
import json
import os

import numpy as np
import pytest
import torch

from flashinfer_mlsys_amd import workloads as wl
from oracle import cpu_ref, np_ref

from conftest import GOLDEN_DIR, assert_close_bf16, bf16_bits_to_f32, golden_lists, load_golden, quant_edge_rows

ALL = list(wl.WORKLOADS)


def test_e4m3_decode_matches_spec():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy().astype(np.float64)
    want = np_ref.e4m3_table()
    nan = np.isnan(want)
    assert nan.sum() == 2 and np.isnan(got[nan]).all()
    np.testing.assert_array_equal(got[~nan], want[~nan])
    # spot values from the OCP table: max normal, min normal, min subnormal
    assert np_ref.e4m3_value(0x7E) == 448.0
    assert np_ref.e4m3_value(0x08) == 2.0 ** -6
    assert np_ref.e4m3_value(0x01) == 2.0 ** -9


@pytest.mark.parametrize("name", ALL)
def test_inputs_regenerate(name):
    w = wl.WORKLOADS[name]
    g = load_golden(name)
    acts = wl.workload_activations(w)
    assert [wl.fingerprint(a) for a in acts] == [str(h) for h in g["in_sha256"]]


def test_weights_regenerate():
    with open(os.path.join(GOLDEN_DIR, "weights.json")) as f:
        meta = json.load(f)
    ts = wl.make_weights()
    for t, k in zip(ts, ["gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale"]):
        assert wl.fingerprint(t) == meta[k], k


@pytest.mark.parametrize("name", ALL)
def test_oracle_routing_matches_reference(name):
    w = wl.WORKLOADS[name]
    g = load_golden(name)
    lg, b, _, _ = wl.workload_activations(w)
    topk_idx = cpu_ref.route(lg, b, w.routed_scaling_factor)[0]
    np.testing.assert_array_equal(cpu_ref.sorted_selection(topk_idx).numpy(), g["sel_ids"].astype(np.int64))
    lists = cpu_ref.dispatch(topk_idx, w.local_expert_offset)
    np.testing.assert_array_equal([len(l) for l in lists], g["counts"])
    for a, b_ in zip(lists, golden_lists(g)):
        np.testing.assert_array_equal(a.numpy(), b_)


@pytest.mark.parametrize("name", ALL)
def test_oracle_correctly_rounded_exp_routing(name):
    """exp="correctly_rounded" (exp(-x) in float64, rounded once: the kernel's rule)
    keeps every reference selection of the workloads, and its sigmoid equals an
    independent numpy evaluation bit for bit."""
    w = wl.WORKLOADS[name]
    g = load_golden(name)
    lg, b, _, _ = wl.workload_activations(w)
    topk_idx, _, s, _, _ = cpu_ref.route(lg, b, w.routed_scaling_factor, exp="correctly_rounded")
    np.testing.assert_array_equal(cpu_ref.sorted_selection(topk_idx).numpy(), g["sel_ids"].astype(np.int64))
    one = np.float32(1.0)
    x = lg[:64].numpy()
    s_np = one / (one + np.exp(-x.astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(s[:64].numpy(), s_np)


@pytest.mark.parametrize("name", ["t16", "skew_t4096", "prefill_t1024"])
def test_routing_brute_force(name):
    """Exhaustive group-subset search (70 subsets) + full sort on the first 24 tokens."""
    w = wl.WORKLOADS[name]
    lg, b, _, _ = wl.workload_activations(w)
    lg = lg[:24]
    ids, wts = np_ref.brute_force_route(lg.numpy(), b.float().numpy(), w.routed_scaling_factor)
    topk_idx, dense, _, _, _ = cpu_ref.route(lg, b, w.routed_scaling_factor)
    sel = cpu_ref.sorted_selection(topk_idx).numpy()
    np.testing.assert_array_equal(sel, ids)
    np.testing.assert_allclose(np.take_along_axis(dense.numpy(), sel, 1), wts, rtol=1e-6)
    # weights sum to rsf * S / (S + 1e-20) = rsf
    np.testing.assert_allclose(dense.sum(1).numpy(), w.routed_scaling_factor, rtol=1e-6)


def test_routing_invariants_t8192():
    w = wl.WORKLOADS["prefill_t8192"]
    lg, b, _, _ = wl.workload_activations(w)
    topk_idx, dense, s, sb, gs = cpu_ref.route(lg, b, w.routed_scaling_factor)
    sel = cpu_ref.sorted_selection(topk_idx)
    assert (sel[:, 1:] > sel[:, :-1]).all()
    groups = sel // 32
    top4 = torch.topk(gs, 4, dim=1).indices
    kept = torch.zeros_like(gs, dtype=torch.bool).scatter_(1, top4, True)
    assert torch.gather(kept, 1, groups).all(), "every selected expert lies in a kept group"
    # the selected set is the top-8 of the biased scores among the kept groups
    cand = sb.masked_fill(~kept.repeat_interleave(32, 1), float("-inf"))
    kth = torch.sort(cand, 1, descending=True).values[:, 7:8]
    assert (torch.gather(sb, 1, sel) >= kth).all()
    # unbiased weights: proportional to s over the selected set
    ws = torch.gather(dense, 1, sel)
    ratio = ws / torch.gather(s, 1, sel)
    assert torch.allclose(ratio, ratio[:, :1].expand_as(ratio), rtol=1e-6)


@pytest.mark.parametrize("name", ["t16", "decode_t1", "decode_t2", "decode_t8", "decode_t64"])
def test_oracle_output_matches_reference(name):
    w = wl.WORKLOADS[name]
    g = load_golden(name)
    args = wl.make_inputs(name)
    out = cpu_ref.run(*args)
    got = out.view(torch.int16).numpy().view(np.uint16)[g["out_rows"]]
    assert_close_bf16(bf16_bits_to_f32(got), bf16_bits_to_f32(g["out_bf16"]), name)
    # same torch build and thread count as the fixture: expect the reference's bits
    if (str(g["torch_version"]) == torch.__version__ and int(g["num_threads"]) == torch.get_num_threads()
            and str(g["cpu_capability"]) == torch.backends.cpu.get_cpu_capability()):
        np.testing.assert_array_equal(got, g["out_bf16"])


def test_oracle_rows_match_float64():
    name = "t16"
    w = wl.WORKLOADS[name]
    args = wl.make_inputs(name)
    out = cpu_ref.run(*args).float().numpy()
    topk_idx, dense, _, _, _ = cpu_ref.route(args[0], args[1], w.routed_scaling_factor)
    sel = cpu_ref.sorted_selection(topk_idx).numpy()
    sel_w = np.take_along_axis(dense.numpy(), sel, 1)
    tokens = [t for t in range(w.T) if ((sel >= 0) & (sel < 32)).any(1)[t]][:3]
    u8 = lambda t: t.view(torch.uint8).numpy()
    ref = np_ref.rows_fp64(tokens, sel, sel_w, u8(args[2]), args[3].numpy(), u8(args[4]), args[5].numpy(),
                           u8(args[6]), args[7].numpy(), w.local_expert_offset)
    np.testing.assert_allclose(out[tokens], ref, rtol=8e-3, atol=1e-4)


# --- producer-side activation quantiser -------------------------------------

@pytest.mark.parametrize("name", ALL)
def test_quantize_reproduces_reference_inputs(name):
    """On a workload's bf16 hidden states the quantiser restatement gives exactly
    the e4m3 hidden_states and scales the reference was run on (their sha256 in
    the golden fixture)."""
    w = wl.WORKLOADS[name]
    g = load_golden(name)
    q, s = cpu_ref.quantize_activations(wl.hidden_bf16(w.T, w.seed))
    assert wl.fingerprint(q) == str(g["in_sha256"][2])
    assert wl.fingerprint(s) == str(g["in_sha256"][3])


def test_quantize_closed_forms():
    x = quant_edge_rows()
    q, s = cpu_ref.quantize_activations(x)
    codes = q.view(torch.uint8).numpy()
    s = s.numpy()
    # power-of-two scale: every code exact, ties to the even code
    assert s[0, 0] == 2.0 ** -3 and s[1, 0] == 2.0 ** -3
    want = np_ref.e4m3_encode((x[0, :128].float() / 2.0 ** -3).numpy())
    np.testing.assert_array_equal(codes[0, :128], want)
    assert codes[0, 0] == 0x7E                      # the block max is +448
    assert codes[0, 255] == 0xFE                     # and its negation -448
    # all-zero block: zeros with the floor scale
    assert (codes[0, 256:384] == 0).all() and s[2, 0] == np.float32(1e-12) / np.float32(448.0)
    # bf16 subnormals quantise like any other block; -0.0 keeps its sign
    assert codes[1, 384] == 0x80
    np.testing.assert_array_equal(
        codes[1, 256:384], np_ref.e4m3_encode((x[1, 256:384].float() / float(s[2, 1])).clamp(-448, 448).numpy()))
    # the largest bf16 values: scale = amax / 448 stays finite
    assert np.isfinite(s[4, 2]) and codes[2, 639] == 0x7E and codes[2, 512] == 0xFE


def test_quantize_matches_independent_encoder():
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(8, cpu_ref.H, generator=gen) * torch.logspace(-6, 6, 8).unsqueeze(1)).to(torch.bfloat16)
    q, s = cpu_ref.quantize_activations(x)
    xs = (x.float().reshape(8, 56, 128) / s.t().reshape(8, 56, 1)).clamp(-448, 448).reshape(8, -1).numpy()
    np.testing.assert_array_equal(q.view(torch.uint8).numpy(), np_ref.e4m3_encode(xs))


# --- planted mistakes: each must make the checks above fail -----------------

def _swapped_swiglu(A_e, W13_e, W2_e):
    G1 = A_e.matmul(W13_e.t())
    X1, X2 = G1[:, :cpu_ref.I], G1[:, cpu_ref.I:]
    return ((X1 / (1.0 + torch.exp(-X1))) * X2).matmul(W2_e.t())


def _transposed_block_scale(w, s):
    wf = w.to(torch.float32)
    sf = s.to(torch.float32)
    d = wf.dim() - 2
    sf = sf.transpose(d, d + 1).contiguous().reshape(sf.shape)  # scale blocks read in the wrong order
    sf = torch.repeat_interleave(torch.repeat_interleave(sf, 128, dim=d), 128, dim=d + 1)
    return wf * sf


def _route_without_bias(logits, bias, rsf, exp="torch"):
    return _orig_route(logits, torch.zeros_like(bias), rsf, exp=exp)


_orig_route = cpu_ref.route


def test_planted_quantiser_mistake_is_caught(monkeypatch):
    """A quantiser that divides by the e4m3fnuz maximum (240) instead of 448 must
    fail the reference-input check."""
    def wrong(x_bf16):
        T = x_bf16.shape[0]
        xb = x_bf16.to(torch.float32).reshape(T, 56, 128)
        scale = xb.abs().amax(dim=2).clamp(min=1e-12) / 240.0
        q = (xb / scale.unsqueeze(2)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        return q.reshape(T, -1), scale.t().contiguous()
    monkeypatch.setattr(cpu_ref, "quantize_activations", wrong)
    with pytest.raises(AssertionError):
        test_quantize_reproduces_reference_inputs("t16")


@pytest.mark.parametrize("mutation", ["swiglu_halves", "block_scale_order", "bias_dropped"])
def test_planted_mistakes_are_caught(monkeypatch, mutation):
    name = "t16"
    g = load_golden(name)
    args = wl.make_inputs(name)
    if mutation == "swiglu_halves":
        monkeypatch.setattr(cpu_ref, "expert_ffn", _swapped_swiglu)
    elif mutation == "block_scale_order":
        monkeypatch.setattr(cpu_ref, "dequant_weight", _transposed_block_scale)
    else:
        monkeypatch.setattr(cpu_ref, "route", _route_without_bias)
    out = cpu_ref.run(*args)
    got = bf16_bits_to_f32(out.view(torch.int16).numpy().view(np.uint16)[g["out_rows"]])
    with pytest.raises(AssertionError):
        assert_close_bf16(got, bf16_bits_to_f32(g["out_bf16"]), mutation)


def test_router_oracle_pins():
    """cpu_ref.router_logits (torch fp32) against what fixes it independently: the
    float64 restatement within the fp32 summation bound n u / (1 - n u) of sum |x g|
    (n = 7168 terms); one-hot tokens give exactly one scaled gate column; a gate of
    unit rows gives exactly the selected hidden columns."""
    x, g = wl.hidden_bf16(7, 11), wl.gate_weight_bf16()
    got = cpu_ref.router_logits(x, g).numpy().astype(np.float64)
    ref, mag = np_ref.router_logits_f64(x, g)
    n, u = 7168, 2.0 ** -24
    assert (np.abs(got - ref) <= n * u / (1 - n * u) * mag).all()
    assert abs(float(got.std()) - 1.0) < 0.2  # the benchmark's N(0, 1) logits scale
    _router_closed_forms(cpu_ref.router_logits)


def _router_closed_forms(fn):
    g = wl.gate_weight_bf16()
    ks = [0, 127, 128, 3000, 7167]
    x1 = torch.zeros((len(ks), 7168), dtype=torch.bfloat16)
    vals = torch.tensor([1.0, -2.5, 0.0078125, 3.0, -448.0], dtype=torch.bfloat16)
    for i, k in enumerate(ks):
        x1[i, k] = vals[i]
    got = fn(x1, g)
    exp = torch.stack([vals[i].float() * g[:, k].float() for i, k in enumerate(ks)])
    assert torch.equal(got, exp), "one-hot tokens must give one gate column exactly"
    idx = (torch.arange(256) * 28 + 5) % 7168
    gu = torch.zeros((256, 7168), dtype=torch.bfloat16)
    gu[torch.arange(256), idx] = 1.0
    x = wl.hidden_bf16(3, 12)
    assert torch.equal(fn(x, gu), x.float()[:, idx]), "unit gate rows must give the hidden columns exactly"


def test_planted_router_mistake_is_caught():
    """Experts taken in reverse order (a transposed or flipped gate index) fails the closed forms."""
    with pytest.raises(AssertionError):
        _router_closed_forms(lambda x, g: x.float().matmul(g.flip(0).float().t()))

