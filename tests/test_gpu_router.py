"""Router GEMM on the GPU (routing_logits = hidden_bf16 @ gate_weight.T, the linear
layer that produces the operator's routing_logits input, reference
moe/weight_origins_dataflow.md:21, :151-154), and the producer chain
hidden_bf16 -> (router logits, FP8 hidden states + scales) -> operator."""
import numpy as np
import pytest
import torch

import flashinfer_mlsys_amd as fm
from flashinfer_mlsys_amd import workloads as wl
from oracle import cpu_ref, np_ref

from conftest import assert_close_bf16

pytestmark = pytest.mark.gpu

N_TERMS, U = 7168, 2.0 ** -24
GAMMA = N_TERMS * U / (1 - N_TERMS * U)  # fp32 summation error bound of a 7168-term dot product


@pytest.fixture(scope="module")
def gate(dev):
    g = wl.gate_weight_bf16()
    return g, g.to(dev)


# token counts on the three kernels (16-token tiles below 576 tokens, 32 x 64 tiles
# with the K steps split over the waves from 576 while they fit on the CUs, 2,048
# tokens on 256 CUs, 128 x 64 tiles beyond) with ragged last tiles and the sizes
# either side of each switch
@pytest.mark.parametrize("T", [1, 5, 16, 17, 64, 100, 575, 576, 1024, 2047, 2048, 2049, 3000, 4100])
def test_router_matches_float64(dev, gate, T):
    print(f"router T={T}", flush=True)
    x = wl.hidden_bf16(T, 900 + T)
    got = fm.router_logits(x.to(dev), gate[1]).cpu().numpy().astype(np.float64)
    ref, mag = np_ref.router_logits_f64(x, gate[0])
    err = np.abs(got - ref)
    assert (err <= GAMMA * mag).all(), f"max error / bound {float((err / (GAMMA * mag)).max()):.3g}"


def test_router_closed_forms(dev, gate):
    """One-hot tokens give exactly one scaled gate column; a gate of unit rows gives
    exactly the selected hidden columns (catches any index or layout mistake)."""
    ks = [0, 127, 128, 3000, 7167]
    x1 = torch.zeros((len(ks), 7168), dtype=torch.bfloat16)
    vals = torch.tensor([1.0, -2.5, 0.0078125, 3.0, -448.0], dtype=torch.bfloat16)
    for i, k in enumerate(ks):
        x1[i, k] = vals[i]
    got = fm.router_logits(x1.to(dev), gate[1]).cpu()
    exp = torch.stack([vals[i].float() * gate[0][:, k].float() for i, k in enumerate(ks)])
    assert torch.equal(got, exp)
    idx = (torch.arange(256) * 28 + 5) % 7168
    gu = torch.zeros((256, 7168), dtype=torch.bfloat16)
    gu[torch.arange(256), idx] = 1.0
    for T in (3, 40, 700, 3100):
        x = wl.hidden_bf16(T, 12)
        assert torch.equal(fm.router_logits(x.to(dev), gu.to(dev)).cpu(), x.float()[:, idx]), T


@pytest.mark.parametrize("T", [8, 2048])
def test_router_deterministic_and_in_place(dev, gate, T):
    x = wl.hidden_bf16(T, 77).to(dev)
    a = fm.router_logits(x, gate[1])
    out = torch.full((T, 256), 5.0, device=dev)
    b = fm.router_logits(x, gate[1], out=out)
    assert b is out and torch.equal(a, b)


@pytest.mark.parametrize("T", [1, 5, 16, 17, 64, 100, 575, 576, 1024, 3000])
def test_fused_producer_equals_separate_kernels(dev, gate, T):
    """router_logits_and_quantize writes the same logits, e4m3 rows and scales, bit
    for bit, as router_logits and quantize_activations (both kernels' tilings, ragged
    tiles); the rows and scales also equal the CPU oracle's quantiser."""
    print(f"fused producer T={T}", flush=True)
    x = wl.hidden_bf16(T, 300 + T)
    xd = x.to(dev)
    lg, q, s = fm.router_logits_and_quantize(xd, gate[1])
    assert torch.equal(lg, fm.router_logits(xd, gate[1]))
    q2, s2 = fm.quantize_activations(xd)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s, s2)
    if T <= 100:
        qr, sr = cpu_ref.quantize_activations(x)
        assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8)) and torch.equal(s.cpu(), sr)


@pytest.mark.parametrize("T", [37, 700])
def test_producer_graph_replay(dev, gate, T):
    """The producer step (fused below 576 tokens, two kernels from 576) captured in a
    HIP graph: each replay, with eager work in between, reproduces the eager result."""
    x = wl.hidden_bf16(T, 41).to(dev)
    bufs = (torch.empty((T, 256), device=dev), torch.empty((T, 7168), dtype=torch.float8_e4m3fn, device=dev),
            torch.empty((56, T), device=dev))
    fm.router_logits_and_quantize(x, gate[1], out=bufs)
    torch.cuda.synchronize()
    ref = [b.clone() for b in bufs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fm.router_logits_and_quantize(x, gate[1], out=bufs)
    for i in range(3):
        for b in bufs:
            b.view(torch.uint8).fill_(0x55)
        fm.router_logits(wl.hidden_bf16(16, 6).to(dev), gate[1])  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for b, r in zip(bufs, ref):
            assert torch.equal(b.view(torch.uint8), r.view(torch.uint8)), f"replay {i}"


# (T, local_expert_offset, seed): the first seed from 9000 + T whose oracle-chain
# selection margins are at least 256 fp32 ulps (the GPU logits differ from the CPU's
# fp32 matmul by summation order, far below that) and that routes a local pair.
CHAIN = [(4, 0, 9004), (48, 96, 9049), (300, 224, 9302)]


@pytest.mark.parametrize("T,offset,seed", CHAIN)
def test_producer_chain_matches_oracle(weights, dev, gate, T, offset, seed):
    """hidden_bf16 -> router_logits + quantize_activations -> kernel, against the oracle
    chain (cpu router, cpu quantiser, cpu operator)."""
    print(f"producer chain T={T} offset={offset} seed={seed}", flush=True)
    x = wl.hidden_bf16(T, seed)
    bias = wl.make_activations(T, seed, offset)[1]
    lg_ref = cpu_ref.router_logits(x, gate[0])
    g, e = cpu_ref.selection_margins(lg_ref, bias)
    assert min(g, e) >= 256, "the seed must keep the selection far from near-ties"
    hq_ref, hs_ref = cpu_ref.quantize_activations(x)
    ref = cpu_ref.run(lg_ref, bias, hq_ref, hs_ref, *weights[0], offset, 2.5).float().numpy()
    xd = x.to(dev)
    lg = fm.router_logits(xd, gate[1])
    hq, hs = fm.quantize_activations(xd)
    out = fm.run(lg, bias.to(dev), hq, hs, *weights[1], offset, 2.5).float().cpu().numpy()
    ids, _, _ = fm.route(lg, bias.to(dev), 2.5)
    ref_ids = cpu_ref.sorted_selection(cpu_ref.route(lg_ref, bias, 2.5)[0])
    assert torch.equal(ids.cpu().long(), ref_ids)
    assert_close_bf16(out, ref, f"chain T={T}")
