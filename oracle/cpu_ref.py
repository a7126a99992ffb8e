"""PyTorch-on-CPU restatement of the reference operator (TEST INFRASTRUCTURE ONLY).

Follows ``reference moe/ref_moe.py:4-168`` operation by operation in fp32 so that,
on the same torch build, it reproduces the reference's routing bits exactly and
its output to within CPU SGEMM ordering. Only tests, the smoke check and the
CPU-baseline leg of the benchmark use it.

Pinned by: the golden vectors written from the reference itself
(``tests/golden/``), the OCP-e4m3 decode table, the brute-force routing search
and the float64 recomputation in ``oracle/np_ref.py``.
"""
from __future__ import annotations

import torch

H = 7168
I = 2048
E_GLOBAL = 256
E_LOCAL = 32
BLOCK = 128
TOP_K = 8
N_GROUP = 8
TOPK_GROUP = 4
GROUP_SIZE = E_GLOBAL // N_GROUP


def check_geometry(routing_logits, hidden_states, hidden_states_scale, gemm1_weights,
                   gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, routing_bias):
    """Shape asserts of ``ref_moe.py:33-63``."""
    T = routing_logits.shape[0]
    assert routing_logits.shape[1] == E_GLOBAL, "num_experts must be 256"
    assert gemm1_weights.shape[0] == E_LOCAL, "num_local_experts must be 32"
    assert hidden_states.shape == (T, H)
    assert hidden_states_scale.shape == (H // BLOCK, T)
    assert gemm1_weights.shape == (E_LOCAL, 2 * I, H)
    assert gemm1_weights_scale.shape == (E_LOCAL, 2 * I // BLOCK, H // BLOCK)
    assert gemm2_weights.shape == (E_LOCAL, H, I)
    assert gemm2_weights_scale.shape == (E_LOCAL, H // BLOCK, I // BLOCK)
    assert routing_bias.shape[-1] == E_GLOBAL
    return T


def dequant_hidden(hidden_states, hidden_states_scale):
    """``ref_moe.py:67-78``: A[t,h] = fp8(x[t,h]) * S[h/128, t] in fp32."""
    T = hidden_states.shape[0]
    a = hidden_states.to(torch.float32)
    s_th = hidden_states_scale.to(torch.float32).permute(1, 0).contiguous()
    s_full = s_th.unsqueeze(-1).repeat(1, 1, BLOCK).reshape(T, H).contiguous()
    return a * s_full


def quantize_activations(x_bf16):
    """Producer-side quantiser, the step before the operator: per 1x128 block of
    bf16 hidden states, scale = max(amax, 1e-12) / 448 and q = e4m3(x / scale)
    (torch's round-to-nearest-even cast), as solution/triton/dsl-temp1.py:479-484
    quantises an activation. bf16 [T, 7168] -> (e4m3 [T, 7168], fp32 [56, T]).
    The clamp to +-448 only guards the division's last-bit rounding (torch rounds
    such values to 448 anyway)."""
    T = x_bf16.shape[0]
    xb = x_bf16.to(torch.float32).reshape(T, H // BLOCK, BLOCK)
    scale = xb.abs().amax(dim=2).clamp(min=1e-12) / 448.0
    q = (xb / scale.unsqueeze(2)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.reshape(T, H), scale.t().contiguous()


def router_logits(x_bf16, gate_weight):
    """Router GEMM, ``reference moe/weight_origins_dataflow.md:21, :151-154``:
    routing_logits [T, 256] fp32 = x [T, 7168] @ gate_weight.T ([256, 7168]), a linear
    layer with no activation, on bf16 inputs computed in fp32."""
    return x_bf16.to(torch.float32).matmul(gate_weight.to(torch.float32).t())


def dequant_weight(w, s):
    """``ref_moe.py:80-92`` for one or more experts: W = fp8 * S[n/128, k/128] in fp32."""
    wf = w.to(torch.float32)
    sf = s.to(torch.float32)
    dim_n = wf.dim() - 2
    sf = torch.repeat_interleave(sf, BLOCK, dim=dim_n)
    sf = torch.repeat_interleave(sf, BLOCK, dim=dim_n + 1)
    return wf * sf


def route(routing_logits, routing_bias, routed_scaling_factor, exp="torch"):
    """noaux_tc routing, ``ref_moe.py:94-126``.

    Returns (topk_idx [T,8] int64 in torch.topk's own order, weights [T,256] fp32,
    s [T,256], s_with_bias [T,256], group_scores [T,8]).

    ``exp="torch"`` evaluates exp(-x) with torch's float32 exp, as the reference
    does; ``exp="correctly_rounded"`` takes exp(-x) in float64 rounded once to
    float32 (the HIP kernel's rule). The two differ in the last bit on about
    0.4 % of logits, which can flip a selection only where two candidates lie
    within an ulp of each other at a cut; every other step is the reference's.
    """
    T = routing_logits.shape[0]
    logits = routing_logits.to(torch.float32)
    bias = routing_bias.to(torch.float32).reshape(-1)
    if exp == "torch":
        e = torch.exp(-logits)
    elif exp == "correctly_rounded":
        e = torch.exp(-logits.to(torch.float64)).to(torch.float32)
    else:
        raise ValueError(exp)
    s = 1.0 / (1.0 + e)
    s_with_bias = s + bias
    grouped = s_with_bias.view(T, N_GROUP, GROUP_SIZE)
    top2_vals, _ = torch.topk(grouped, k=2, dim=2, largest=True, sorted=False)
    group_scores = top2_vals.sum(dim=2)
    _, group_idx = torch.topk(group_scores, k=TOPK_GROUP, dim=1, largest=True, sorted=False)
    group_mask = torch.zeros_like(group_scores)
    group_mask.scatter_(1, group_idx, 1.0)
    score_mask = group_mask.unsqueeze(2).expand(T, N_GROUP, GROUP_SIZE).reshape(T, E_GLOBAL)
    pruned = s_with_bias.masked_fill(score_mask == 0, torch.finfo(torch.float32).min)
    _, topk_idx = torch.topk(pruned, k=TOP_K, dim=1, largest=True, sorted=False)
    m = torch.zeros_like(s)
    m.scatter_(1, topk_idx, 1.0)
    weights = s * m
    weights_sum = weights.sum(dim=1, keepdim=True) + 1e-20
    weights = (weights / weights_sum) * routed_scaling_factor
    return topk_idx, weights, s, s_with_bias, group_scores


def dispatch(topk_idx, local_expert_offset):
    """Per-local-expert token lists in ascending token order, ``ref_moe.py:131-145``.

    Returns a list of 32 int64 tensors (empty where the expert has no token or its
    global id falls outside [0, 256)).
    """
    lists = []
    for le in range(E_LOCAL):
        ge = int(local_expert_offset) + le
        if ge < 0 or ge >= E_GLOBAL:
            lists.append(torch.empty(0, dtype=torch.int64))
            continue
        sel = (topk_idx == ge).any(dim=1)
        lists.append(torch.nonzero(sel, as_tuple=False).squeeze(1))
    return lists


def sorted_selection(topk_idx):
    """The selected expert set per token as ascending ids (canonical order)."""
    return torch.sort(topk_idx, dim=1).values


def expert_ffn(A_e, W13_e, W2_e):
    """One expert's GEMM1 -> SwiGLU -> GEMM2 in fp32, ``ref_moe.py:152-162``."""
    G1 = A_e.matmul(W13_e.t())
    X1 = G1[:, :I]
    X2 = G1[:, I:]
    silu_X2 = X2 / (1.0 + torch.exp(-X2))
    C = silu_X2 * X1
    return C.matmul(W2_e.t())


@torch.no_grad()
def run(routing_logits, routing_bias, hidden_states, hidden_states_scale,
        gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale,
        local_expert_offset, routed_scaling_factor, materialize_all=False, exp="torch"):
    """Whole operator on the CPU, ``ref_moe.py:4-168``; returns bf16 [T, 7168].

    ``materialize_all=True`` dequantises all 32 experts up front as the reference
    does (its dominant fixed cost, used for the CPU baseline timing). The default
    dequantises each expert when it is first used; the values are elementwise
    identical, so the output is the same. ``exp`` as in ``route``.
    """
    T = check_geometry(routing_logits, hidden_states, hidden_states_scale, gemm1_weights,
                       gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, routing_bias)
    A = dequant_hidden(hidden_states, hidden_states_scale)
    if materialize_all:
        W13_all = dequant_weight(gemm1_weights, gemm1_weights_scale)
        W2_all = dequant_weight(gemm2_weights, gemm2_weights_scale)
    topk_idx, weights, _, _, _ = route(routing_logits, routing_bias, routed_scaling_factor, exp=exp)

    output = torch.zeros((T, H), dtype=torch.float32)
    lists = dispatch(topk_idx, local_expert_offset)
    for le in range(E_LOCAL):
        token_idx = lists[le]
        if token_idx.numel() == 0:
            continue
        ge = int(local_expert_offset) + le
        if materialize_all:
            W13_e, W2_e = W13_all[le], W2_all[le]
        else:
            W13_e = dequant_weight(gemm1_weights[le], gemm1_weights_scale[le])
            W2_e = dequant_weight(gemm2_weights[le], gemm2_weights_scale[le])
        A_e = A.index_select(0, token_idx)
        O = expert_ffn(A_e, W13_e, W2_e)
        w_tok = weights.index_select(0, token_idx)[:, ge]
        output.index_add_(0, token_idx, O * w_tok.unsqueeze(1))
    return output.to(torch.bfloat16)


def selection_margins(routing_logits, routing_bias):
    """Smallest gaps at the two selection boundaries, in fp32 ulps of the larger value.

    Returns (min over tokens of (4th - 5th group score), min over tokens of
    (8th - 9th candidate s_with_bias among the kept groups)), each as ulps.
    A gap of a few ulps could flip a selection between two exp implementations.
    """
    T = routing_logits.shape[0]
    if T == 0:
        return float("inf"), float("inf")
    _, _, _, sb, gs = route(routing_logits, routing_bias, 1.0)
    gsort = torch.sort(gs, dim=1, descending=True).values
    g_gap = (gsort[:, 3] - gsort[:, 4]) / torch.abs(gsort[:, 3]).clamp_min(1e-30) / 2 ** -23
    top4 = torch.topk(gs, k=TOPK_GROUP, dim=1).indices
    keep = torch.zeros_like(gs, dtype=torch.bool).scatter_(1, top4, True)
    cand = sb.masked_fill(~keep.repeat_interleave(GROUP_SIZE, dim=1), float("-inf"))
    csort = torch.sort(cand, dim=1, descending=True).values
    e_gap = (csort[:, 7] - csort[:, 8]) / torch.abs(csort[:, 7]).clamp_min(1e-30) / 2 ** -23
    return float(g_gap.min()), float(e_gap.min())
