"""Independent NumPy checks for the oracle (TEST INFRASTRUCTURE ONLY).

These restate the operator from the mathematics rather than from torch, so a
mistake in ``oracle/cpu_ref.py`` (a swapped SwiGLU half, a wrong scale index, a
dropped bias, a transposed weight) shows up as a disagreement:

* ``e4m3_value`` / ``e4m3_table`` -- OCP FP8 E4M3 decode from the bit fields
  (bias 7, no infinities, S.1111.111 is NaN, exponent 0 is subnormal m * 2^-9).
* ``brute_force_route`` -- routing by exhaustive search: every one of the
  C(8,4) = 70 group subsets is scored and the best kept, then the 8 largest
  biased scores inside it are taken by a full sort (``ref_moe.py:94-126``).
  Where equal scores straddle a cut the values allow several sets; the one
  torch.topk(sorted=False) keeps is then taken from ``oracle/topk_order.py``
  (std::nth_element's order) and checked to be one of them.
* ``rows_fp64`` -- selected output rows recomputed in float64 from the dequantised
  operands (``ref_moe.py:67-92`` and ``:147-166``).
"""
from __future__ import annotations

import itertools
import math

import numpy as np

H = 7168
I = 2048
BLOCK = 128


def e4m3_value(code: int) -> float:
    sign = -1.0 if code & 0x80 else 1.0
    exp = (code >> 3) & 0xF
    man = code & 0x7
    if exp == 0xF and man == 0x7:
        return math.nan
    if exp == 0:
        return sign * man * 2.0 ** -9
    return sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)


def e4m3_table() -> np.ndarray:
    return np.array([e4m3_value(c) for c in range(256)], dtype=np.float64)


def brute_force_route(logits: np.ndarray, bias: np.ndarray, rsf: float):
    """Per token: (sorted ids of the 8 selected experts, float64 weights in that order).

    ``logits`` fp32 [T,256]; ``bias`` fp32 [256] (already widened from bf16).
    Scores are formed in float32 (exp(-x) correctly rounded to float32, the
    value torch's exp gives on the logits it is used with here); the subset
    search and the weight normalisation run in float64. Ties at a cut are
    resolved in torch.topk(sorted=False)'s order (``oracle/topk_order.py``).
    """
    from oracle import topk_order
    logits = np.asarray(logits, dtype=np.float32)
    bias = np.asarray(bias, dtype=np.float32)
    one = np.float32(1.0)
    s = one / (one + np.exp(-logits.astype(np.float64)).astype(np.float32))
    sb = (s + bias).astype(np.float32)
    ids_out, w_out = [], []
    subsets = list(itertools.combinations(range(8), 4))
    fmin = float(np.finfo(np.float32).min)
    for t in range(logits.shape[0]):
        gscore = []
        for g in range(8):
            vals = sorted(sb[t, g * 32:(g + 1) * 32].tolist(), reverse=True)
            gscore.append(float(np.float32(vals[0]) + np.float32(vals[1])))
        # the best subsets by the sum of their (exact) scores: ties at the cut give several
        score = {sub: sorted((gscore[g] for g in sub), reverse=True) for sub in subsets}
        top = max(score.values())
        best_sets = {frozenset(sub) for sub in subsets if score[sub] == top}
        best = frozenset(topk_order.topk_indices(gscore, 4))
        assert best in best_sets, "torch's group set must be one of the best subsets"
        masked = [float(sb[t, e]) if e // 32 in best else fmin for e in range(256)]
        cand = sorted((masked[e] for e in range(256)), reverse=True)
        ids = sorted(topk_order.topk_indices(masked, 8))
        assert sorted((masked[e] for e in ids), reverse=True) == cand[:8], "8 largest candidates"
        denom = sum(float(s[t, e]) for e in ids) + 1e-20
        ids_out.append(ids)
        w_out.append([float(s[t, e]) / denom * rsf for e in ids])
    return np.array(ids_out, dtype=np.int64), np.array(w_out, dtype=np.float64)


def _dequant_block(w_fp8_as_f64: np.ndarray, scale: np.ndarray) -> np.ndarray:
    n, k = w_fp8_as_f64.shape
    s = np.repeat(np.repeat(scale.astype(np.float64), BLOCK, axis=0), BLOCK, axis=1)
    assert s.shape == (n, k)
    return w_fp8_as_f64 * s


def rows_fp64(tokens, sel_ids, sel_w, hidden_codes, hidden_scale, w13_codes, s13, w2_codes, s2,
              local_expert_offset):
    """float64 output rows for ``tokens``.

    ``sel_ids`` [T,8] selected global ids, ``sel_w`` [T,8] their routing weights,
    ``*_codes`` uint8 e4m3 bit patterns, scales fp32. Returns float64 [len(tokens), H].
    """
    table = e4m3_table()
    out = np.zeros((len(tokens), H), dtype=np.float64)
    cache = {}
    for r, t in enumerate(tokens):
        a = table[hidden_codes[t]] * np.repeat(hidden_scale[:, t].astype(np.float64), BLOCK)
        for j in range(8):
            le = int(sel_ids[t, j]) - int(local_expert_offset)
            if le < 0 or le >= 32:
                continue
            if le not in cache:
                cache[le] = (_dequant_block(table[w13_codes[le]], s13[le]),
                             _dequant_block(table[w2_codes[le]], s2[le]))
            w13, w2 = cache[le]
            g1 = w13 @ a
            x1, x2 = g1[:I], g1[I:]
            c = x1 * (x2 / (1.0 + np.exp(-x2)))
            out[r] += float(sel_w[t, j]) * (w2 @ c)
    return out


def e4m3_encode(x):
    """float32 array -> OCP e4m3 codes (uint8), round to nearest, ties to the even
    code, from the table of finite values (independent of torch's cast). Values
    must lie in [-448, 448]; -0.0 encodes as 0x80."""
    x = np.asarray(x, dtype=np.float32)
    assert np.all(np.abs(x) <= 448.0)
    table = e4m3_table()
    pos_codes = np.arange(0x00, 0x7F)            # 0 .. 448, increasing values
    pos_vals = table[pos_codes]
    a = np.abs(x).astype(np.float64)
    hi = np.clip(np.searchsorted(pos_vals, a, side="left"), 0, len(pos_vals) - 1)
    lo = np.clip(hi - 1, 0, None)
    d_hi = np.abs(pos_vals[hi] - a)
    d_lo = np.abs(a - pos_vals[lo])
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & (pos_codes[lo] % 2 == 0))
    code = np.where(pick_lo, pos_codes[lo], pos_codes[hi]).astype(np.uint8)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)


def router_logits_f64(x_bf16, gate_weight):
    """x @ gate_weight.T in float64 from the bf16 bit patterns (independent of torch's
    matmul): every bf16 x bf16 product is exact in float64 and the 7168-term sums
    carry float64 rounding only. Returns (logits, sum over k of |x_k g_k|), the
    second being the scale of any fp32 summation error."""
    def f64(t):
        bits = t.contiguous().cpu().view(_torch().int16).numpy()
        return (bits.astype(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    xf, gf = f64(x_bf16), f64(gate_weight)
    return xf @ gf.T, np.abs(xf) @ np.abs(gf).T


def _torch():
    import torch
    return torch
