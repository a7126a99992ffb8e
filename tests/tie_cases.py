"""Routing inputs whose selections hinge on EXACT ties (test data).

The reference picks groups and experts with ``torch.topk(sorted=False)``
(``reference moe/ref_moe.py:111``, ``:119``); when equal scores straddle the cut
(the 4th and 5th group scores, or the 8th and 9th candidate experts, are equal)
the kept set is fixed by the order ``std::nth_element`` leaves the entries in,
not by the values. Every case here is built so that its values are either exactly
equal or far apart (distinct fp32 sigmoids at least 64 ulps apart near the cuts,
and logits whose float32 sigmoid is the same whether exp is torch's or correctly
rounded), so that the expected selection does not depend on the last bit of exp.

* ``tie_zero_official`` -- all-zero logits under the official workloads' bias
  profile (every bias 4.9375 or 4.96875, ``input_analysis/input_check.ipynb``
  cell 5): the groups holding two high-bias experts tie, and so do the experts.
* ``tie_const``         -- constant logits, zero bias: every group and expert ties.
* ``tie_sets``          -- logits and bias drawn from a few values each.
* ``tie_adversarial``   -- rows built so that introselect exhausts its depth limit
  and takes the heap-select path, with a tie across the 8th/9th expert.
* ``tie_cut``           -- N(0,1) logits, zero bias, with an exact tie planted at
  the group cut (even tokens: the 5th group becomes a copy of the 4th) or at the
  expert cut (odd tokens: the 9th candidate gets the 8th's logit).

``make_case(name)`` returns (logits fp32 [T,256], bias bf16 [256], offset, rsf).
"""
from __future__ import annotations

import numpy as np
import torch

E = 256
FMIN = float(np.finfo(np.float32).min)

# logits whose float32 sigmoid equals the correctly rounded one and torch's
TIE_LOGITS = np.array([-0.5, 0.0, 0.25, 0.5, 0.75, 1.0, 2.0, 3.0], dtype=np.float32)
TIE_BIAS = np.array([0.0, 0.25, 0.5], dtype=np.float32)

CASES = ["tie_zero_official", "tie_const", "tie_sets", "tie_adversarial", "tie_cut"]


def sigmoid_cr(x):
    """float32 1/(1+exp(-x)) with exp(-x) correctly rounded to float32."""
    one = np.float32(1.0)
    return one / (one + np.exp(-np.asarray(x, np.float32).astype(np.float64)).astype(np.float32))


def _official_bias(seed):
    bits = np.random.Generator(np.random.PCG64([seed, 13])).integers(0, 2, E)
    return (np.float32(4.9375) + np.float32(0.03125) * bits.astype(np.float32)).astype(np.float32)


def _adversarial_row(masked_groups):
    """Values (-1 = masked) forcing introselect(256, nth=7) through 16 rounds of
    worst-case median-of-3 pivots into heap-select: McIlroy's adaptive adversary
    ("A killer adversary for quicksort", 1999) freezes an undetermined value
    whenever two meet, making each pivot as small as possible; values still
    undetermined when heap-select starts stay equal (they tie at the top)."""
    from oracle import topk_order as T
    GAS = 1 << 30
    val = [GAS] * E
    for g in masked_groups:
        for i in range(32):
            val[g * 32 + i] = -1
    st = {"n": 0, "cand": None, "on": True}

    def comp(x, y):
        i, j = x[1], y[1]
        if st["on"] and val[i] == GAS and val[j] == GAS:
            k = i if i == st["cand"] else j
            val[k] = st["n"]
            st["n"] += 1
        if val[i] == GAS:
            st["cand"] = i
        elif val[j] == GAS:
            st["cand"] = j
        return val[i] > val[j]

    old_comp, old_hs = T._comp, T._heap_select

    def hs(a, f, m, l):
        st["on"] = False
        old_hs(a, f, m, l)

    T._comp, T._heap_select = comp, hs
    try:
        T.introselect([(0.0, j) for j in range(E)], 7)
    finally:
        T._comp, T._heap_select = old_comp, old_hs
    n = st["n"]
    return [v if v != GAS else n for v in val], n


def _margins_ok(sb, min_ulps=64):
    """Distinct values near both cuts at least min_ulps apart (equal ones allowed);
    the candidates are those of the 4 best groups (any of equal ones: in the
    cases built here equal group scores come from identical groups)."""
    def far(a, b):
        return a == b or abs(float(a) - float(b)) >= min_ulps * float(np.spacing(np.float32(max(abs(a), abs(b)))))
    g = np.sort(sb.reshape(8, 32), axis=1)[:, ::-1]
    gsc = (g[:, 0] + g[:, 1]).astype(np.float32)
    order = np.argsort(-gsc, kind="stable")
    gs = gsc[order]
    if not all(far(gs[i], gs[i + 1]) for i in range(2, 5)):
        return False
    cand = np.sort(np.concatenate([sb[k * 32:(k + 1) * 32] for k in order[:4]]))[::-1]
    return all(far(cand[i], cand[i + 1]) for i in range(5, 10))


def _tie_cut(T, seed):
    rng = np.random.Generator(np.random.PCG64([seed, 31]))
    rows = []
    while len(rows) < T:
        x = rng.standard_normal(E, dtype=np.float32)
        s = sigmoid_cr(x)
        gsc = np.array([np.sort(s[g * 32:(g + 1) * 32])[-2:].sum(dtype=np.float32) for g in range(8)])
        order = np.argsort(-gsc, kind="stable")
        if len(rows) % 2 == 0:  # group cut: the 5th group becomes a copy of the 4th
            g4, g5 = order[3], order[4]
            x[g5 * 32:(g5 + 1) * 32] = x[g4 * 32:(g4 + 1) * 32]
        else:  # expert cut: the 9th candidate takes the 8th's logit
            ids = np.concatenate([np.arange(k * 32, (k + 1) * 32) for k in order[:4]])
            o = ids[np.argsort(-s[ids], kind="stable")]
            x[o[8]] = x[o[7]]
        if _margins_ok(sigmoid_cr(x)):
            rows.append(x)
    return np.stack(rows)


def make_case(name):
    if name == "tie_zero_official":
        return np.zeros((4, E), np.float32), _official_bias(5101), 160, 2.5
    if name == "tie_const":
        lg = np.stack([np.full(E, v, np.float32) for v in (1.0, 0.0, -2.0)])
        return lg, np.zeros(E, np.float32), 160, 2.5
    if name == "tie_sets":
        rng = np.random.default_rng(4242)
        lg = TIE_LOGITS[rng.integers(0, len(TIE_LOGITS), size=(64, E))]
        b = TIE_BIAS[rng.integers(0, len(TIE_BIAS), size=E)]
        return lg.astype(np.float32), b, 0, 2.5
    if name == "tie_adversarial":
        rows = []
        for masked in ([4, 5, 6, 7], [1, 3, 5, 7], [0, 2, 5, 6]):
            vals, n = _adversarial_row(masked)
            # value v -> logit -2 + v/64 (distinct sigmoids far apart); masked groups -> -10
            rows.append(np.array([-10.0 if v < 0 else -2.0 + v / 64.0 for v in vals], np.float32))
        return np.stack(rows), np.zeros(E, np.float32), 0, 2.5
    if name == "tie_cut":
        return _tie_cut(128, 6100), np.zeros(E, np.float32), 0, 2.5
    raise KeyError(name)


def case_tensors(name):
    """(logits fp32 tensor, bias bf16 tensor, offset, rsf); the bias values are exact in bf16."""
    lg, b, off, rsf = make_case(name)
    bias = torch.from_numpy(np.asarray(b, np.float32)).to(torch.bfloat16)
    assert np.array_equal(bias.float().numpy(), np.asarray(b, np.float32))
    return torch.from_numpy(np.ascontiguousarray(lg)), bias, off, rsf
