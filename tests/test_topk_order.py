"""The tie order of torch.topk(sorted=False): the restatement in oracle/topk_order.py
against torch itself and against the reference's selections on exact-tie inputs.

The reference's routing (``reference moe/ref_moe.py:107-119``) keeps whatever
std::nth_element leaves in front when equal scores straddle a cut; these tests
pin that order (CPU only).
"""
import os

import numpy as np
import pytest
import torch

from oracle import cpu_ref, np_ref, topk_order
from conftest import GOLDEN_DIR

import tie_cases as tc

FMIN = float(np.finfo(np.float32).min)


def _torch_topk(row, k):
    return torch.topk(torch.from_numpy(np.asarray(row, np.float32)), k, largest=True, sorted=False).indices.tolist()


def _tie_rows(n, count, seed, mask):
    rng = np.random.default_rng(seed)
    for _ in range(count):
        nv = int(rng.integers(1, 7))
        vals = rng.normal(size=nv).astype(np.float32)
        row = vals[rng.integers(0, nv, n)]
        if mask and rng.random() < 0.7:  # four masked groups, as the expert selection sees them
            for g in rng.permutation(8)[:4]:
                row[g * 32:(g + 1) * 32] = FMIN
        yield row


@pytest.mark.parametrize("n,k", [(8, 4), (32, 2), (256, 8)])
def test_restatement_matches_torch_on_ties(n, k):
    """Same indices in the same order as torch.topk, on rows of few distinct values."""
    for row in _tie_rows(n, 600, 100 + n, mask=n == 256):
        assert topk_order.topk_indices(row.tolist(), k) == _torch_topk(row, k)


@pytest.mark.parametrize("n,k", [(8, 4), (32, 2), (256, 8)])
def test_restatement_all_equal(n, k):
    row = np.full(n, 0.5, np.float32)
    got = topk_order.topk_indices(row.tolist(), k)
    assert got == _torch_topk(row, k)
    if n == 256:
        assert sorted(got) == list(range(168, 176))  # not the lowest ids


@pytest.mark.parametrize("masked", [[4, 5, 6, 7], [1, 3, 5, 7], [0, 2, 5, 6]])
def test_restatement_heap_select_path(masked):
    """Rows that exhaust the depth limit (16 rounds at n = 256) and take the
    heap-select fallback, with the 8th and 9th largest values equal."""
    vals, n = tc._adversarial_row(masked)
    row = np.array([FMIN if v < 0 else float(v) for v in vals], np.float32)
    st = {}
    got = topk_order.topk_indices(row.tolist(), 8, st)
    assert st["heap_select"] and st["rounds"] == 16
    srt = np.sort(row)[::-1]
    assert srt[7] == srt[8], "a tie straddles the cut"
    assert got == _torch_topk(row, 8)


def _fixture(name):
    path = os.path.join(GOLDEN_DIR, f"ties_{name}.npz")
    if not os.path.exists(path):
        pytest.skip(f"tie fixture {name} not generated")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _inputs(z):
    lg = torch.from_numpy(z["logits"])
    b = torch.from_numpy(z["bias_bf16"].view(np.int16)).view(torch.bfloat16)
    return lg, b


def _restated_route(lg, b):
    _, _, _, sb, gs = cpu_ref.route(lg, b, 1.0)
    out = []
    for t in range(lg.shape[0]):
        groups = topk_order.topk_indices(gs[t].tolist(), 4)
        keep = torch.zeros(256, dtype=torch.bool)
        for g in groups:
            keep[g * 32:(g + 1) * 32] = True
        out.append(topk_order.topk_indices(sb[t].masked_fill(~keep, FMIN).tolist(), 8))
    return np.array(out)


@pytest.mark.parametrize("name", tc.CASES)
def test_tie_fixture_inputs_regenerate(name):
    z = _fixture(name)
    lg, b, off, rsf = tc.make_case(name)
    np.testing.assert_array_equal(z["logits"], lg)
    np.testing.assert_array_equal(z["bias_bf16"], tc.case_tensors(name)[1].view(torch.int16).numpy().view(np.uint16))
    assert int(z["local_expert_offset"]) == off and float(z["routed_scaling_factor"]) == rsf


@pytest.mark.parametrize("name", tc.CASES)
def test_reference_tie_order_reproduced(name):
    """The reference's own topk_idx (captured from its third torch.topk) equals the
    oracle route's and the restated introselect's, entry for entry; the brute-force
    search, resolving its ties the same way, gives the same sets."""
    z = _fixture(name)
    lg, b = _inputs(z)
    ids, dense, _, _, _ = cpu_ref.route(lg, b, float(z["routed_scaling_factor"]))
    np.testing.assert_array_equal(ids.numpy(), z["topk_idx"].astype(np.int64))
    np.testing.assert_array_equal(_restated_route(lg, b), z["topk_idx"].astype(np.int64))
    bf_ids, bf_w = np_ref.brute_force_route(lg.numpy(), b.float().numpy(), float(z["routed_scaling_factor"]))
    np.testing.assert_array_equal(bf_ids, z["sel_ids"].astype(np.int64))
    np.testing.assert_allclose(np.take_along_axis(dense.numpy(), bf_ids, 1), bf_w, rtol=1e-6)


def test_ties_differ_from_lowest_id_rule():
    """The fixtures exercise the order: the lowest-id-first rule picks other sets."""
    differ = 0
    for name in tc.CASES:
        z = _fixture(name)
        lg, b = _inputs(z)
        _, _, _, sb, gs = cpu_ref.route(lg, b, 1.0)
        for t in range(lg.shape[0]):
            g = np.argsort(-gs[t].numpy(), kind="stable")[:4]
            keep = np.zeros(256, bool)
            for k in g:
                keep[k * 32:(k + 1) * 32] = True
            low = np.sort(np.argsort(-np.where(keep, sb[t].numpy(), FMIN), kind="stable")[:8])
            differ += not np.array_equal(low, z["sel_ids"][t])
    assert differ >= 50


@pytest.mark.parametrize("mistake", ["median_of_first_mid_last", "depth_limit_log2"])
def test_planted_introselect_mistake_is_caught(monkeypatch, mistake):
    """A plausible slip in the restatement changes the order on the fixtures."""
    if mistake == "median_of_first_mid_last":
        orig = topk_order._partition_pivot

        def pivot(a, first, last):
            mid = first + (last - first) // 2
            topk_order._move_median_to_first(a, first, first, mid, last - 1)
            return topk_order._unguarded_partition(a, first + 1, last, first)
        monkeypatch.setattr(topk_order, "_partition_pivot", pivot)
        assert orig is not pivot
    else:
        orig = topk_order.introselect

        def shallow(a, nth, stats=None):
            # depth limit log2(n) instead of 2 log2(n)
            first, last = 0, len(a)
            depth = (last - first).bit_length() - 1
            while last - first > 3:
                if depth == 0:
                    topk_order._heap_select(a, first, nth + 1, last)
                    a[first], a[nth] = a[nth], a[first]
                    return a
                depth -= 1
                cut = topk_order._partition_pivot(a, first, last)
                first, last = (cut, last) if cut <= nth else (first, cut)
            topk_order._insertion_sort(a, first, last)
            return a
        monkeypatch.setattr(topk_order, "introselect", shallow)
    caught = 0
    for name in tc.CASES:
        z = _fixture(name)
        lg, b = _inputs(z)
        caught += not np.array_equal(_restated_route(lg, b), z["topk_idx"].astype(np.int64))
    assert caught > 0
