"""torch.topk(..., largest=True, sorted=False) on the CPU, restated (TEST INFRASTRUCTURE ONLY).

The reference selects groups and experts with ``torch.topk(sorted=False)``
(``reference moe/ref_moe.py:107``, ``:111``, ``:119``). On the CPU torch runs
``topk_impl_loop`` (``ATen/native/TopKImpl.h:14-95`` in torch 2.10.0): it fills a
queue of (value widened to double, index) pairs in index order and, when
``k * 64 > n`` (true for all three calls: 2 of 32, 4 of 8, 8 of 256), calls
``std::nth_element(queue, queue + k - 1, end, comp)`` with
``comp(x, y) = (isnan(x) && !isnan(y)) || x > y`` and returns the first k
entries. Which of several EQUAL values end up among the first k is therefore
fixed by libstdc++'s introselect, the third-party algorithm the selection's tie
order lives in. torch 2.10.0 was built with GCC 11.2 (``torch.__config__.show()``);
the steps below follow that release's ``bits/stl_algo.h`` (``__introselect``,
``__unguarded_partition_pivot``, ``__move_median_to_first``,
``__unguarded_partition``, ``__insertion_sort``, ``__heap_select``) and
``bits/stl_heap.h`` (``__make_heap``, ``__adjust_heap``, ``__push_heap``,
``__pop_heap``):

* depth limit ``2 * floor(log2 n)``; while more than 3 elements remain: at depth
  0 heap-select the first nth+1 and swap the first with the nth, done;
  otherwise move the median of (first+1, mid, last-1) to first, Hoare-partition
  the rest around it and keep the side that holds nth;
* finally insertion-sort the (at most 3) remaining elements.

Pinned by ``tests/test_topk_order.py``: identical indices, in the same order, as
``torch.topk`` on rows with heavy ties (few distinct values, masked -FLT_MAX
halves, all-equal rows), at the three shapes the operator uses, including rows
that exhaust the depth limit. Pure Python: for the small cases of the tests.
"""
from __future__ import annotations

import math


def _comp(x, y):
    # x, y: (value, index); "x goes before y" for largest=True
    return (math.isnan(x[0]) and not math.isnan(y[0])) or x[0] > y[0]


def _move_median_to_first(a, result, i, j, k):
    if _comp(a[i], a[j]):
        if _comp(a[j], a[k]):
            m = j
        elif _comp(a[i], a[k]):
            m = k
        else:
            m = i
    elif _comp(a[i], a[k]):
        m = i
    elif _comp(a[j], a[k]):
        m = k
    else:
        m = j
    a[result], a[m] = a[m], a[result]


def _unguarded_partition(a, first, last, pivot):
    while True:
        while _comp(a[first], a[pivot]):
            first += 1
        last -= 1
        while _comp(a[pivot], a[last]):
            last -= 1
        if not first < last:
            return first
        a[first], a[last] = a[last], a[first]
        first += 1


def _partition_pivot(a, first, last):
    mid = first + (last - first) // 2
    _move_median_to_first(a, first, first + 1, mid, last - 1)
    return _unguarded_partition(a, first + 1, last, first)


def _insertion_sort(a, first, last):
    if first == last:
        return
    for i in range(first + 1, last):
        if _comp(a[i], a[first]):
            val = a[i]
            a[first + 1:i + 1] = a[first:i]
            a[first] = val
        else:
            val = a[i]
            hole, nxt = i, i - 1
            while _comp(val, a[nxt]):
                a[hole] = a[nxt]
                hole, nxt = nxt, nxt - 1
            a[hole] = val


def _push_heap(a, first, hole, top, value):
    parent = (hole - 1) // 2
    while hole > top and _comp(a[first + parent], value):
        a[first + hole] = a[first + parent]
        hole = parent
        parent = (hole - 1) // 2
    a[first + hole] = value


def _adjust_heap(a, first, hole, n, value):
    top = hole
    child = hole
    while child < (n - 1) // 2:
        child = 2 * (child + 1)
        if _comp(a[first + child], a[first + child - 1]):
            child -= 1
        a[first + hole] = a[first + child]
        hole = child
    if n % 2 == 0 and child == (n - 2) // 2:
        child = 2 * (child + 1)
        a[first + hole] = a[first + child - 1]
        hole = child - 1
    _push_heap(a, first, hole, top, value)


def _make_heap(a, first, last):
    n = last - first
    if n < 2:
        return
    parent = (n - 2) // 2
    while True:
        _adjust_heap(a, first, parent, n, a[first + parent])
        if parent == 0:
            return
        parent -= 1


def _heap_select(a, first, middle, last):
    _make_heap(a, first, middle)
    for i in range(middle, last):
        if _comp(a[i], a[first]):
            value = a[i]  # __pop_heap(first, middle, i)
            a[i] = a[first]
            _adjust_heap(a, first, 0, middle - first, value)


def introselect(a, nth, stats=None):
    """std::nth_element(a.begin(), a.begin() + nth, a.end(), comp) in place on a
    list of (value, index) pairs. ``stats``, if a dict, receives the number of
    partition rounds and whether the heap-select fallback ran."""
    first, last = 0, len(a)
    if first == last or nth == last:
        return a
    depth = 2 * ((last - first).bit_length() - 1)
    rounds = 0
    while last - first > 3:
        if depth == 0:
            _heap_select(a, first, nth + 1, last)
            a[first], a[nth] = a[nth], a[first]
            if stats is not None:
                stats.update(rounds=rounds, heap_select=True)
            return a
        depth -= 1
        rounds += 1
        cut = _partition_pivot(a, first, last)
        if cut <= nth:
            first = cut
        else:
            last = cut
    _insertion_sort(a, first, last)
    if stats is not None:
        stats.update(rounds=rounds, heap_select=False)
    return a


def topk_indices(values, k, stats=None):
    """Indices torch.topk(values, k, largest=True, sorted=False) returns on the CPU,
    in its order, for one row of float32 values (given as Python floats)."""
    n = len(values)
    assert 0 < k <= n
    assert k * 64 > n, "the partial_sort branch of topk_impl_loop is not restated"
    q = [(float(v), j) for j, v in enumerate(values)]
    introselect(q, k - 1, stats)
    return [j for _, j in q[:k]]
