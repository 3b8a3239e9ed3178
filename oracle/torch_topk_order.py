"""torch.topk's order among exactly equal values (CPU), restated.

TEST INFRASTRUCTURE ONLY (same rule as bolt3_oracle: only tests/, smoke() and
bench.py's cpu_baseline leg may import it).

The reference picks tokens and slots with ``torch.topk`` on the CPU
(vsa_lm/config/bolt3.py:137-138 for the eviction candidates and the keep
values, :183 for the fill).  Among exactly equal values the order it returns is
not specified by torch's documentation; it is the order of the algorithms its
CPU kernel runs.  That kernel (PyTorch, aten/src/ATen/native/TopKImpl.h, torch
2.10.0 in this build's container; the source is not part of the reference tree)
fills a queue of (value, index) pairs in index order and runs, with a
comparator on the values only (NaN ordered first when ``largest``, last
otherwise):

* ``std::partial_sort(begin, begin + k, end)`` when ``64 * k <= n``;
* otherwise ``std::nth_element(begin, begin + k - 1, end)`` then
  ``std::sort(begin, begin + k - 1)``.

Those are the C++ standard library's introselect / introsort / heap
algorithms (libstdc++'s published implementation: median-of-three pivot moved
to the front, unguarded Hoare partition, insertion sort below 17 (sort) or 4
(select) elements, heap fallbacks at a depth limit of 2*floor(log2 n)).

Two restatements live here:

* ``topk_order_seq`` follows those algorithms step by step;
* ``topk_order_wave`` is the form the HIP kernel runs on one wavefront
  (vsa-lm_amd/csrc/bolt3_chain.hip, ``tie_order_wave``): each Hoare partition
  is computed in one pass from the ranks of its left and right stops, the sort's
  ranges are partitioned independently, and the final insertion sort is a
  stable rank.

tests/test_tie_order.py pins both against torch.topk itself on tie-heavy
arrays (NaN, -0/+0, long runs of equal values, both directions, both library
paths).
"""
from __future__ import annotations

import numpy as np

SORT_THRESHOLD = 16      # ranges of at most this many elements are left to insertion sort
SELECT_THRESHOLD = 3     # introselect stops partitioning at this many elements


def _lg(n: int) -> int:
    return n.bit_length() - 1


def order_key(v: float, largest: bool) -> int:
    """32-bit key, lowest for the element that comes first: NaN first when largest and last
    otherwise; -0 and +0 equal (a float comparison)."""
    f = np.float32(v) + np.float32(0.0)
    if f != f:
        k = 0xFFFFFFFF
    else:
        u = int(np.array([f], np.float32).view(np.uint32)[0])
        k = (~u & 0xFFFFFFFF) if (u & 0x80000000) else (u | 0x80000000)
    return (~k & 0xFFFFFFFF) if largest else k


# ---------------------------------------------------------------- sequential restatement

class _Seq:
    """The library algorithms on a list of (key, index); ``lt`` compares keys only."""

    def __init__(self, keys):
        self.a = [(k, i) for i, k in enumerate(keys)]

    def lt(self, i, j):
        return self.a[i][0] < self.a[j][0]

    def swap(self, i, j):
        self.a[i], self.a[j] = self.a[j], self.a[i]

    def median_to_first(self, res, a, b, c):
        if self.lt(a, b):
            t = b if self.lt(b, c) else (c if self.lt(a, c) else a)
        else:
            t = a if self.lt(a, c) else (c if self.lt(b, c) else b)
        self.swap(res, t)

    def partition(self, f, l):
        """Median of (f+1, mid, l-1) to f, then the unguarded Hoare partition of (f, l)."""
        self.median_to_first(f, f + 1, f + (l - f) // 2, l - 1)
        lo, hi = f + 1, l
        while True:
            while self.lt(lo, f):
                lo += 1
            hi -= 1
            while self.lt(f, hi):
                hi -= 1
            if not lo < hi:
                return lo
            self.swap(lo, hi)
            lo += 1

    def insertion(self, f, l):
        for i in range(f + 1, l):
            v, j = self.a[i], i
            while j > f and v[0] < self.a[j - 1][0]:
                self.a[j] = self.a[j - 1]
                j -= 1
            self.a[j] = v

    # heap (partial_sort and the depth-limit fallbacks)
    def _push(self, f, hole, top, v):
        parent = (hole - 1) // 2
        while hole > top and self.a[f + parent][0] < v[0]:
            self.a[f + hole] = self.a[f + parent]
            hole, parent = parent, (parent - 1) // 2
        self.a[f + hole] = v

    def _adjust(self, f, hole, n, v):
        top, child = hole, hole
        while child < (n - 1) // 2:
            child = 2 * (child + 1)
            if self.a[f + child][0] < self.a[f + child - 1][0]:
                child -= 1
            self.a[f + hole] = self.a[f + child]
            hole = child
        if n % 2 == 0 and child == (n - 2) // 2:
            child = 2 * (child + 1)
            self.a[f + hole] = self.a[f + child - 1]
            hole = child - 1
        self._push(f, hole, top, v)

    def _pop(self, f, l, res):
        v = self.a[res]
        self.a[res] = self.a[f]
        self._adjust(f, 0, l - f, v)

    def heap_select(self, f, m, l):
        if m - f >= 2:
            for parent in range((m - f - 2) // 2, -1, -1):
                self._adjust(f, parent, m - f, self.a[f + parent])
        for i in range(m, l):
            if self.lt(i, f):
                self._pop(f, m, i)

    def sort_heap(self, f, l):
        while l - f > 1:
            l -= 1
            self._pop(f, l, l)

    def partial_sort(self, f, m, l):
        self.heap_select(f, m, l)
        self.sort_heap(f, m)

    def introsort_loop(self, f, l, depth):
        while l - f > SORT_THRESHOLD:
            if depth == 0:
                self.partial_sort(f, l, l)
                return
            depth -= 1
            cut = self.partition(f, l)
            self.introsort_loop(cut, l, depth)
            l = cut

    def sort(self, f, l):
        if l > f:
            self.introsort_loop(f, l, 2 * _lg(l - f))
            self.insertion(f, l)       # final insertion sort (its unguarded half sorts alike)

    def nth_element(self, f, nth, l):
        depth = 2 * _lg(l - f)
        while l - f > SELECT_THRESHOLD:
            if depth == 0:
                self.heap_select(f, nth + 1, l)
                self.swap(f, nth)
                return
            depth -= 1
            cut = self.partition(f, l)
            if cut <= nth:
                f = cut
            else:
                l = cut
        self.insertion(f, l)


def topk_order_seq(values, k: int, largest: bool = True) -> list[int]:
    """Indices of torch.topk(values, k, largest) on the CPU, ties included."""
    n = len(values)
    if k <= 0:
        return []
    s = _Seq([order_key(v, largest) for v in values])
    if 64 * k <= n:
        s.partial_sort(0, k, n)
    else:
        s.nth_element(0, k - 1, n)
        s.sort(0, k - 1)
    return [i for _, i in s.a[:k]]


# ---------------------------------------------------------------- the kernel's form

def _partition_wave(key, idx, f, l):
    """One median move + Hoare partition of (f, l) from the ranks of its stops (all at once)."""
    a, b, c = f + 1, f + (l - f) // 2, l - 1
    if key[a] < key[b]:
        t = b if key[b] < key[c] else (c if key[a] < key[c] else a)
    else:
        t = a if key[a] < key[c] else (c if key[b] < key[c] else b)
    key[f], key[t] = key[t], key[f]
    idx[f], idx[t] = idx[t], idx[f]
    piv = key[f]
    seg = key[a:l]
    stop_l = seg >= piv                       # left scan stops (not ordered before the pivot)
    stop_r = seg <= piv                       # right scan stops (not ordered after it)
    rank_l = np.cumsum(stop_l)                # 1-based rank of each left stop, ascending
    above = int(stop_r.sum()) - np.cumsum(stop_r)   # right stops strictly above a position
    m = int((stop_l & (above >= rank_l)).sum())     # swaps: i-th left stop below the i-th right stop
    pos = np.arange(a, l)
    right_by_rank = {int(r) + 1: int(p) for p, r, s in zip(pos, above, stop_r) if s and r + 1 <= m}
    lefts = pos[stop_l]
    for i in range(1, m + 1):
        p, q = int(lefts[i - 1]), right_by_rank[i]
        key[p], key[q] = key[q], key[p]
        idx[p], idx[q] = idx[q], idx[p]
    l_next = int(lefts[m]) if len(lefts) > m else None
    cands = [x for x in (l_next, right_by_rank.get(m)) if x is not None]
    return min(cands)


def _stable(key, idx, f, l):
    order = sorted(range(f, l), key=lambda i: (key[i], i))
    key[f:l] = key[order].copy()
    idx[f:l] = idx[order].copy()


def topk_order_wave(values, k: int, largest: bool = True) -> tuple[list[int], bool]:
    """The kernel's restatement.  Returns (indices, depth_limit_reached); when the flag is set
    the library's heap fallback would have run and the order is not the library's."""
    n = len(values)
    if k <= 0:
        return [], False
    if 64 * k <= n:
        return topk_order_seq(values, k, largest), False     # heap steps, as in the sequential form
    key = np.array([order_key(v, largest) for v in values], dtype=np.int64)
    idx = np.arange(n)
    limit = False
    f, l, depth = 0, n, 2 * _lg(n)
    while l - f > SELECT_THRESHOLD:
        if depth == 0:
            limit = True
            break
        depth -= 1
        cut = _partition_wave(key, idx, f, l)
        if cut <= k - 1:
            f = cut
        else:
            l = cut
    _stable(key, idx, f, l)
    ks = k - 1
    if ks > SORT_THRESHOLD:
        stack = [(0, ks, 2 * _lg(ks))]
        while stack:
            sf, sl, d = stack.pop()
            if sl - sf <= SORT_THRESHOLD:
                continue
            if d == 0:
                limit = True
                continue
            cut = _partition_wave(key, idx, sf, sl)
            stack += [(cut, sl, d - 1), (sf, cut, d - 1)]
    _stable(key, idx, 0, ks)
    return [int(i) for i in idx[:k]], limit


def tie_in_prefix(sorted_values, n: int) -> bool:
    """Whether a run of equal values in a sorted array reaches into its first n positions (the
    kernel restates the library order only then; elsewhere the order among equal values does
    not change a decision)."""
    v = [order_key(x, False) for x in sorted_values]
    return any((i > 0 and v[i] == v[i - 1]) or (i + 1 < len(v) and v[i] == v[i + 1])
               for i in range(min(n, len(v))))
