"""torch.topk's CPU order among equal values, restated (oracle/torch_topk_order.py), against
torch.topk itself.

The reference's slot decisions are torch.topk calls (vsa_lm/config/bolt3.py:137-138, :183).
The kernel reproduces their order among exactly equal values with the wave-parallel form
(``topk_order_wave``), so both restatements are pinned here on arrays built to tie: small
integer ranges, long runs of -1e9 (merged tokens), a sorted run, NaN and -0/+0 mixed in, every
length the kernel sees (124..256) and the partial_sort path (64*k <= n).
"""
import random

import numpy as np
import pytest
import torch

from oracle.torch_topk_order import tie_in_prefix, topk_order_seq, topk_order_wave


def _case(t: int, rng: random.Random):
    n = rng.choice([3, 4, 5, 17, 33, 100, 124, 127, 128, 129, 130, 200, 255, 256])
    k = max(1, min(n, rng.choice([1, 2, 3, 4, n // 2, n - 1, n, min(n, 128), rng.randint(1, n)])))
    r = np.random.default_rng(t)
    kind = t % 7
    if kind == 0:
        v = r.integers(0, 3, n).astype(np.float32)
    elif kind == 1:
        v = r.integers(0, 20, n).astype(np.float32)
    elif kind == 2:
        v = r.standard_normal(n).astype(np.float32)
        v[r.random(n) < 0.5] = -1e9
    elif kind == 3:
        v = np.sort(r.integers(0, 10, n)).astype(np.float32)
        v = v[::-1].copy() if t % 2 else v
    elif kind == 4:
        v = np.full(n, 0.5, np.float32)
        v[r.random(n) < 0.2] = np.nan
    elif kind == 5:
        v = r.integers(0, 4, n).astype(np.float32)
        v[r.random(n) < 0.1] = np.nan
        v[r.random(n) < 0.2] = -0.0
    else:
        v = r.standard_normal(n).astype(np.float32)
    return v, k, rng.random() < 0.5


@pytest.mark.parametrize("form", ["seq", "wave"])
def test_restatement_matches_torch_topk(form):
    rng = random.Random(7)
    bad = []
    for t in range(2500):
        v, k, largest = _case(t, rng)
        want = torch.topk(torch.from_numpy(v), k, largest=largest)[1].tolist()
        if form == "seq":
            got = topk_order_seq(v.tolist(), k, largest)
        else:
            got, limit = topk_order_wave(v.tolist(), k, largest)
            assert not limit, (t, len(v), k)
        if got != want:
            bad.append((t, len(v), k, largest))
    assert not bad, bad[:5]


def test_slot_decision_shapes():
    """The kernel's calls: candidates (n = l tokens, k = min(l, 128), largest) and keep values
    (n = 128 slots, k = min(l, 128), smallest), with runs of equal keeps (mutual nearest slots
    of equal utility) and of -1e9 (merged tokens)."""
    for t in range(300):
        r = np.random.default_rng(1000 + t)
        l = int(r.choice([124, 128, 129, 200, 255, 256]))
        kc = min(l, 128)
        cand = r.random(l).astype(np.float32)
        cand[r.random(l) < 0.4] = -1e9
        keep = (0.15 * 0.995 ** int(r.integers(0, 20)) * (1 - np.minimum(r.random(128), 0.98))).astype(np.float32)
        pairs = r.permutation(128)[:40].reshape(20, 2)
        keep[pairs[:, 1]] = keep[pairs[:, 0]]                    # mutual nearest: equal keep
        keep[r.random(128) < 0.1] = np.float32(0.15 * 0.02)     # saturated redundancy clamp
        for vals, largest in ((cand, True), (keep, False)):
            want = torch.topk(torch.from_numpy(vals), kc, largest=largest)[1].tolist()
            assert topk_order_wave(vals.tolist(), kc, largest)[0] == want


def test_tie_in_prefix():
    assert tie_in_prefix([5.0, 4.0, 4.0, 1.0], 2)
    assert not tie_in_prefix([5.0, 4.0, 3.0, 3.0], 2)
    assert tie_in_prefix([5.0, 4.0, 3.0, 3.0], 3)
    assert tie_in_prefix([0.0, -0.0, 1.0], 1)
    assert tie_in_prefix([float("nan"), float("nan"), 1.0], 1)
