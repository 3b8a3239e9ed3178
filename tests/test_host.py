"""Host-side logic of the HIP path that runs without a GPU: the step grouping of the forward's
consolidation chain, the packed-parameter cache, the refusal of CPU tensors, and bench.py's
one-GPU contract."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest
import torch

from bolt3_amd import Bolt3Attn
from bolt3_amd.bolt3 import _n_groups, _step_groups

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CFG = dict(dim=64, num_heads=4, num_kv_heads=2, head_dim=16, rope_theta=1e4, eps=1e-6, qk_norm=True)


@pytest.mark.parametrize("n", [1, 2, 3, 5, 14, 30, 62, 510])
@pytest.mark.parametrize("k", [1, 2, 3, 4, 6])
def test_step_groups_cover_the_steps_in_order(n, k):
    g = _step_groups(n, k)
    assert 1 <= len(g) <= min(k, n)
    assert g[0][0] == 0 and g[-1][1] == n
    assert all(s0 < s1 for s0, s1 in g)
    assert all(g[i][1] == g[i + 1][0] for i in range(len(g) - 1))
    if len(g) > 2:
        # the first group is the short one, the others within one step of each other
        rest = [s1 - s0 for s0, s1 in g[1:]]
        assert g[0][1] - g[0][0] <= min(rest)
        assert max(rest) - min(rest) <= 1


def test_step_groups_of_the_benchmark_forward():
    # cfg2: T = 4096, C = 128 -> 30 consolidation steps, three groups
    assert _n_groups(30) == 3
    assert _step_groups(30, 3) == [(0, 8), (8, 19), (19, 30)]
    # the consolidation-heavy configuration: T = 65536 -> 510 steps in 16 groups of about 32
    assert _n_groups(510) == 16
    g = _step_groups(510, 16)
    assert len(g) == 16 and max(s1 - s0 for s0, s1 in g) <= 33


def test_packed_parameters_follow_in_place_updates():
    torch.manual_seed(0)
    mod = Bolt3Attn(CFG)
    W1, _, side1 = mod._packed(torch.float32, torch.device("cpu"))
    assert mod._packed(torch.float32, torch.device("cpu"))[0] is W1      # cached while nothing changes
    with torch.no_grad():
        mod.k_proj.weight.add_(1.0)
    W2, _, side2 = mod._packed(torch.float32, torch.device("cpu"))
    assert W2 is not W1
    kw = mod.k_proj.weight
    H, HD = CFG["num_heads"], CFG["head_dim"]
    assert torch.equal(W2[H * HD:H * HD + kw.shape[0]], kw)
    # the forward's split projections and the decoder's packed one hold the same rows
    assert torch.equal(side2["wkv"][:kw.shape[0]], kw)
    assert W2.shape[0] % 16 == 0 and side2["wq"].shape[0] % 16 == 0


def test_forward_refuses_cpu_tensors():
    mod = Bolt3Attn(CFG)
    with pytest.raises(RuntimeError, match="ROCm device"):
        mod(torch.zeros(1, 8, CFG["dim"]))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr
