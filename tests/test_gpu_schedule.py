"""The forward's scheduling aid on the GPU: bolt3_wait_count and the start counter that the
chain's slot-decision workgroups bump (b3_chain_args.started).

* A counter already at or past the target lets the stream through; one below it holds the
  stream for at most max_polls polls (forced from the host with a small poll limit, so the
  kernel always ends) and the work queued behind it still runs.  The comparison is modulo 2^32.
* A bf16 forward bumps the counter once per workgroup of its first step group (B * HKV) and
  gives the same output with the wait as without it (the wait only orders launches).
"""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

CFG = dict(dim=256, num_heads=4, num_kv_heads=2, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)


def _wait(counter, target, polls):
    from bolt3_amd import _abi as A
    rc = A.load().bolt3_wait_count(counter.data_ptr(), target & 0xFFFFFFFF, polls, A.stream_of(counter.device))
    assert rc == 0


def test_wait_count_passes_and_is_bounded(gpu):
    print("[case] bolt3_wait_count", flush=True)
    c = torch.tensor([7], dtype=torch.int32, device=gpu)
    out = torch.zeros(4, device=gpu)
    _wait(c, 7, 1_000_000)          # reached: passes at once
    out[0] = 1
    _wait(c, 3, 1_000_000)          # passed
    out[1] = 1
    _wait(c, 8, 64)                 # not reached: gives up after 64 polls
    out[2] = 1
    c.fill_(-2)                     # 0xFFFFFFFE: target 0xFFFFFFFD is behind it, target 1 ahead
    _wait(c, 0xFFFFFFFD, 1_000_000)
    _wait(c, 1, 64)
    out[3] = 1
    torch.cuda.synchronize()
    assert out.tolist() == [1, 1, 1, 1]


def test_forward_counts_first_group_and_wait_changes_nothing(gpu):
    from bolt3_amd import Bolt3Attn
    from bolt3_amd import bolt3 as B3
    import recipes
    print("[case] forward start counter, B=2 T=2048 bf16", flush=True)
    torch.manual_seed(0)
    mod = recipes.init_module(Bolt3Attn(CFG), 5, nondefault=True).to(torch.bfloat16).to(gpu)
    x = torch.randn(2, 2048, CFG["dim"], device=gpu).to(torch.bfloat16)
    with torch.no_grad():
        y_gated = mod(x)
        ctr = B3._started_counter(gpu)
        torch.cuda.synchronize()
        before = int(ctr[0].item())
        assert before == ctr[1] & 0xFFFFFFFF
        y_gated = mod(x)
        torch.cuda.synchronize()
        assert int(ctr[0].item()) - before == 2 * CFG["num_kv_heads"]
        orig = B3._n_cus
        B3._n_cus = lambda dev: 0      # too few compute units: no counter, no wait
        try:
            y_plain = mod(x)
        finally:
            B3._n_cus = orig
        torch.cuda.synchronize()
        assert int(ctr[0].item()) - before == 2 * CFG["num_kv_heads"]
    assert torch.equal(y_gated, y_plain)
