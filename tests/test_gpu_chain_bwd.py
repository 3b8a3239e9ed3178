"""bolt3_chain_bwd (the consolidation chain's backward for bf16 storage) against the torch
restatement chain_backward, which tests/test_backward_host.py pins to autograd through the
oracle's consolidate.

Both run on one bf16 forward trace of clustered input at head_dim 128 (tokens merge, replace
slots and go to M_res), with seeded gradients for every step's slot keys, slot values and M_res.
The slot path is copies and scalings (fp32 in both); the delta rule's products run on MFMA with
bf16 hi/lo splits in the kernels and in fp32 in torch, so the bound is 1e-4 relative."""
import pytest
import torch

import recipes
from bolt3_amd import Bolt3Attn
from bolt3_amd import _abi as A
from bolt3_amd.backward import chain_backward, chain_backward_hip, replay_slots
from helpers import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b,T,seed", [(1, 1024, 31), (2, 1152, 7)])
def test_chain_backward_kernels_match_torch(b, T, seed, gpu):
    cfg = dict(dim=256, num_heads=8, num_kv_heads=2, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)
    mod = recipes.init_module(Bolt3Attn(cfg), seed, nondefault=True).to(torch.bfloat16).to(gpu)
    x = recipes.clustered_hidden(seed, b, T, 256, n_centres=512, noise=0.15).to(torch.bfloat16).to(gpu)
    print(f"[case] chain backward kernels vs torch b={b} T={T} seed={seed}", flush=True)
    tr = {}
    with torch.no_grad():
        mod._forward_hip(x, tr)
    HKV, HD, S, C = mod.HKV, mod.HD, mod.S, mod.C
    bh = b * HKV
    n = tr["log"].shape[0]
    ns = min(mod.n_sinks, C)
    log = tr["log"]
    assert float(log[:, :, A.LOG_FIELDS.index("merge")].sum()) > 0          # merges happen
    assert float(log[:, :, A.LOG_FIELDS.index("win")].sum()) > 0            # evictions happen
    assert float(log[:, :, A.LOG_FIELDS.index("delta")].sum()) > 0          # M_res writes happen
    g = torch.Generator(device=gpu).manual_seed(seed + 1)
    o = dict(d_slot_k=torch.randn(n, bh, S, HD, generator=g, device=gpu),
             d_slot_v=torch.randn(n, bh, S, HD, generator=g, device=gpu),
             d_m=torch.randn(n, bh, HD, HD, generator=g, device=gpu))
    gam = mod.gamma_delta().detach().to(gpu)
    got = chain_backward_hip(mod, tr, o, gam, b, n)
    pos = torch.arange(T, device=gpu, dtype=torch.float32)
    steps, masses, pms = replay_slots(log, pos, S, C, ns)
    for i in range(n):     # the forward's snapshots are the replay's state
        assert torch.equal(masses[i], tr["snap_mass"][i]), i
        assert torch.equal(pms[i], tr["snap_pm"][i]), i
    want = chain_backward(steps, o["d_slot_k"], o["d_slot_v"], o["d_m"], pms, mod.rope.inv_freq.to(gpu).float(),
                          tr["k_raw"].reshape(bh, T, HD), tr["v"].reshape(bh, T, HD), tr["beta"].reshape(bh, T),
                          gam, tr["snap_m"], True, b, HKV)
    errs = [rel_err(a.float().cpu(), w.float().cpu()) for a, w in zip(got, want)]
    print("  d_kr %.2e d_v %.2e d_beta %.2e d_gamma %.2e" % tuple(errs), flush=True)
    assert max(errs) <= 1e-4, errs
