"""bolt3_chain_bwd (the consolidation chain's backward) against the torch restatement
chain_backward (tests/chain_bwd_ref.py), which tests/test_backward_host.py pins to autograd
through the oracle's consolidate.

Both run on one forward trace of clustered input (tokens merge, replace slots and go to M_res),
with seeded gradients for every step's slot keys, slot values and M_res: bf16 and fp32 storage,
head_dim 128 and 64, and chunks of 64 tokens (steps shorter than the kernels' 128-token tiles,
zero-padded).  The slot path is copies and scalings (fp32 in both); the delta rule's products run
on MFMA with bf16 hi/lo splits in the kernels and in fp32 in torch, so the bound is 1e-4
relative."""
import pytest
import torch

import recipes
from bolt3_amd import Bolt3Attn
from bolt3_amd import _abi as A
from bolt3_amd.backward import chain_backward_hip
from chain_bwd_ref import chain_backward, replay_slots
from helpers import rel_err

pytestmark = pytest.mark.gpu

CASES = [  # dtype, head_dim, heads (H, HKV), C, b, T, seed
    (torch.bfloat16, 128, (8, 2), 128, 1, 1024, 31),
    (torch.bfloat16, 128, (8, 2), 128, 2, 1152, 7),
    (torch.float32, 128, (8, 2), 128, 1, 1024, 31),
    (torch.bfloat16, 64, (4, 2), 128, 2, 1024, 11),
    (torch.float32, 64, (4, 2), 128, 2, 1024, 11),
    (torch.bfloat16, 128, (8, 2), 64, 1, 768, 13),
    (torch.float32, 64, (4, 2), 64, 1, 704, 17),
]


@pytest.mark.parametrize("dtype,head_dim,heads,C,b,T,seed", CASES)
def test_chain_backward_kernels_match_torch(dtype, head_dim, heads, C, b, T, seed, gpu):
    H, HKV = heads
    cfg = dict(dim=256, num_heads=H, num_kv_heads=HKV, head_dim=head_dim, rope_theta=1e6, eps=1e-6, qk_norm=True)
    mod = recipes.init_module(Bolt3Attn(cfg, C=C), seed, nondefault=True).to(dtype).to(gpu)
    x = recipes.clustered_hidden(seed, b, T, 256, n_centres=512, noise=0.15).to(dtype).to(gpu)
    print(f"[case] chain backward kernels vs torch {dtype} head_dim={head_dim} C={C} b={b} T={T} seed={seed}",
          flush=True)
    tr = {}
    with torch.no_grad():
        mod._forward_hip(x, tr)
    HD, S = mod.HD, mod.S
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
                          gam, tr["snap_m"], dtype == torch.bfloat16, b, HKV)
    errs = [rel_err(a.float().cpu(), w.float().cpu()) for a, w in zip(got, want)]
    print("  d_kr %.2e d_v %.2e d_beta %.2e d_gamma %.2e" % tuple(errs), flush=True)
    assert max(errs) <= 1e-4, errs
