"""RoPE at the configurations' positions on the GPU: the head preparation (bolt3_heads) at
pos0 = 8192 (the decode configuration), 32768 and 65408 (the end of the consolidation-heavy
prefill), and the slot keys (bolt3_slot_keys) at fractional mean positions up to 65535, against
the oracle's rope_at (vsa_lm/surgery.py:86-93, vsa_lm/config/bolt3.py:17-20).  fp32: relative
error <= 1e-4.  bf16: every element equal except where the oracle's fp32 cos / sin lie within
2 fp32 ulps of a bf16 rounding boundary (their rounding may go either way), and those differ by
at most one bf16 ulp."""
import pytest
import torch
import torch.nn.functional as F

import recipes
from helpers import rel_err
from oracle import bolt3_oracle as O

pytestmark = pytest.mark.gpu

CASES = [(torch.float32, 128, 1e6), (torch.bfloat16, 128, 1e6), (torch.float32, 64, 1e4), (torch.bfloat16, 64, 1e4)]


def _module(hd, theta, dt):
    from bolt3_amd import Bolt3Attn
    cfg = dict(dim=256, num_heads=4, num_kv_heads=2, head_dim=hd, rope_theta=theta, eps=1e-6, qk_norm=True)
    return recipes.init_module(Bolt3Attn(cfg), 3, nondefault=True).to(dt)


def _near_boundary(pos, inv_freq, dt):
    """[T, HD] mask of rotation entries whose fp32 cos or sin lies within 2 fp32 ulps of the
    midpoint between two bf16 neighbours (low 16 bits near 0x8000), where rounding to bf16 may go
    either way for values a few ulps apart."""
    ang = pos.float()[:, None] * inv_freq.float()[None, :]
    ang = torch.cat((ang, ang), dim=-1)
    mask = torch.zeros_like(ang, dtype=torch.bool)
    if dt == torch.bfloat16:
        for f in (ang.cos(), ang.sin()):
            low = f.view(torch.int32) & 0xFFFF
            mask |= (low - 0x8000).abs() <= 2
    return mask


def _compare(got, ref, dt, near, what):
    if dt == torch.float32:
        assert rel_err(got, ref) <= 1e-4, (what, rel_err(got, ref))
        return
    diff = got.float() != ref.float()
    if diff.any():
        bad = diff & ~near
        assert not bad.any(), (what, int(bad.sum()), int(diff.sum()))
        d = (got.float() - ref.float()).abs()[diff]
        ulp = (ref.float().abs()[diff] * 2 ** -7).clamp_min(2 ** -133)
        assert bool((d <= 2 * ulp).all()), what


@pytest.mark.parametrize("dt,hd,theta", CASES)
@pytest.mark.parametrize("pos0", [8192, 32768, 65408])
def test_heads_rope_at_large_positions(dt, hd, theta, pos0, gpu):
    print(f"[case] heads rope {dt} head_dim={hd} theta={theta:g} pos0={pos0}", flush=True)
    mod = _module(hd, theta, dt)
    p = O.Bolt3Params.from_module(mod)
    B, T = 2, 128
    x = recipes.hidden(4, B, T, 256).to(dt)
    q_raw, k_raw, v, beta, eta = O.project(p, x)
    pos = torch.arange(pos0, pos0 + T, dtype=torch.float32)
    mod = mod.to(gpu)
    W, bias, side = mod._packed(dt, gpu)
    lin = F.linear(x.to(gpu), W, bias)
    H, HKV = mod.H, mod.HKV
    out = {n: torch.empty(B, h, T, hd, dtype=dt, device=gpu) for n, h in
           (("q_raw", H), ("q_rope", H), ("k_raw", HKV), ("k_rope", HKV), ("v", HKV))}
    b_o, e_o = torch.empty(B, HKV, T, device=gpu), torch.empty(B, H, T, device=gpu)
    mod._heads(lin, B, T, dt, side, pos0, out["q_raw"], out["q_rope"], out["k_raw"], out["k_rope"], out["v"],
               b_o, e_o)
    torch.cuda.synchronize()
    near = _near_boundary(pos, p.inv_freq, dt)[None, None]
    # the projections differ from the CPU's by summation order; RoPE itself is checked on the
    # kernel's own un-roped heads, the heads against the oracle's to the output tolerance
    q_g, k_g = out["q_raw"].cpu(), out["k_raw"].cpu()
    for got, ref, what in ((q_g, q_raw, "q_raw"), (k_g, k_raw, "k_raw")):
        if dt == torch.float32:
            assert rel_err(got, ref) <= 1e-4, what
        else:
            assert (got.float() - ref.float()).abs().max() <= 2e-2, what
    q_ref, k_ref = O.rope_at(q_g, pos, p.inv_freq), O.rope_at(k_g, pos, p.inv_freq)
    _compare(out["q_rope"].cpu(), q_ref, dt, near.expand_as(q_ref), "q_rope")
    _compare(out["k_rope"].cpu(), k_ref, dt, near.expand_as(k_ref), "k_rope")


@pytest.mark.parametrize("dt,hd,theta", CASES)
def test_slot_keys_at_fractional_positions(dt, hd, theta, gpu):
    """Slot keys roped at mean positions (fractional, up to 65535), as the chain and the decode
    step read them."""
    from bolt3_amd import _abi as A
    print(f"[case] slot keys {dt} head_dim={hd}", flush=True)
    mod = _module(hd, theta, dt)
    p = O.Bolt3Params.from_module(mod)
    b, bh, S = 2, 2 * mod.HKV, 128
    g = torch.Generator().manual_seed(1)
    st = O.SlotState.empty(bh, S, hd, dt)
    st.ak = torch.randn(bh, S, hd, generator=g).to(dt)
    st.pm = (65535.0 - torch.rand(bh, S, generator=g) * 600.0).float()
    st.mass = 1.0 + torch.rand(bh, S, generator=g) * 5
    st.act = torch.rand(bh, S, generator=g) > 0.1
    ref_k, ref_b = O.slot_keys(p, st, b), O.slot_bias(p, st, b)
    dev = lambda t: t.to(gpu).contiguous()
    ak, pm, mass, act = dev(st.ak), dev(st.pm), dev(st.mass), dev(st.act.to(torch.uint8))
    kap, invf = dev(p.kappa.float()), dev(p.inv_freq.float())
    sk, sb = torch.empty_like(ak), torch.empty(bh, S, device=gpu)
    a = A.SlotKeysArgs()
    a.dtype, a.B, a.HKV, a.HD, a.S = A.dtype_code(dt), b, mod.HKV, hd, S
    a.ak, a.pm, a.mass, a.act = ak.data_ptr(), pm.data_ptr(), mass.data_ptr(), act.data_ptr()
    a.kappa, a.inv_freq, a.slot_k, a.slot_bias = kap.data_ptr(), invf.data_ptr(), sk.data_ptr(), sb.data_ptr()
    A.call("bolt3_slot_keys", a, gpu)
    torch.cuda.synchronize()
    near = torch.stack([_near_boundary(st.pm[r], p.inv_freq, dt) for r in range(bh)])
    _compare(sk.cpu(), ref_k, dt, near, "slot keys")
    fin = torch.isfinite(ref_b)
    assert torch.equal(torch.isfinite(sb.cpu()), fin)
    assert rel_err(sb.cpu()[fin], ref_b[fin]) <= 1e-6
