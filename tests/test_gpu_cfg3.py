"""The decode configuration's layer under check: Qwen3-4B layer shape (hidden 2560, 32 / 8
heads, head_dim 128, theta 1e6, q/k norm), bf16, B = 64 sequences, the real 8192-token prefill
(64 chunks, 63 consolidations over all 512 (batch, kv-head) rows), then 130 single-token steps
through the fused bf16 layer step (a steady consolidation at step 128).  The gates' projections,
kappa and gamma are drawn (eta != 0, so the M_res readout reaches the output) and res_norm keeps
the reference's initial 0.05.  Everything against the
oracle's layer_step (the reference's decoder semantics) forced onto the kernel's decisions: the
prefill output chunk by chunk, every step's output (bf16 tolerance: max-abs 2e-2, or two bf16
ulps where the value's magnitude makes that larger, and cosine 0.9995), every consolidation's
decisions against the oracle's own from the same state (bit-exact except
near-ties within 1e-4, counted), and the end state."""
import copy

import pytest
import torch

import recipes
from helpers import bf16_check, decisions_from_kernel_log
from oracle import bolt3_oracle as O
from test_gpu_parity import _check_state, _compare_step

pytestmark = pytest.mark.gpu


def test_cfg3_prefill_8192_and_decode_steps(gpu):
    from bolt3_amd import Bolt3Attn, Bolt3Decoder, Bolt3LayerState, HybridLM
    B, D, C, T0, n_dec = 64, 2560, 128, 8192, 130
    cfg = dict(dim=D, num_heads=32, num_kv_heads=8, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)
    mod = recipes.init_module(Bolt3Attn(cfg), 41, nondefault=True)
    with torch.no_grad():     # drawn gates, kappa and gamma; res_norm at the reference's 0.05
        mod.res_norm.weight.fill_(0.05)
    mod = mod.to(torch.bfloat16)
    p = O.Bolt3Params.from_module(mod)
    g = torch.Generator().manual_seed(41)
    xs = torch.empty(B, T0 + n_dec, D, dtype=torch.bfloat16)
    for r in range(B):
        xs[r] = torch.randn(T0 + n_dec, D, generator=g).to(torch.bfloat16)
    print(f"[case] cfg3 layer: B={B}, prefill {T0}, {n_dec} steps", flush=True)
    # the HIP path: the decoder's prefill, then single-token steps
    dmod = copy.deepcopy(mod).to(gpu)
    model = HybridLM(vocab_size=8, dim=D, num_layers=0, num_heads=32, num_kv_heads=8, intermediate=8,
                     layer_types=[]).to(gpu)
    dec = Bolt3Decoder(model)
    st = Bolt3LayerState(dmod, B, gpu, torch.bfloat16)
    m = torch.zeros(B, 8, 128, 128, device=gpu)
    rec = []
    xd = xs.to(gpu)
    with torch.no_grad():
        out_pre = dec._bolt3_prefill(dmod, xd[:, :T0], m, st, rec).cpu()
        n_pre = len(rec)
        outs = [dec._bolt3_layer(dmod, xd[:, T0 + i:T0 + i + 1], T0 + i, m, st, rec).cpu() for i in range(n_dec)]
    del xd
    print(f"[case] cfg3 HIP path done: {n_pre} consolidations in the prefill, {len(rec) - n_pre} in the steps",
          flush=True)
    assert n_pre == T0 // C - 1 and len(rec) == n_pre + 1
    # the oracle along the kernel's decisions
    forced = iter([decisions_from_kernel_log(e["log"]) for e in rec])
    cache, m_r = O.LayerCache(), torch.zeros(B, 8, 128, 128)
    logs = []
    worst = (0.0, 1.0)
    with torch.no_grad():
        for c in range(T0 // C):
            _, out, m_r = O.layer_step(p, xs[:, c * C:(c + 1) * C], c * C, m_r, cache, log=logs,
                                       force=lambda: next(forced))
            got = out_pre[:, c * C:(c + 1) * C]
            ok, ma, ratio, cs = bf16_check(got, out)
            worst = (max(worst[0], ma), min(worst[1], cs))
            assert ok, ("prefill chunk", c, ma, ratio, cs)
        print(f"[case] cfg3 prefill output vs forced oracle, worst chunk: max-abs {worst[0]:.3e} cos {worst[1]:.6f}",
              flush=True)
        for i in range(n_dec):
            pos = T0 + i
            _, out, m_r = O.layer_step(p, xs[:, pos:pos + 1], pos, m_r, cache, log=logs, force=lambda: next(forced))
            ok, ma, ratio, cs = bf16_check(outs[i], out)
            assert ok, ("step", i, ma, ratio, cs)
    mism = near = ties = rnd = 0
    for e, (gl, lg) in enumerate(zip(rec, logs)):
        a, b, t, d = _compare_step(lg, gl["log"].cpu(), B * 8, gl["tokens"], f"cfg3 event {e}", bf16=True)
        mism, near, ties, rnd = mism + a, near + b, ties + t, rnd + d
    print(f"[decisions] cfg3: events={len(rec)} x {B * 8} rows mismatches={mism} near-ties={near} "
          f"rounding divergences={rnd} rows ordered on exact ties={ties}", flush=True)
    assert mism == 0 and rnd <= len(rec) * B * 8 // 1000 and len(logs) == len(rec)
    # M_res after 61 steady delta-rule steps (products of fp32 operands split into bf16 hi + lo keep
    # about 16 bits each step, and gamma ~ 0.9 carries each step's rounding into the next ones)
    _check_state(st, m.view(B * 8, 128, 128), cache.st, torch.bfloat16, "cfg3 end state vs forced oracle",
                 m_tol=2e-3)
    assert st.n_filled == cache.st.n_filled == 128
