"""The decode configuration's layer under check: Qwen3-4B layer shape (hidden 2560, 32 / 8
heads, head_dim 128, theta 1e6, q/k norm), bf16, B = 64 sequences, three chunks of prefill
(the slots fill), then 130 single-token steps through the fused bf16 layer step, so that a
steady consolidation over all 512 (batch, kv-head) rows runs at step 128.  Every step's output
against the oracle's layer_step (bf16 tolerance: max-abs 2e-2, cosine 0.9995) up to the first
near-tie of the trajectory; that consolidation's decisions teacher-forced from the oracle's
state (bit-exact except near-ties within 1e-4, counted)."""
import copy

import pytest
import torch

import recipes
from helpers import cosine, max_abs
from oracle import bolt3_oracle as O
from test_gpu_parity import _compare_step, _gpu_step

pytestmark = pytest.mark.gpu


def test_cfg3_layer_steps_and_consolidation(gpu):
    from bolt3_amd import Bolt3Attn, Bolt3Decoder, Bolt3LayerState, HybridLM
    B, D, C = 64, 2560, 128
    cfg = dict(dim=D, num_heads=32, num_kv_heads=8, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)
    mod = recipes.init_module(Bolt3Attn(cfg), 41, nondefault=True).to(torch.bfloat16)
    p = O.Bolt3Params.from_module(mod)
    g = torch.Generator().manual_seed(41)
    xs = (torch.randn(B, 3 * C + 130, D, generator=g)).to(torch.bfloat16)
    print("[case] cfg3 layer: B=64, prefill 384, 130 steps", flush=True)
    # oracle trajectory, keeping the input of the steady consolidation at step 127
    cache, m_r = O.LayerCache(), torch.zeros(B, 8, 128, 128)
    outs_r, logs_r = [], []
    with torch.no_grad():
        for c in range(3):
            _, out, m_r = O.layer_step(p, xs[:, c * C:(c + 1) * C], c * C, m_r, cache, log=logs_r)
        for i in range(130):
            pos = 3 * C + i
            if i == C - 1:
                forced = (cache.st.clone(), m_r.clone(), cache.prev)
            _, out, m_r = O.layer_step(p, xs[:, pos:pos + 1], pos, m_r, cache, log=logs_r)
            outs_r.append(out)
    assert [lg["kind"] for lg in logs_r] == ["fill", "fill", "steady"]
    # the HIP path on the same inputs
    dmod = copy.deepcopy(mod).to(gpu)
    model = HybridLM(vocab_size=8, dim=D, num_layers=0, num_heads=32, num_kv_heads=8, intermediate=8,
                     layer_types=[]).to(gpu)
    dec = Bolt3Decoder(model)
    st = Bolt3LayerState(dmod, B, gpu, torch.bfloat16)
    m = torch.zeros(B, 8, 128, 128, device=gpu)
    rec = []
    xd = xs.to(gpu)
    near = mism = 0
    with torch.no_grad():
        for c in range(3):
            dec._bolt3_layer(dmod, xd[:, c * C:(c + 1) * C], c * C, m, st, rec)
        for i in range(130):
            pos = 3 * C + i
            out = dec._bolt3_layer(dmod, xd[:, pos:pos + 1], pos, m, st, rec).cpu()
            ma, cs = max_abs(out, outs_r[i]), cosine(out, outs_r[i])
            assert ma <= 2e-2 and cs >= 0.9995, (i, ma, cs)
        for e, (gl, lg) in enumerate(zip(rec, logs_r)):
            a, b, _ = _compare_step(lg, gl["log"].cpu(), B * 8, gl["tokens"], f"cfg3 event {e}")
            mism, near = mism + a, near + b
            if b:
                break
    print(f"[decisions] cfg3 trajectory: events={len(rec)} mismatches={mism} near-ties={near}", flush=True)
    assert mism == 0 and len(rec) == 3
    # the steady consolidation (512 rows) from the oracle's exact state
    st_in, m_in, prev = forced
    kr, kp, v, pos_t, beta = prev
    bh, n = B * 8, kr.shape[2]
    st_in.m_res = m_in.reshape(bh, 128, 128).clone()
    chunk = (kr.reshape(bh, n, 128), kp.reshape(bh, n, 128), v.reshape(bh, n, 128), pos_t.reshape(n),
             beta.reshape(bh, n))
    gam = O.gamma_delta(p.log_gamma)
    lg = {}
    ref = O.consolidate(p, st_in, *chunk, gam, B, log=lg)
    st_g, m_g, log = _gpu_step(dmod, st_in, chunk, gam, B, gpu)
    a, b, t = _compare_step(lg, log, bh, n, "cfg3 forced")
    print(f"[decisions] cfg3 steady consolidation, {bh} rows teacher-forced: mismatches={a} near-ties={b} "
          f"rows ordered on exact ties={t}", flush=True)
    assert a == 0
    if b == 0:
        assert torch.equal(st_g["act"].bool(), ref.act) and torch.equal(st_g["mass"], ref.mass)
        assert float((m_g - ref.m_res).norm() / ref.m_res.norm()) <= 1e-3
