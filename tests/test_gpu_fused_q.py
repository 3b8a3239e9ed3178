"""The bf16 forward without a trace prepares the query heads (q RMSNorm, RoPE, the eta gate)
inside the attention kernel from the q projection output (b3_attn_args.q_lin, with the (cos, sin)
table b3_heads_args.rope_cs).  Its output must equal, bit for bit, that of the same forward with
the head preparation as a pass of its own (bolt3_heads, whose outputs the parity tests check
against the oracle): every attention kernel shape (one, two, four and eight query heads per kv
head), head_dim 64 and 128, with and without the q/k norm, biased projections, a partial last
chunk.  The forward also stays within the bf16 bar of the oracle."""
from __future__ import annotations

import pytest
import torch

import recipes
from helpers import cosine, max_abs
from oracle import bolt3_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,HKV,HD,qk_norm,bias", [
    (16, 4, 128, True, False),    # four query heads per kv head: two workgroups per compute unit
    (8, 8, 64, False, False),     # one, no q/k norm
    (8, 1, 128, True, True),      # eight, biased projections
    (4, 2, 64, True, False),      # two
])
def test_fused_query_preparation_is_exact(H, HKV, HD, qk_norm, bias, gpu):
    from bolt3_amd import Bolt3Attn
    from bolt3_amd import bolt3 as B3
    cfg = dict(dim=256, num_heads=H, num_kv_heads=HKV, head_dim=HD, rope_theta=1e6, eps=1e-6, qk_norm=qk_norm,
               qkv_bias=bias)
    print(f"[case] fused q preparation H={H} HKV={HKV} HD={HD} qk_norm={qk_norm} bias={bias} T=700", flush=True)
    bf = torch.bfloat16
    mod = recipes.init_module(Bolt3Attn(cfg), 17, nondefault=True).to(bf)
    x = recipes.hidden(17, 2, 700, cfg["dim"]).to(bf)
    mod_d = mod.to(gpu)
    with torch.no_grad():
        assert B3.FUSED_Q_PREP
        y_fused = mod_d(x.to(gpu))
        B3.FUSED_Q_PREP = False
        try:
            y_plain = mod_d(x.to(gpu))
        finally:
            B3.FUSED_Q_PREP = True
    torch.cuda.synchronize()
    assert torch.isfinite(y_fused).all()
    assert torch.equal(y_fused, y_plain), float((y_fused.float() - y_plain.float()).abs().max())
    with torch.no_grad():
        ref = O.forward(O.Bolt3Params.from_module(mod.cpu()), x, ties="torch")
    ma, cs = max_abs(y_fused.cpu(), ref), cosine(y_fused.cpu(), ref)
    assert ma <= 2e-2 and cs >= 0.9995, (ma, cs)
