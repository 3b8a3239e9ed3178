"""The fused one-token decode layer step (bolt3_decode_layer) on the GPU, Qwen3-4B layer shape.

* Its two projections against a plain fp32 torch product of the same bf16 operands: every
  element within one bf16 rounding (2^-8 relative) plus an fp32 summation allowance.  The
  input projection is seen through the new token's value row, which the step appends to the
  window ring as projected (values are not normalised); o_proj through the step's output.
* The whole step against the unfused step (torch projections around bolt3_decode) run on an
  identically prefilled state: bf16 bar, max-abs <= 2e-2 and cosine >= 0.9995.
Batches 64 (the decode benchmark), 5 (a partial row tile) and 70 (two row blocks).
"""
from __future__ import annotations

import pytest
import torch

from helpers import cosine, max_abs

pytestmark = pytest.mark.gpu

CFG = dict(dim=2560, num_heads=32, num_kv_heads=8, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)


def _proj_ok(got, x, w, b, what):
    ref = x.float() @ w.float().t()
    if b is not None:
        ref = ref + b.float()
    err = (got.float() - ref).abs()
    bound = ref.abs() * 2.0 ** -8 + 1e-3
    bad = int((err > bound).sum())
    assert bad == 0, f"{what}: {bad} elements beyond one bf16 rounding (max err {float(err.max()):.3e})"


@pytest.mark.parametrize("B", [64, 5, 70])
def test_decode_layer_vs_unfused_and_fp32_projections(B, gpu):
    from bolt3_amd import Bolt3Attn, Bolt3Decoder, Bolt3LayerState, HybridLM
    import recipes
    bf = torch.bfloat16
    print(f"[case] decode_layer B={B}", flush=True)
    mod = recipes.init_module(Bolt3Attn(CFG), 3, nondefault=True).to(bf).to(gpu)
    model = HybridLM(vocab_size=8, dim=CFG["dim"], num_layers=0, num_heads=32, num_kv_heads=8, intermediate=8,
                     layer_types=[]).to(gpu)
    fused, plain = Bolt3Decoder(model), Bolt3Decoder(model)
    plain.fuse_projections = False
    g = torch.Generator(device=gpu).manual_seed(5)
    sa, sb = Bolt3LayerState(mod, B, gpu, bf), Bolt3LayerState(mod, B, gpu, bf)
    ma, mb = torch.zeros(B, 8, 128, 128, device=gpu), torch.zeros(B, 8, 128, 128, device=gpu)
    W, bias, side = mod._packed(bf, gpu)
    with torch.no_grad():
        for c in range(4):
            h = torch.randn(B, mod.C, CFG["dim"], generator=g, device=gpu).to(bf)
            fused._bolt3_layer(mod, h, c * mod.C, ma, sa)
            plain._bolt3_layer(mod, h, c * mod.C, mb, sb)
        assert sa.has_slots and sa.n_sink > 0
        for i in range(3):
            pos = 4 * mod.C + i
            h = torch.randn(B, 1, CFG["dim"], generator=g, device=gpu).to(bf)
            ni = sa.cur[0] + sa.cur[1]   # ring index the new token goes to
            out_a = fused._bolt3_layer(mod, h, pos, ma, sa)
            _, _, _, y, _, _, _, _ = sa._dec
            torch.cuda.synchronize()
            v0 = (mod.H + mod.HKV) * mod.HD      # value columns of the packed projection
            v_rows = sa.win_v[:, :, ni].reshape(B, -1)
            _proj_ok(v_rows, h.view(B, -1), W[v0:v0 + mod.HKV * mod.HD],
                     None if bias is None else bias[v0:v0 + mod.HKV * mod.HD], f"input projection, step {i}")
            _proj_ok(out_a.view(B, -1), y, side["wo"], None, f"o_proj, step {i}")
            out_b = plain._bolt3_layer(mod, h, pos, mb, sb)
            ma_, cs = max_abs(out_a.float().cpu(), out_b.float().cpu()), cosine(out_a.float().cpu(), out_b.float().cpu())
            assert ma_ <= 2e-2 and cs >= 0.9995, f"step {i}: fused vs unfused max-abs {ma_:.3e} cos {cs:.6f}"
