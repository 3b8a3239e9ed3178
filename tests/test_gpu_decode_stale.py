"""Decode steps do not depend on memory outside the state's valid ranges.  The bf16 decode
attention reads its last key tile with the rows past the last key clamped to the new token's
ring (or cache) position, read before the token is written there; those rows carry zero
probability, but a zero times a NaN left in that memory is NaN.  Here every position of the
Bolt-3 window rings outside the live segments, and of the softmax layer's key/value cache past
its length, is filled with NaN after the prefill, and the steps that follow must give exactly the
outputs of the same steps on an untouched copy of the state."""
import pytest
import torch

import recipes
from test_gpu_graph import _model

pytestmark = pytest.mark.gpu


def _poison(kv):
    nan = float("nan")
    for st in kv:
        if hasattr(st, "win_v"):   # Bolt-3 layer: the window ring outside prev and cur
            live = torch.zeros(st.cap, dtype=torch.bool, device=st.win_v.device)
            for s0, n in (st.prev, st.cur):
                live[s0:s0 + n] = True
            dead = ~live
            for t in (st.win_kr, st.win_kp, st.win_v):
                t[:, :, dead] = nan
        else:                      # softmax layer: the cache past its length
            st.k[:, :, st.n:] = nan
            st.v[:, :, st.n:] = nan


@pytest.mark.parametrize("T", [100, 300])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_decode_ignores_stale_memory(T, head_dim, gpu):
    from bolt3_amd import Bolt3Decoder
    print(f"[case] decode after stale memory T={T} head_dim={head_dim}", flush=True)
    model = _model(31, ["vsa", "softmax", "vsa"], head_dim=head_dim).to(torch.bfloat16).to(gpu)
    dec = Bolt3Decoder(model)
    ids = recipes.tokens(31, 2, T + 6, 512).to(gpu)
    with torch.no_grad():
        _, st_a, kv_a = dec.prefill(ids[:, :T])
        _, st_b, kv_b = dec.prefill(ids[:, :T])
        _poison(kv_b)
        for i in range(6):
            tok = ids[:, T + i:T + i + 1]
            ha, _, _ = dec.step(tok, T + i, st_a, kv_a)
            hb, _, _ = dec.step(tok, T + i, st_b, kv_b)
            assert bool(torch.isfinite(hb).all()), i
            assert torch.equal(ha, hb), (i, float((ha.float() - hb.float()).abs().max()))
