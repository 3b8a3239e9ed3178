"""The end-to-end configuration under check: the full Qwen3-4B-shape hybrid
stack (36 layers, every 4th a softmax anchor: 27 Bolt-3 + 9 anchors, hidden 2560, SwiGLU 9728,
vocabulary 151936, random bf16 weights, Bolt-3 parameters at the reference's defaults), B=32,
a 2048-token prompt of uniform-random ids.

  * Layer taps: the inputs of three Bolt-3 layers (the first, one in the middle, the last but
    one) are captured during the decoder's prefill.  On two batch rows the oracle's decoder
    step (the reference's semantics), run chunk by chunk on those inputs and forced onto the
    kernel's decisions, gives every chunk's output and the layer's end state; every
    consolidation's decisions equal the oracle's own from the same state (near-ties counted).
  * Property checks: 130 greedy steps (a consolidation in every Bolt-3 layer at step 128) of
    the graph-captured step against the eager step from the same state, bit for bit, with
    finite logits."""
import pytest
import torch

import recipes
from helpers import bf16_check, decisions_from_kernel_log
from oracle import bolt3_oracle as O
from test_gpu_parity import _check_state, _compare_step

pytestmark = pytest.mark.gpu

TAPS = (0, 13, 34)
ROWS = 2


def _clone_state(model, states, kv, B, capacity, dev):
    """An independent copy of a decode state (Bolt-3 layers through the reference's dict form)."""
    from bolt3_amd import AnchorCache, Bolt3LayerState
    st2, kv2 = [], []
    for li, blk in enumerate(model.blocks):
        st2.append(None if states[li] is None else states[li].clone())
        if hasattr(blk, "vsa"):
            kv2.append(Bolt3LayerState.from_dict(blk.vsa, kv[li].to_dict(), device=dev))
        else:
            c = kv[li]
            cache = AnchorCache(B, c.k.shape[1], capacity, c.k.shape[3], dev, dt=c.k.dtype)
            cache.append(c.k[:, :, :c.n], c.v[:, :, :c.n])
            kv2.append(cache)
    return st2, kv2


def test_cfg5_hybrid_stack(gpu):
    import bench
    from bolt3_amd import Bolt3Decoder
    B, T, n_steps, C = 32, 2048, 130, 128
    print(f"[case] cfg5: 36 layers, B={B}, prompt {T}, {n_steps} greedy steps", flush=True)
    m = bench.build_e2e(gpu)
    assert sum(hasattr(b, "vsa") for b in m.blocks) == 27 and all(hasattr(m.blocks[li], "vsa") for li in TAPS)
    ids = recipes.tokens(bench.SEED + 4, B, T, m.config["vocab_size"]).to(gpu)
    dec = Bolt3Decoder(m)
    index = {id(blk.vsa): li for li, blk in enumerate(m.blocks) if hasattr(blk, "vsa")}
    taps = {}
    prefill_layer = dec._bolt3_prefill

    def tapped(ly, h, m_state, st, record=None):
        li = index[id(ly)]
        if li not in TAPS:
            return prefill_layer(ly, h, m_state, st, record)
        rec = []
        out = prefill_layer(ly, h, m_state, st, rec)
        rows = ROWS * ly.HKV
        taps[li] = dict(h=h[:ROWS].cpu(), out=out[:ROWS].cpu(),
                        rec=[dict(log=e["log"][:rows].cpu(), tokens=e["tokens"]) for e in rec],
                        state={k: st[k][:rows].cpu() for k in ("ak", "av", "mass", "util", "pm", "act")},
                        m_res=m_state[:ROWS].cpu())
        return out

    dec._bolt3_prefill = tapped
    with torch.no_grad():
        h, states, kv = dec.prefill(ids)
    assert set(taps) == set(TAPS)
    print("[case] cfg5 prefill done; graph vs eager", flush=True)

    # graph-captured steps against eager steps from the same state
    cap = T + n_steps + 64
    st_g, kv_g = _clone_state(m, states, kv, B, cap, gpu)
    dec_g = Bolt3Decoder(m)
    with torch.no_grad():
        logits = m.lm_head(h[:, -1])
        graph = dec_g._graph_runner(B, cap, gpu, st_g, kv_g, T)
        assert graph is not None
        tok = logits.argmax(dim=-1, keepdim=True)
        for i in range(n_steps):
            h, _, _ = dec.step(tok, T + i, states, kv)
            want = m.lm_head(h[:, -1])
            got = graph.step(tok).clone()
            assert torch.isfinite(want).all(), i
            assert torch.equal(got, want), (i, float((got.float() - want.float()).abs().max()))
            tok = want.argmax(dim=-1, keepdim=True)
    for li, blk in enumerate(m.blocks):
        if hasattr(blk, "vsa"):
            assert torch.equal(states[li], st_g[li]) and kv[li].n_filled == kv_g[li].n_filled == 128
    print(f"[case] cfg5: {n_steps} graph steps equal the eager steps", flush=True)

    # the tapped layers against the oracle forced onto the kernel's decisions
    for li in TAPS:
        tp = taps[li]
        ly = m.blocks[li].vsa
        p = O.Bolt3Params.from_module(ly)
        forced = iter([decisions_from_kernel_log(e["log"]) for e in tp["rec"]])
        cache, m_r = O.LayerCache(), torch.zeros(ROWS, ly.HKV, ly.HD, ly.HD)
        logs = []
        worst = (0.0, 1.0)
        with torch.no_grad():
            for c in range(T // C):
                _, out, m_r = O.layer_step(p, tp["h"][:, c * C:(c + 1) * C], c * C, m_r, cache, log=logs,
                                           force=lambda: next(forced))
                got = tp["out"][:, c * C:(c + 1) * C]
                ok, ma, ratio, cs = bf16_check(got, out)
                worst = (max(worst[0], ma), min(worst[1], cs))
                assert ok, (li, c, ma, ratio, cs)
        mism = near = ties = rnd = 0
        for e, (gl, lg) in enumerate(zip(tp["rec"], logs)):
            a, b, t, d = _compare_step(lg, gl["log"], ROWS * ly.HKV, gl["tokens"], f"cfg5 layer {li} event {e}",
                                       bf16=True)
            mism, near, ties, rnd = mism + a, near + b, ties + t, rnd + d
        print(f"[decisions] cfg5 layer {li}: events={len(logs)} x {ROWS * ly.HKV} rows mismatches={mism} "
              f"near-ties={near} rounding divergences={rnd} rows ordered on exact ties={ties}; output worst chunk "
              f"max-abs {worst[0]:.3e} cos {worst[1]:.6f}", flush=True)
        assert mism == 0 and rnd == 0 and len(logs) == len(tp["rec"]) == T // C - 1
        _check_state(tp["state"], tp["m_res"].reshape(-1, ly.HD, ly.HD), cache.st, torch.bfloat16,
                     f"cfg5 layer {li} end state")
