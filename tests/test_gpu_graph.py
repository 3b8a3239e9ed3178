"""The graph-captured one-token step (DecodeGraph) against the eager step, and the anchor
layers' fused HIP step against the oracle.  A graph replays the same kernels on the same
inputs, so every replay must equal the eager step bit for bit; the replays are interleaved with
unrelated eager work and cross two consolidations (the descriptors rewritten from the host)."""
import copy

import pytest
import torch

import recipes
from helpers import cosine, rel_err
from oracle import bolt3_oracle as O

pytestmark = pytest.mark.gpu


def _model(seed, layer_types, dim=256, heads=(4, 2), head_dim=64, vocab=512):
    from bolt3_amd import HybridLM
    m = HybridLM(vocab_size=vocab, dim=dim, num_layers=len(layer_types), num_heads=heads[0], num_kv_heads=heads[1],
                 intermediate=256, layer_types=layer_types, head_dim=head_dim, qk_norm=True, rope_theta=1e6, eps=1e-6)
    m.load_state_dict(recipes.model_params([(k, tuple(v.shape)) for k, v in m.state_dict().items()], seed),
                      strict=False)
    for li, blk in enumerate(m.blocks):
        if hasattr(blk, "vsa"):
            recipes.init_module(blk.vsa, seed + li, nondefault=True)
    return m.to(torch.bfloat16).eval()


@pytest.mark.parametrize("head_dim", [64, 128])
def test_graph_replay_equals_eager(head_dim, gpu):
    from bolt3_amd import Bolt3Decoder
    print(f"[case] graph vs eager head_dim={head_dim}", flush=True)
    model = _model(21, ["vsa", "softmax", "vsa"], head_dim=head_dim).to(gpu)
    dec_e, dec_g = Bolt3Decoder(model), Bolt3Decoder(model)
    ids = recipes.tokens(21, 3, 300 + 240, 512).to(gpu)
    with torch.no_grad():
        h_e, st_e, kv_e = dec_e.prefill(ids[:, :300])
        h_g, st_g, kv_g = dec_g.prefill(ids[:, :300])
        graph = dec_g._graph_runner(3, 600, gpu, st_g, kv_g, 300)
        assert graph is not None
        noise = torch.randn(1 << 20, device=gpu)
        for i in range(240):                    # consolidations at positions 384 and 512
            pos = 300 + i
            tok = ids[:, pos:pos + 1]
            h, _, _ = dec_e.step(tok, pos, st_e, kv_e)
            want = model.lm_head(h[:, -1])
            got = graph.step(tok).clone()
            noise.mul_(0.5).add_(1.0)           # unrelated eager work between replays
            assert torch.equal(got, want), (i, rel_err(got.float().cpu(), want.float().cpu()))
        for li in (0, 2):
            assert torch.equal(st_e[li], st_g[li])
            assert kv_e[li].prev == kv_g[li].prev and kv_e[li].cur == kv_g[li].cur
            assert torch.equal(kv_e[li]["ak"], kv_g[li]["ak"]) and torch.equal(kv_e[li]["mass"], kv_g[li]["mass"])
        assert kv_e[1].n == kv_g[1].n == 540


def test_generate_with_and_without_graph(gpu):
    from bolt3_amd import Bolt3Decoder
    model = _model(22, ["vsa", "vsa", "softmax"]).to(gpu)
    ids = recipes.tokens(22, 2, 260, 512).to(gpu)
    dec = Bolt3Decoder(model)
    with torch.no_grad():
        t_g, n_g = dec.generate_batch(ids, 150, temperature=0.0, eos_ids={7})
        dec.use_graphs = False
        t_e, n_e = dec.generate_batch(ids, 150, temperature=0.0, eos_ids={7})
    assert torch.equal(t_g, t_e) and torch.equal(n_g, n_e)


@pytest.mark.parametrize("head_dim,heads", [(64, (4, 2)), (128, (8, 1)), (128, (8, 8))])
def test_anchor_fused_step_vs_oracle(head_dim, heads, gpu):
    """Single-token steps of a softmax-anchor layer (fused HIP step: projections, q/k norm, RoPE,
    append, causal softmax over the cache, o_proj) against the oracle's StaticKV + SDPA, every step,
    from a 300-token prefill up to 2300 cached keys (beyond the Bolt-3 window's key count)."""
    from bolt3_amd import Bolt3Decoder
    print(f"[case] anchor fused step head_dim={head_dim} heads={heads}", flush=True)
    model = _model(23, ["softmax"], head_dim=head_dim, heads=heads)
    ref = O.HybridRef(model)
    dec = Bolt3Decoder(copy.deepcopy(model).to(gpu))
    ids = recipes.tokens(23, 2, 2300, 512)
    with torch.no_grad():
        _, st_r = ref.prefill(ids[:, :2000])
        _, states, kv = dec.prefill(ids[:, :2000].to(gpu))
        for i in range(300):
            pos = 2000 + i
            hr = ref.step(ids[:, pos:pos + 1], pos, st_r)
            h, states, kv = dec.step(ids[:, pos:pos + 1].to(gpu), pos, states, kv)
            hc, hr = h.float().cpu(), hr.float()
            assert rel_err(hc, hr) <= 1e-2 and cosine(hc, hr) >= 0.9995, (i, rel_err(hc, hr), cosine(hc, hr))
    assert kv[0].n == 2300
