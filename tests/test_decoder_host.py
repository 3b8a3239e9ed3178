"""Host-side decoder pieces on the CPU: the anchor cache, the device-resident generation
bookkeeping, sampling and the state-size count (no kernel calls)."""
import random

import torch

from bolt3_amd import AnchorCache, Bolt3Decoder, HybridLM, sample_tokens
from bolt3_amd.decoder import _Bookkeeping


def test_anchor_cache_append_and_grow():
    """append returns the cached prefix, like concatenation (vsa_lm/decode.py:94-106), across
    page growth."""
    c = AnchorCache(2, 3, 100, 8, "cpu", dt=torch.float32)
    assert c.capacity == 256
    ks, vs = [], []
    for t in (1, 7, 128, 200, 1, 300):
        k, v = torch.randn(2, 3, t, 8), torch.randn(2, 3, t, 8)
        ks.append(k)
        vs.append(v)
        kk, vv = c.append(k, v)
        assert torch.equal(kk, torch.cat(ks, dim=2)) and torch.equal(vv, torch.cat(vs, dim=2))
    assert c.n == 637 and c.capacity % AnchorCache.PAGE == 0 and c.capacity >= 637


def _rules(stream, eos, close, n_max):
    """The reference's per-row rules (vsa_lm/config/bolt3.py:469-494) as a plain loop."""
    B = len(stream[0])
    done, closed, lengths, cur = [False] * B, [False] * B, [n_max] * B, [-1] * B
    budget = max(64, n_max - 64)
    out = []
    for i in range(n_max):
        nxt = list(stream[i])
        if close:
            if i == budget:
                for r in range(B):
                    if not closed[r] and not done[r] and cur[r] < 0:
                        cur[r] = 0
            for r in range(B):
                if cur[r] >= 0:
                    nxt[r] = close[cur[r]]
                    cur[r] += 1
                    if cur[r] >= len(close):
                        cur[r], closed[r] = -1, True
            if len(close) > 1:
                for r in range(B):
                    closed[r] = closed[r] or nxt[r] == close[1]
        out.append(nxt)
        for r in range(B):
            if eos and not done[r] and nxt[r] in eos:
                lengths[r], done[r] = i + 1, True
    return out, lengths, closed


def test_bookkeeping_matches_reference_rules():
    rng = random.Random(3)
    for trial in range(40):
        B, n_max = rng.randint(1, 6), rng.choice([10, 65, 100, 130, 200])
        vocab = rng.choice([6, 12, 40])
        stream = [[rng.randrange(vocab) for _ in range(B)] for _ in range(n_max)]
        eos = set(rng.sample(range(vocab), rng.randint(0, 2)))
        close = rng.sample(range(vocab), rng.randint(0, 3))
        book = _Bookkeeping(B, n_max, eos, close, "cpu")
        for i in range(n_max):
            book.take(i, torch.tensor(stream[i]).view(B, 1))
        want, lengths, closed = _rules(stream, eos, close, n_max)
        assert book.toks.T.tolist() == want, trial
        assert book.lengths.tolist() == lengths, trial
        assert book.closed.tolist() == closed, trial


def test_sampling_limits():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(5, 50, generator=g)
    top = logits.argmax(-1, keepdim=True)
    assert torch.equal(sample_tokens(logits, 0.0), top)
    assert torch.equal(sample_tokens(logits, 0.7, top_k=1, top_p=1.0), top)
    assert torch.equal(sample_tokens(logits, 0.7, top_p=0.0), top)     # only the top token has no mass ahead
    s = sample_tokens(logits, 1.0, top_k=5, top_p=1.0)
    assert s.shape == (5, 1) and all(int(t) in logits[r].topk(5).indices.tolist() for r, t in enumerate(s[:, 0]))


def test_state_bytes_counts():
    """Fixed bytes: M_res fp32 + slot keys/values + a two-chunk window, 2 bytes a value, per Bolt-3
    layer; per-token bytes: keys and values of every anchor (vsa_lm/config/bolt3.py:290-300)."""
    m = HybridLM(vocab_size=16, dim=64, num_layers=4, num_heads=4, num_kv_heads=2, intermediate=32, head_dim=32,
                 layer_types=["vsa", "vsa", "softmax", "vsa"])
    fixed, per_tok = Bolt3Decoder.state_bytes(m)
    hkv, hd, S, C = 2, 32, 128, 128
    assert fixed == 3 * (hkv * hd * hd * 4 + 2 * S * hkv * hd * 2 + 4 * C * hkv * hd * 2)
    assert per_tok == 1 * (2 * hkv * hd * 2)


def test_serve_dispatch():
    """make_decoder gives a Bolt3Decoder for stacks with a Bolt-3 layer and None otherwise
    (the reference server builds VSARecurrentDecoder for everything, vsa_lm/server.py:141,159)."""
    from bolt3_amd.serve import is_bolt3_model, make_decoder
    hyb = HybridLM(vocab_size=16, dim=64, num_layers=2, num_heads=4, num_kv_heads=2, intermediate=32, head_dim=32,
                   layer_types=["vsa", "softmax"])
    soft = HybridLM(vocab_size=16, dim=64, num_layers=1, num_heads=4, num_kv_heads=2, intermediate=32, head_dim=32,
                    layer_types=["softmax"])
    assert is_bolt3_model(hyb) and not is_bolt3_model(soft) and not is_bolt3_model(torch.nn.Linear(2, 2))
    dec = make_decoder(hyb)
    assert isinstance(dec, Bolt3Decoder) and dec.max_cache_pos == 8192 and dec.wrap_positions is False
    assert make_decoder(hyb, "cuda:0").max_cache_pos == 65536
    assert make_decoder(soft) is None
