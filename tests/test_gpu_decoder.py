"""Decoder API on the GPU against the oracle (the reference's decoder semantics on the CPU):
state round trip through the reference's kv_caches dict, memorize / forget, multi-token steps
in the middle of a chunk, and greedy generation with end-of-sequence and close-of-thinking
rules.  Tolerances as in test_gpu_parity: fp32 relative 1e-4; bf16 hidden states relative 1e-2
and cosine 0.9995."""
from __future__ import annotations

import copy
import io

import pytest
import torch

import recipes
from helpers import cosine, rel_err
from oracle import bolt3_oracle as O

pytestmark = pytest.mark.gpu


def _model(seed, layer_types, dim=64, heads=(4, 2), head_dim=64, inter=128, vocab=1024, dtype=torch.float32,
           theta=1e4, eps=1e-5, beta_off=False):
    from bolt3_amd import HybridLM
    m = HybridLM(vocab_size=vocab, dim=dim, num_layers=len(layer_types), num_heads=heads[0],
                 num_kv_heads=heads[1], intermediate=inter, layer_types=layer_types, head_dim=head_dim,
                 qk_norm=True, rope_theta=theta, eps=eps)
    m.load_state_dict(recipes.model_params([(k, tuple(v.shape)) for k, v in m.state_dict().items()], seed),
                      strict=False)
    for li, blk in enumerate(m.blocks):
        if hasattr(blk, "vsa"):
            recipes.init_module(blk.vsa, seed + li, nondefault=True)
            if beta_off:    # beta = sigmoid(-1e4) = 0: M_res only decays
                with torch.no_grad():
                    blk.vsa.beta_proj.weight.zero_()
                    blk.vsa.beta_proj.bias.fill_(-1e4)
    return m.to(dtype).eval()


def _close(a, b, dtype, what):
    if dtype == torch.float32:
        assert rel_err(a, b) <= 1e-4, (what, rel_err(a, b))
    else:
        assert rel_err(a, b) <= 1e-2 and cosine(a, b) >= 0.9995, (what, rel_err(a, b), cosine(a, b))


def _to_cpu(states, kv):
    """The decode state in the form the reference's memory bank saves (vsa_lm/memory_bank.py:57-68)."""
    from bolt3_amd import AnchorCache
    out_kv = []
    for c in kv:
        if isinstance(c, AnchorCache):
            out_kv.append((c.k[:, :, :c.n].cpu(), c.v[:, :, :c.n].cpu()))
        else:
            out_kv.append({k: (v.cpu() if torch.is_tensor(v) else v) for k, v in c.to_dict().items()})
    return [None if s is None else s.cpu() for s in states], out_kv


def _from_cpu(model, saved_states, saved_kv, dev, capacity):
    from bolt3_amd import AnchorCache, Bolt3LayerState
    states, kv = [], []
    for blk, s, c in zip(model.blocks, saved_states, saved_kv):
        states.append(None if s is None else s.to(dev).contiguous())
        if hasattr(blk, "vsa"):
            kv.append(Bolt3LayerState.from_dict(blk.vsa, c, device=dev))
        else:
            k, v = c
            cache = AnchorCache(k.shape[0], k.shape[1], capacity, k.shape[3], dev, dt=k.dtype)
            cache.append(k.to(dev), v.to(dev))
            kv.append(cache)
    return states, kv


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_state_round_trip_through_reference_dict(dtype, gpu):
    """Prefill, save the state as the reference's memory bank does (CPU dicts, torch.save), load it
    with weights_only=True, rebuild it and decode on: every step equals the uninterrupted run."""
    from bolt3_amd import Bolt3Decoder
    print(f"[case] state round trip {dtype}", flush=True)
    model = _model(5, ["vsa", "softmax"], dtype=dtype).to(gpu)
    dec = Bolt3Decoder(model)
    ids = recipes.tokens(5, 2, 300 + 150, 1024).to(gpu)
    with torch.no_grad():
        h, states, kv = dec.prefill(ids[:, :300])
        buf = io.BytesIO()
        s_cpu, kv_cpu = _to_cpu(states, kv)
        torch.save({"vsa_states": s_cpu, "kv_caches": kv_cpu}, buf)
        buf.seek(0)
        saved = torch.load(buf, weights_only=True)
        # the same anchor capacity: torch's attention may sum in another order for another row stride
        states2, kv2 = _from_cpu(model, saved["vsa_states"], saved["kv_caches"], gpu, kv[1].capacity)
        assert kv2[0].n_filled == kv[0].n_filled and kv2[0].prev[1] == kv[0].prev[1]
        for i in range(150):      # crosses a consolidation (at 384) with the rebuilt state
            pos = 300 + i
            h1, states, kv = dec.step(ids[:, pos:pos + 1], pos, states, kv)
            h2, states2, kv2 = dec.step(ids[:, pos:pos + 1], pos, states2, kv2)
            assert torch.equal(h1, h2), (i, rel_err(h1.float().cpu(), h2.float().cpu()))
    assert torch.equal(states[0], states2[0])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_state_setitem_rewrites_state(dtype, gpu):
    """Assigning a reference key rewrites that part (here: the slot masses) and the cached slot
    bias follows: kappa * log(max(mass, 1)) on active slots, after the prefill and after the
    assignment.  kappa is not 1 and differs per kv head; in bf16 the module's kappa and inv_freq
    are converted to fp32 for the rotation kernel, so a conversion freed before that kernel runs
    would show here as a wrong bias."""
    from bolt3_amd import Bolt3Decoder
    model = _model(6, ["vsa"], dtype=dtype)
    ly = model.blocks[0].vsa
    with torch.no_grad():
        ly.kappa.copy_(torch.tensor([0.75, 1.625]).to(ly.kappa.dtype))
    model = model.to(gpu)
    dec = Bolt3Decoder(model)
    ids = recipes.tokens(6, 1, 400, 1024).to(gpu)
    kap = ly.kappa.float().to(gpu).view(-1, 1)

    def expect_bias(st):
        b = kap * torch.log(st["mass"].clamp_min(1.0))
        return b.masked_fill(~st["act"], float("-inf"))

    with torch.no_grad():
        _, states, kv = dec.prefill(ids)
        st = kv[0]
        assert torch.allclose(st.slot_bias, expect_bias(st), rtol=1e-6, atol=0.0)
        m = st["mass"].clone()
        m[:, 5] = 7.0
        m[:, 17:40] = torch.linspace(1.5, 30.0, 23, device=gpu)
        st["mass"] = m
        assert torch.equal(st["mass"], m)
        assert torch.allclose(st.slot_bias[:, 5], kap[:, 0] * torch.log(torch.tensor(7.0, device=gpu)), rtol=1e-6)
        assert torch.allclose(st.slot_bias, expect_bias(st), rtol=1e-6, atol=0.0)
        assert set(st.keys()) == set(st.KEYS) and st.get("n_filled") == 128


def test_memorize_save_load_forget(gpu):
    """memorize -> save -> load -> forget (vsa_lm/config/bolt3.py:528-557, as the memory bank uses
    them): traces and the restored M_res against the oracle, and forget's result against its
    closed form M - gamma^k * delta on the loaded tensors."""
    from bolt3_amd import Bolt3Decoder
    print("[case] memorize / forget", flush=True)
    model = _model(7, ["vsa", "softmax"])
    ref = O.HybridRef(model)
    dmodel = copy.deepcopy(model).to(gpu)
    dec = Bolt3Decoder(dmodel)
    ids = recipes.tokens(7, 1, 260 + 384 + 256, 1024)
    prompt, doc, after = ids[:, :260], ids[:, 260:644], ids[:, 644:]
    with torch.no_grad():
        _, st_r = ref.prefill(prompt)
        pos_r, tr_r = ref.memorize(doc, st_r, 260)
        _, states, kv = dec.prefill(prompt.to(gpu))
        states, kv, pos, traces = dec.memorize(doc.to(gpu), states, kv, 260)
        assert pos == pos_r == 644 and traces[1] is None
        _close(traces[0][1].cpu(), tr_r[0][1], torch.float32, "trace")
        buf = io.BytesIO()
        s_cpu, kv_cpu = _to_cpu(states, kv)
        torch.save({"vsa_states": s_cpu, "kv_caches": kv_cpu, "next_pos": pos,
                    "traces": [None if t is None else (t[0], t[1].cpu()) for t in traces]}, buf)
        buf.seek(0)
        saved = torch.load(buf, weights_only=True)
        states, kv = _from_cpu(dmodel, saved["vsa_states"], saved["kv_caches"], gpu, 1024)
        h, pos = dec._feed(after.to(gpu), saved["next_pos"], states, kv)
        for s0 in range(0, after.shape[1], 128):
            ref.step(after[:, s0:s0 + 128], 644 + s0, st_r)
        m_before = states[0].clone()
        loaded = [None if t is None else (t[0], t[1].to(gpu)) for t in saved["traces"]]
        states = dec.forget(loaded, states, pos)
        ref.forget(tr_r, st_r, 644 + 256)
    gam = model.blocks[0].vsa.gamma_delta().view(1, -1, 1, 1).to(gpu)
    expect = m_before - gam ** 2 * loaded[0][1]                 # 256 positions after the trace: k = 2
    assert torch.allclose(states[0], expect, rtol=1e-6, atol=1e-7)
    _close(states[0].cpu(), st_r[0][0], torch.float32, "M_res after forget")


def test_memorize_pure_decay_closed_form(gpu):
    """With beta = 0 nothing is written into M_res, so memorizing n tokens only decays it:
    M_after = gamma^(n // C) * M_before and the trace is zero to rounding."""
    from bolt3_amd import Bolt3Decoder
    model = _model(8, ["vsa"], beta_off=False).to(gpu)
    dec = Bolt3Decoder(model)
    ids = recipes.tokens(8, 2, 680 + 256 + 384, 1024).to(gpu)
    with torch.no_grad():
        _, states, kv = dec.prefill(ids[:, :680])      # two steady consolidations: M_res is non-zero
        assert states[0].abs().max() > 0
        ly = model.blocks[0].vsa
        ly.beta_proj.weight.zero_()
        ly.beta_proj.bias.fill_(-1e4)
        # the window keeps each token's beta from when it came in: 256 tokens more, so that the chunks
        # memorize consolidates all came in with beta = 0
        _, pos = dec._feed(ids[:, 680:936], 680, states, kv)
        m0 = states[0].clone()
        states, kv, pos, traces = dec.memorize(ids[:, 936:], states, kv, 936)
    gam = ly.gamma_delta().view(1, -1, 1, 1).to(gpu)
    assert torch.allclose(states[0], gam ** 3 * m0, rtol=1e-5, atol=1e-8)
    assert float(traces[0][1].abs().max()) <= 1e-5 * float(m0.abs().max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_multi_token_step_mid_chunk(dtype, gpu):
    """A 100-token step while the current chunk already holds 44 tokens (the causal offset inside
    the current segment, then a consolidation of a 144-token chunk), then single tokens up to the
    next consolidation, every step against the oracle."""
    from bolt3_amd import Bolt3Decoder
    print(f"[case] multi-token step mid-chunk {dtype}", flush=True)
    model = _model(9, ["vsa"], dtype=dtype)
    ref = O.HybridRef(model)
    dec = Bolt3Decoder(copy.deepcopy(model).to(gpu))
    ids = recipes.tokens(9, 2, 300 + 100 + 130, 1024)
    with torch.no_grad():
        h_r, st_r = ref.prefill(ids[:, :300])
        h, states, kv = dec.prefill(ids[:, :300].to(gpu))
        _close(h.float().cpu(), h_r.float(), dtype, "prefill")
        h_r = ref.step(ids[:, 300:400], 300, st_r)
        h, states, kv = dec.step(ids[:, 300:400].to(gpu), 300, states, kv)
        _close(h.float().cpu(), h_r.float(), dtype, "100-token step")
        assert kv[0].n_filled == st_r[0][1].st.n_filled
        for i in range(130):
            pos = 400 + i
            h_r = ref.step(ids[:, pos:pos + 1], pos, st_r)
            h, states, kv = dec.step(ids[:, pos:pos + 1].to(gpu), pos, states, kv)
            _close(h.float().cpu(), h_r.float(), dtype, f"step {i}")
    _close(states[0].cpu(), st_r[0][0], torch.float32 if dtype == torch.float32 else torch.bfloat16, "M_res")


def test_generate_eos_and_close_think(gpu):
    """generate_batch (greedy) with end-of-sequence ids and a forced close-of-thinking sequence,
    tokens and lengths against the oracle's restatement of the reference loop, up to the first
    step whose top two logits are within 1e-4."""
    from bolt3_amd import Bolt3Decoder
    print("[case] generate eos / close-think", flush=True)
    model = _model(10, ["vsa", "softmax"], vocab=96)
    ref = O.HybridRef(model)
    dec = Bolt3Decoder(copy.deepcopy(model).to(gpu))
    ids = recipes.tokens(10, 3, 260, 96)
    eos, close = {11, 42}, [5, 6, 7]
    with torch.no_grad():
        t_r, n_r, gaps = ref.generate_greedy(ids, 150, eos_ids=eos, close_think_ids=close)
        toks, lengths = dec.generate_batch(ids.to(gpu), 150, temperature=0.0, eos_ids=eos, close_think_ids=close)
    toks = toks.cpu()
    n_cmp = next((i for i, g in enumerate(gaps) if g <= 1e-4), len(gaps))
    print(f"[case] oracle tokens {t_r.shape[1]}, kernel tokens {toks.shape[1]}, compared {n_cmp}", flush=True)
    assert torch.equal(toks[:, :n_cmp], t_r[:, :n_cmp])
    if n_cmp == len(gaps):
        assert toks.shape == t_r.shape and torch.equal(lengths.cpu(), n_r)


def test_generate_greedy_reduced_qwen3_stack(gpu):
    """The end-to-end configuration's layers at a reduced depth: Qwen3-4B layer shape (hidden 2560,
    32/8 heads, head_dim 128, SwiGLU 9728), three Bolt-3 layers and a softmax anchor, bf16,
    2 sequences of 300 prompt tokens, 24 greedy tokens; token by token against the oracle up to
    the first step whose top two logits are within a bf16 rounding of each other."""
    from bolt3_amd import Bolt3Decoder
    print("[case] reduced Qwen3-4B stack, greedy", flush=True)
    torch.manual_seed(0)
    model = _model(11, ["vsa", "vsa", "vsa", "softmax"], dim=2560, heads=(32, 8), head_dim=128, inter=9728,
                   vocab=2048, dtype=torch.bfloat16, theta=1e6, eps=1e-6)
    ref = O.HybridRef(model)
    dec = Bolt3Decoder(copy.deepcopy(model).to(gpu))
    ids = recipes.tokens(11, 2, 300, 2048)
    with torch.no_grad():
        t_r, _, gaps = ref.generate_greedy(ids, 24)
        toks, _ = dec.generate_batch(ids.to(gpu), 24, temperature=0.0)
    toks = toks.cpu()
    n_cmp = next((i for i, g in enumerate(gaps) if g <= 0.0625), len(gaps))
    print(f"[case] compared {n_cmp} of 24 tokens; gaps {['%.3f' % g for g in gaps[:8]]}", flush=True)
    assert n_cmp >= 1
    assert torch.equal(toks[:, :n_cmp], t_r[:, :n_cmp])


class _CharTokenizer:
    """A toy tokenizer over the model's vocabulary: one id per character (code point mod vocab)."""

    def __init__(self, vocab, eos):
        self.vocab, self.eos_token_id = vocab, eos

    def apply_chat_template(self, messages, tokenize=False, add_generation_prompt=True):
        raise NotImplementedError     # exercise the role-prefixed fallback

    def encode(self, text, add_special_tokens=False):
        return [ord(ch) % self.vocab for ch in text]

    def decode(self, ids, skip_special_tokens=True):
        return "".join(chr(33 + (i % 90)) for i in ids if not (skip_special_tokens and i == self.eos_token_id))


def test_serve_generate_completion(gpu):
    """The serving completion on a Bolt-3 stack equals the oracle's greedy continuation of the same
    prompt, cut at the first end-of-sequence id."""
    from bolt3_amd.serve import generate_completion, make_decoder
    model = _model(12, ["vsa", "softmax"], vocab=96)
    tok = _CharTokenizer(96, eos=42)
    msgs = [{"role": "user", "content": "x" * 150 + "tell me about slots"}]
    prompt = "\n".join(f"{m['role']}: {m['content']}" for m in msgs) + "\nassistant: "
    ids = torch.tensor([tok.encode(prompt)])
    ref = O.HybridRef(model)
    with torch.no_grad():
        t_r, n_r, gaps = ref.generate_greedy(ids, 40, eos_ids={42})
    dmodel = copy.deepcopy(model).to(gpu)
    reply = generate_completion(dmodel, tok, gpu, msgs, max_tokens=40, decoder=make_decoder(dmodel, gpu))
    n_cmp = next((i for i, g in enumerate(gaps) if g <= 1e-4), len(gaps))
    want = t_r[0, :int(n_r[0])].tolist()
    if want and want[-1] == 42:
        want = want[:-1]
    expect = tok.decode(want)               # one character per token, none of them blank
    assert reply[:n_cmp] == expect[:n_cmp], (reply, expect)
    if n_cmp == len(gaps):
        assert reply == expect


@pytest.mark.parametrize("name", ["gen_eos_close", "gen_all_done", "gen_full_length"])
def test_generate_matches_reference_fixture(name, gpu):
    """generate_batch (greedy, B = 3) against the reference's own tokens and lengths
    (tests/golden/gen_*: per-row end of sequence, the forced close-of-thinking sequence at the
    budget point, a row closing on its own, the all-rows-done stop at a 16-token check, a row
    running to the 150-token limit).  Every greedy pick of the fixtures has a top-2 logit gap
    above 0.06, so the tokens must match exactly; the graph-replayed step is not used (fp32)."""
    from bolt3_amd import Bolt3Decoder
    from helpers import build_fixture_model, fixture
    g, meta = fixture(name)
    model, ids = build_fixture_model(meta, meta["n_prompt"])
    print(f"[case] generate vs reference fixture {name}", flush=True)
    dec = Bolt3Decoder(model.to(gpu))
    with torch.no_grad():
        toks, lengths = dec.generate_batch(ids.to(gpu), meta["n_new"], temperature=0.0,
                                           eos_ids=set(meta["eos_ids"]), close_think_ids=meta["close_think_ids"])
    assert toks.shape == g["toks"].shape and torch.equal(toks.cpu(), g["toks"])
    assert torch.equal(lengths.cpu(), g["lengths"])


def test_memorize_forget_matches_reference_fixture(gpu):
    """memorize -> more tokens -> forget -> decode (tests/golden/mem_forget, the reference's own
    vectors): the trace, M_res after memorize, before and after forget, and the hidden states of
    the steps decoded afterwards, fp32 tolerance."""
    from bolt3_amd import Bolt3Decoder
    from helpers import build_fixture_model, fixture
    g, meta = fixture("mem_forget")
    n0, nd, na, npb = meta["n_prompt"], meta["n_doc"], meta["n_after"], meta["n_probe"]
    model, ids = build_fixture_model(meta, n0 + nd + na + npb)
    print("[case] memorize / forget vs reference fixture", flush=True)
    dec = Bolt3Decoder(model.to(gpu))
    ids = ids.to(gpu)
    with torch.no_grad():
        _, states, kv = dec.prefill(ids[:, :n0])
        states, kv, pos, traces = dec.memorize(ids[:, n0:n0 + nd], states, kv, n0)
        assert pos == meta["trace_end"] and traces[1] is None
        _close(traces[0][1].cpu(), g["trace"], torch.float32, "trace")
        _close(states[0].cpu(), g["m_memorized"], torch.float32, "M_res after memorize")
        _, pos = dec._feed(ids[:, n0 + nd:n0 + nd + na], pos, states, kv)
        _close(states[0].cpu(), g["m_before_forget"], torch.float32, "M_res before forget")
        states = dec.forget(traces, states, pos)
        _close(states[0].cpu(), g["m_after_forget"], torch.float32, "M_res after forget")
        hs = []
        for i in range(npb):
            h, states, kv = dec.step(ids[:, pos + i:pos + i + 1], pos + i, states, kv)
            hs.append(h[:, -1])
    _close(torch.stack(hs, dim=1).cpu(), g["h_probe"], torch.float32, "steps after forget")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_step_longer_than_a_chunk(dtype, gpu):
    """A step of more than C tokens (the reference's step takes any t, vsa_lm/config/bolt3.py:335-425):
    200 tokens at once on a current chunk of 44 (one attention over the window and all 244
    tokens, then one consolidation, after which the previous chunk holds 244 tokens), then
    single tokens across the next consolidation (of those 244 tokens), every step against the
    oracle's layer_step; a step that would make a chunk of more than 2C tokens is refused before
    any state changes."""
    from bolt3_amd import Bolt3Decoder
    print(f"[case] step of 200 tokens mid-chunk {dtype}", flush=True)
    model = _model(13, ["vsa", "softmax"], dtype=dtype)
    ref = O.HybridRef(model)
    dec = Bolt3Decoder(copy.deepcopy(model).to(gpu))
    ids = recipes.tokens(13, 2, 300 + 200 + 140, 1024)
    with torch.no_grad():
        h_r, st_r = ref.prefill(ids[:, :300])
        h, states, kv = dec.prefill(ids[:, :300].to(gpu))
        assert kv[0].cur[1] == 44
        h_r = ref.step(ids[:, 300:500], 300, st_r)
        h, states, kv = dec.step(ids[:, 300:500].to(gpu), 300, states, kv)
        _close(h.float().cpu(), h_r.float(), dtype, "200-token step")
        assert kv[0].prev[1] == 244 and kv[0].cur[1] == 0
        for i in range(140):
            pos = 500 + i
            h_r = ref.step(ids[:, pos:pos + 1], pos, st_r)
            h, states, kv = dec.step(ids[:, pos:pos + 1].to(gpu), pos, states, kv)
            _close(h.float().cpu(), h_r.float(), dtype, f"step {i}")
        assert kv[0].n_filled == st_r[0][1].st.n_filled
        _close(states[0].cpu(), st_r[0][0], torch.float32 if dtype == torch.float32 else torch.bfloat16, "M_res")
        before = (states[0].clone(), kv[0].cur, kv[1].n)
        with pytest.raises(NotImplementedError):
            dec.step(ids[:, :250].to(gpu), 640, states, kv)
        assert torch.equal(states[0], before[0]) and kv[0].cur == before[1] and kv[1].n == before[2]
