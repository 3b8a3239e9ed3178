"""The oracle's decision forcing (consolidate(force=...), forward(decisions=...),
HybridRef(decisions=...)), the tool the GPU tests use to follow the kernel's trajectory in the
oracle's arithmetic.  Pinned on the CPU by: forcing the oracle's own decisions changes nothing
(bit for bit); forcing the decisions of the other tie rule reproduces that rule's run bit for
bit (the clustered fixtures order many exact ties, so the two rules' trajectories differ); a
forced merge or replacement produces the closed-form slot contents."""
from __future__ import annotations

import torch

from helpers import build_layer, build_model, decisions_from_oracle_log, fixture
from oracle import bolt3_oracle as O


def _run(name, ties, decisions=None):
    g, meta = fixture(name)
    mod, x = build_layer(meta)
    p = O.Bolt3Params.from_module(mod)
    tr = O.ForwardTrace()
    with torch.no_grad():
        y = O.forward(p, x, trace=tr, ties=ties, decisions=decisions)
    return p, x, y, tr


def _same_state(a: O.SlotState, b: O.SlotState) -> bool:
    return all(torch.equal(getattr(a, k), getattr(b, k)) for k in ("ak", "av", "mass", "util", "pm", "act", "m_res"))


def test_forcing_own_decisions_is_identity():
    _, _, y, tr = _run("fwd_fp32_clustered", "torch")
    dec = [decisions_from_oracle_log(lg) for lg in tr.logs]
    _, _, y2, tr2 = _run("fwd_fp32_clustered", "torch", dec)
    assert torch.equal(y, y2)
    assert all(_same_state(a, b) for a, b in zip(tr.states, tr2.states))
    for lg, lg2 in zip(tr.logs, tr2.logs):     # the oracle's own decisions are logged unchanged
        for k in lg:
            if torch.is_tensor(lg[k]):
                assert torch.equal(lg[k], lg2[k]), k


def test_forcing_other_tie_rule_reproduces_it():
    """fwd_bf16_clustered orders exact ties in many steps: the lowest-index rule and torch.topk's
    order part ways.  The torch-order run forced with the index-rule decisions is the index-rule
    run, bit for bit, and its logs show where its own (torch-order) decisions differ."""
    for name in ("fwd_bf16_clustered", "fwd_fp32_clustered"):
        _, _, y_idx, tr_idx = _run(name, "index")
        _, _, y_tor, tr_tor = _run(name, "torch")
        dec = [decisions_from_oracle_log(lg) for lg in tr_idx.logs]
        _, _, y_f, tr_f = _run(name, "torch", dec)
        assert torch.equal(y_f, y_idx), name
        assert all(_same_state(a, b) for a, b in zip(tr_f.states, tr_idx.states)), name
        if name == "fwd_bf16_clustered":
            assert not torch.equal(y_tor, y_idx)    # the rules do part on this fixture
            n_diff = sum(int((lg["win"] != lg_i["win"]).any() or (lg["top_toks"] != lg_i["top_toks"]).any())
                         for lg, lg_i in zip(tr_f.logs, tr_idx.logs) if lg["kind"] == "steady")
            assert n_diff > 0


def test_forced_merge_and_replacement_closed_form():
    """One steady step from a known state with planted decisions: token 0 merged into slot 3 (a
    slot the oracle would not pick for it), token 1 replacing slot 7: slot 3 becomes the
    mass-weighted mean of itself and token 0's key, slot 7 holds token 1 with mass 1, every other
    slot is unchanged, token 1 and token 0 are kept out of M_res."""
    p, x, _, tr = _run("fwd_fp32_eta", "torch")
    b = fixture("fwd_fp32_eta")[1]["B"]
    i = 3
    st0, chunk = tr.states[i - 1], tr.chunks[i]
    kr, kp, v, pos, beta = chunk
    bh, l, hd = kr.shape
    gam = O.gamma_delta(p.log_gamma)
    lg = {}
    O.consolidate(p, st0, *chunk, gam, b, log=lg)
    slot = lg["slot"].clone()
    merge = torch.zeros(bh, l, dtype=torch.bool)
    slot[:, 0], merge[:, 0] = 3, True
    kc = min(l, p.S)
    top = torch.arange(kc).expand(bh, kc).clone()
    top[:, 0] = 1
    top[:, 1] = 0
    bot = torch.arange(kc).expand(bh, kc).clone()
    bot[:, 0] = 7
    bot[:, 7] = 0
    win = torch.zeros(bh, kc, dtype=torch.bool)
    win[:, 0] = True
    force = dict(slot=slot, merge=merge, top_toks=top, bot_slots=bot, win=win)
    lg2 = {}
    st = O.consolidate(p, st0, *chunk, gam, b, log=lg2, force=force)
    m0 = st0.mass[:, 3]
    want_k = (m0.unsqueeze(-1) * st0.ak[:, 3].float() + kr[:, 0].float()) / (m0 + 1).unsqueeze(-1)
    assert torch.equal(st.ak[:, 3], want_k.to(st.ak.dtype))
    assert torch.equal(st.mass[:, 3], m0 + 1)
    assert torch.equal(st.ak[:, 7], kr[:, 1]) and torch.equal(st.av[:, 7], v[:, 1])
    assert torch.equal(st.mass[:, 7], torch.ones(bh)) and torch.equal(st.pm[:, 7], pos[1].expand(bh))
    others = [s for s in range(p.S) if s not in (3, 7)]
    assert torch.equal(st.ak[:, others], st0.ak[:, others])
    assert torch.equal(st.mass[:, others], st0.mass[:, others])
    applied = lg2["delta_applied"]
    assert not bool(applied[:, 0].any()) and not bool(applied[:, 1].any())
    assert bool(applied[:, 2:].all())     # the rest: neither merged nor replacing
    # the logged own decisions are those of the free run (merges from the same state)
    assert torch.equal(lg2["merge"], lg["merge"]) and torch.equal(lg2["slot"], lg["slot"])


def test_hybrid_ref_forcing_own_decisions_is_identity():
    g, meta = fixture("dec_fp32")
    model, ids = build_model(meta)
    n_prompt = meta["n_prompt"]
    logs = {}
    ref = O.HybridRef(model, logs=logs)
    with torch.no_grad():
        h, st = ref.prefill(ids[:, :n_prompt])
        hs = [ref.step(ids[:, n_prompt + i:n_prompt + i + 1], n_prompt + i, st) for i in range(140)]
    dec = {li: [decisions_from_oracle_log(lg) for lg in lgs] for li, lgs in logs.items()}
    ref2 = O.HybridRef(model, decisions=dec)
    with torch.no_grad():
        h2, st2 = ref2.prefill(ids[:, :n_prompt])
        hs2 = [ref2.step(ids[:, n_prompt + i:n_prompt + i + 1], n_prompt + i, st2) for i in range(140)]
    assert torch.equal(h, h2) and all(torch.equal(a, b) for a, b in zip(hs, hs2))
    assert all(ref2._n_forced[li] == len(v) for li, v in dec.items())
