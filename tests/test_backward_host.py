"""The torch restatement of the chain's backward on the CPU (tests/chain_bwd_ref.py, the checker
of the HIP chain backward): the slot replay and the reverse pass against autograd through the
oracle's consolidate, which the reference's gradient fixtures pin (test_oracle_golden.py).

The decision log is the chain kernel's format (include/bolt3_amd.h, B3_LOG_*), filled here from
the oracle's per-step decisions, so no kernel runs."""
import pytest
import torch

from bolt3_amd import _abi as A
from chain_bwd_ref import chain_backward, replay_slots
from helpers import build_grad_case, fixture, rel_err
from oracle import bolt3_oracle as O

LOG = {name: i for i, name in enumerate(A.LOG_FIELDS)}


def _kernel_log(logs, bh):
    out = torch.zeros(len(logs), bh, A.LOG_ROWS, A.LOG_COLS)
    out[:, :, LOG["top_tok"]] = -1.0
    for i, lg in enumerate(logs):
        if lg["kind"] == "fill":
            m = lg["picked"].shape[1]
            out[i, :, LOG["top_tok"], :m] = lg["picked"].float()
            continue
        l, kc = lg["slot"].shape[1], lg["top_toks"].shape[1]
        out[i, :, LOG["slot"], :l] = lg["slot"].float()
        out[i, :, LOG["merge"], :l] = lg["merge"].float()
        out[i, :, LOG["delta"], :l] = lg["delta"].float()
        out[i, :, LOG["top_tok"], :kc] = lg["top_toks"].float()
        out[i, :, LOG["bot_slot"], :kc] = lg["bot_slots"].float()
        out[i, :, LOG["win"], :kc] = lg["win"].float()
    return out


@pytest.mark.parametrize("name", ["grad_fp32_clustered", "grad_fp32_eta", "grad_fp32_hd128"])
def test_replay_and_chain_backward_match_autograd(name):
    g, meta = fixture(name)
    mod, x, _ = build_grad_case(meta)
    p = O.Bolt3Params.from_module(mod)
    tr = O.ForwardTrace()
    with torch.no_grad():
        O.forward(p, x, trace=tr)
    b, T = x.shape[0], x.shape[1]
    HKV, HD, S, C = p.HKV, p.HD, p.S, p.C
    bh, ns = b * HKV, min(O.N_SINKS, C)
    n = len(tr.states)
    assert n >= 3
    log = _kernel_log(tr.logs, bh)
    pos = torch.arange(T, dtype=torch.float32)
    steps, masses, pms = replay_slots(log, pos, S, C, ns)
    for i, st in enumerate(tr.states):
        assert torch.equal(masses[i], st.mass), i
        assert torch.equal(pms[i], st.pm), i
    # autograd through the oracle's steps with the decisions of the forward above
    q_raw, q_rope, k_raw, k_rope, v_all, beta_all, _ = tr.heads
    kr = k_raw.detach().reshape(bh, T, HD).clone().requires_grad_(True)
    vv = v_all.detach().reshape(bh, T, HD).clone().requires_grad_(True)
    be = beta_all.detach().reshape(bh, T).clone().requires_grad_(True)
    kp = k_rope.detach().reshape(bh, T, HD)
    gam = O.gamma_delta(p.log_gamma).detach().clone().requires_grad_(True)
    gen = torch.Generator().manual_seed(5)
    dk = torch.randn(n, bh, S, HD, generator=gen)
    dv = torch.randn(n, bh, S, HD, generator=gen)
    dm = torch.randn(n, bh, HD, HD, generator=gen)
    st, loss, snaps = None, 0.0, []
    for i in range(n):
        t0, l = (ns, C - ns) if i == 0 else (i * C, C)
        st = O.consolidate(p, st, kr[:, t0:t0 + l], kp[:, t0:t0 + l], vv[:, t0:t0 + l], pos[t0:t0 + l],
                           be[:, t0:t0 + l], gam, b)
        assert torch.equal(st.mass, tr.states[i].mass)
        loss = loss + (O.slot_keys(p, st, b) * dk[i]).sum() + (st.av * dv[i]).sum() + (st.m_res * dm[i]).sum()
        snaps.append(st.m_res.detach())
    loss.backward()
    d_kr, d_v, d_beta, d_gam = chain_backward(steps, dk, dv, dm, pms, p.inv_freq.float(), kr.detach(), vv.detach(),
                                              be.detach(), gam.detach(), torch.stack(snaps), False, b, HKV)
    assert rel_err(d_kr, kr.grad) <= 1e-5, rel_err(d_kr, kr.grad)
    assert rel_err(d_v, vv.grad) <= 1e-5, rel_err(d_v, vv.grad)
    assert rel_err(d_beta, be.grad) <= 1e-5, rel_err(d_beta, be.grad)
    assert rel_err(d_gam, gam.grad) <= 1e-5, rel_err(d_gam, gam.grad)
