"""Torch restatement of the consolidation chain's backward: the checker of bolt3_chain_bwd.

TEST INFRASTRUCTURE ONLY (the product computes this gradient in bolt3_chain_bwd and has no other
path).  Pinned by tests/test_backward_host.py against autograd through the oracle's
consolidate, which the reference's gradient fixtures pin; tests/test_gpu_chain_bwd.py compares
the kernels with it.

* ``replay_slots``   -- the slots' mass and mean position after every step, rebuilt from the
                        chain kernel's decision log (vsa_lm/config/bolt3.py:125-136, :145-150,
                        :182-191);
* ``chain_backward`` -- the reverse pass over the steps (vsa_lm/config/bolt3.py:121-166 for
                        steady steps, :182-191 for fills).
"""
from __future__ import annotations

import torch

from bolt3_amd import _abi as A

LOG = {name: i for i, name in enumerate(A.LOG_FIELDS)}


def _rope_t(g: torch.Tensor, ang: torch.Tensor) -> torch.Tensor:
    """Transpose of x -> x*cos + rotate_half(x)*sin (a rotation by the angle): the rotation by
    minus the angle.  ang broadcasts against g's leading axes, last axis HD/2."""
    a = torch.cat((ang, ang), dim=-1)
    half = g.shape[-1] // 2
    rot = torch.cat((-g[..., half:], g[..., :half]), dim=-1)
    return g * a.cos() - rot * a.sin()


def _snap_m(snap_m: torch.Tensor, i: int, split: bool, bh: int, HD: int) -> torch.Tensor:
    """M_res after step i as fp32 [bh, HD, HD] (bf16 snapshots hold M^T as bf16 hi then lo)."""
    if not split:
        return snap_m[i]
    raw = snap_m[i].view(torch.bfloat16).view(bh, 2, HD, HD)
    return (raw[:, 0].float() + raw[:, 1].float()).transpose(1, 2)


def replay_slots(log: torch.Tensor, pos: torch.Tensor, S: int, C: int, ns: int):
    """Mass and mean position of every slot after each step, rebuilt from the decision log
    (fills set mass 1 and the token's position; merges add counts and position sums,
    vsa_lm/config/bolt3.py:125-136; evictions set mass 1 and the winner's position, :145-150).
    Counts and position sums are integers, so the replay reproduces the forward's fp32 values.
    Returns (steps, masses, positions): per step a record of its decisions."""
    n, bh = log.shape[0], log.shape[1]
    dev = log.device
    mass = torch.ones(bh, S, device=dev)
    pm = torch.zeros(bh, S, device=dev)
    nf = 0
    steps, masses, pms = [], [], []
    for i in range(n):
        t0, l = (ns, C - ns) if i == 0 else (i * C, C)
        p = pos[t0:t0 + l]
        lg = log[i]
        if nf < S:
            m = min(S - nf, l)
            picked = lg[:, LOG["top_tok"], :m].long()
            mass = mass.clone()
            pm = pm.clone()
            mass[:, nf:nf + m] = 1.0
            pm[:, nf:nf + m] = p[picked]
            steps.append(dict(kind="fill", t0=t0, l=l, nf=nf, m=m, picked=picked))
            nf += m
        else:
            kc = min(l, S)
            slot = lg[:, LOG["slot"], :l].long().clamp_min(0)
            merge = lg[:, LOG["merge"], :l] > 0.5
            mo = merge.float()
            cnt = torch.zeros(bh, S, device=dev).scatter_add_(1, slot, mo)
            p_acc = torch.zeros(bh, S, device=dev).scatter_add_(1, slot, mo * p)
            hit = cnt > 0
            new_m = mass + cnt
            rec = dict(kind="steady", t0=t0, l=l, slot=slot, merge=merge, hit=hit, mass=mass, new_m=new_m,
                       toks=lg[:, LOG["top_tok"], :kc].long(), bots=lg[:, LOG["bot_slot"], :kc].long(),
                       win=lg[:, LOG["win"], :kc] > 0.5, delta=lg[:, LOG["delta"], :l] > 0.5)
            pm = torch.where(hit, (mass * pm + p_acc) / new_m, pm)
            mass = torch.where(hit, new_m, mass)
            w, bots = rec["win"], rec["bots"]
            mass = mass.scatter(1, bots, torch.where(w, torch.ones_like(p[rec["toks"]]), mass.gather(1, bots)))
            pm = pm.scatter(1, bots, torch.where(w, p[rec["toks"]], pm.gather(1, bots)))
            steps.append(rec)
        masses.append(mass)
        pms.append(pm)
    return steps, masses, pms


def chain_backward(steps, d_slot_k, d_slot_v, d_m, pms, inv_freq, kr, v, beta, gam, snap_m, m_split, b, HKV):
    """Gradients of the consolidated tokens' keys (un-roped), values and beta, and of gamma,
    from the gradients of every step's slot snapshot (roped keys, values) and M_res, by the
    steps in reverse (vsa_lm/config/bolt3.py:121-166 for steady steps, :182-191 for fills).
    kr, v: [bh, T, HD]; beta: [bh, T].  Returns (d_kr, d_v, d_beta, d_gamma).

    Only two recursions are sequential over the steps: the slots' gradient (copied, scaled by
    mass / new mass at merges, cleared at evictions) and M_res's, G_i = dM_i + A_{i+1} G_{i+1}
    with A = gam I - kn^T diag(bsafe) kn.  Everything else is batched over all steps."""
    bh, T, HD = kr.shape
    S = d_slot_k.shape[2]
    n = len(steps)
    dev = kr.device
    d_kr = torch.zeros(bh, T, HD, device=dev)
    d_v = torch.zeros(bh, T, HD, device=dev)
    d_beta = torch.zeros(bh, T, device=dev)
    gam_bh = gam.float().repeat(b).view(bh, 1, 1)
    steady = [i for i in range(n) if steps[i]["kind"] == "steady"]
    # ---- batched over the steady steps: normalised keys, Gershgorin scales, residuals
    if steady:
        t0s = [steps[i]["t0"] for i in steady]
        l = steps[steady[0]]["l"]
        idx = torch.tensor(t0s, device=dev)[:, None] + torch.arange(l, device=dev)           # [ns, l]
        kri = kr[:, idx].float().transpose(0, 1).reshape(-1, l, HD)                          # [ns*bh, l, HD]
        vi = v[:, idx].float().transpose(0, 1).reshape(-1, l, HD)
        dmask = torch.stack([steps[i]["delta"] for i in steady]).float().reshape(-1, l)
        wv = beta[:, idx].float().transpose(0, 1).reshape(-1, l) * dmask
        M0 = torch.stack([_snap_m(snap_m, i - 1, m_split, bh, HD) for i in steady]).reshape(-1, HD, HD)
        nrm = kri.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        kn = kri / nrm
        P = torch.bmm(kn, kn.transpose(1, 2))
        G = P.abs()
        rs_raw = torch.bmm(G, wv[..., None]).squeeze(-1)
        rs = rs_raw.clamp_min(1.0)
        bs = wv / rs
        R = vi - torch.bmm(kn, M0)
        E = bs[..., None] * R
        kn_s = kn.view(len(steady), bh, l, HD)
        bs_s = bs.view(len(steady), bh, l, 1)
    pos_of = {i: k for k, i in enumerate(steady)}
    # ---- the two sequential recursions
    slot_grad = _rope_t(d_slot_k, torch.stack(pms)[..., None] * inv_freq)    # [n, bh, S, HD]
    dak = torch.zeros(bh, S, HD, device=dev)
    dav = torch.zeros(bh, S, HD, device=dev)
    cur = torch.zeros(bh, HD, HD, device=dev)
    g_m = [None] * n
    at_evict, at_merge = [None] * n, [None] * n
    for i in range(n - 1, -1, -1):
        st = steps[i]
        cur = cur + d_m[i]
        g_m[i] = cur
        dak = dak + slot_grad[i]
        dav = dav + d_slot_v[i]
        if st["kind"] == "fill":
            nf, m, picked = st["nf"], st["m"], st["picked"]
            t0 = st["t0"]
            pi = picked[..., None].expand(-1, -1, HD)
            d_kr[:, t0:t0 + st["l"]].scatter_add_(1, pi, dak[:, nf:nf + m])
            d_v[:, t0:t0 + st["l"]].scatter_add_(1, pi, dav[:, nf:nf + m])
            keep = torch.ones(1, S, 1, device=dev)
            keep[:, nf:nf + m] = 0.0
            dak = dak * keep
            dav = dav * keep
            continue
        at_evict[i] = (dak, dav)
        # a winning pair's slot was overwritten by the token (vsa_lm/config/bolt3.py:145-150)
        wmask = torch.zeros(bh, S, device=dev).scatter_(1, st["bots"], st["win"].float())
        clear = (1.0 - wmask)[..., None]
        dak = dak * clear
        dav = dav * clear
        at_merge[i] = (dak, dav)
        # ak <- (mass * ak + merged keys) / (mass + count) (:125-136)
        keep = torch.where(st["hit"], st["mass"] / st["new_m"], torch.ones_like(st["new_m"]))[..., None]
        dak = dak * keep
        dav = dav * keep
        # M_res: dM_before = gam dM - kn^T (bsafe * (kn dM)) (:157-166)
        k = pos_of[i]
        cur = gam_bh * cur - torch.bmm(kn_s[k].transpose(1, 2), bs_s[k] * torch.bmm(kn_s[k], cur))
    # ---- token gradients of the steady steps, batched
    d_gam = torch.zeros(HKV, device=dev)
    if steady:
        for i in steady:
            st = steps[i]
            t0, l = st["t0"], st["l"]
            wf = st["win"].float()[..., None]
            bi = st["bots"][..., None].expand(-1, -1, HD)
            ti = st["toks"][..., None].expand(-1, -1, HD)
            dak_e, dav_e = at_evict[i]
            d_kr[:, t0:t0 + l].scatter_add_(1, ti, dak_e.gather(1, bi) * wf)
            d_v[:, t0:t0 + l].scatter_add_(1, ti, dav_e.gather(1, bi) * wf)
        coef = torch.stack([steps[i]["merge"].float() / steps[i]["new_m"].gather(1, steps[i]["slot"])
                            for i in steady])[..., None]                                    # [ns, bh, l, 1]
        sidx = torch.stack([steps[i]["slot"] for i in steady])[..., None].expand(-1, -1, -1, HD)
        dak_m = torch.stack([at_merge[i][0] for i in steady])
        dav_m = torch.stack([at_merge[i][1] for i in steady])
        gk = coef * dak_m.gather(2, sidx)                                                  # [ns, bh, l, HD]
        gv = coef * dav_m.gather(2, sidx)
        Gm = torch.stack([g_m[i] for i in steady]).reshape(-1, HD, HD)
        dE = torch.bmm(kn, Gm)
        d_kn = torch.bmm(E, Gm.transpose(1, 2))
        dR = bs[..., None] * dE
        d_kn -= torch.bmm(dR, M0.transpose(1, 2))
        d_bs = (dE * R).sum(-1)
        d_w = d_bs / rs
        d_rs = torch.where(rs_raw >= 1.0, -d_bs * wv / (rs * rs), torch.zeros_like(rs))
        d_w += torch.bmm(G.transpose(1, 2), d_rs[..., None]).squeeze(-1)
        dP = (d_rs[..., None] * wv[:, None, :]) * torch.sign(P)
        d_kn += torch.bmm(dP + dP.transpose(1, 2), kn)
        d_kn = (d_kn - kn * (kn * d_kn).sum(-1, keepdim=True)) / nrm
        gk = gk + d_kn.view(len(steady), bh, l, HD)
        gv = gv + dR.view(len(steady), bh, l, HD)
        d_kr[:, idx] += gk.transpose(0, 1)
        d_v[:, idx] += gv.transpose(0, 1)
        d_beta[:, idx] += (d_w * dmask).view(len(steady), bh, l).transpose(0, 1)
        d_gam = (Gm * M0).sum(dim=(1, 2)).view(len(steady), b, HKV).sum(dim=(0, 1))
    return d_kr, d_v, d_beta, d_gam
