"""Backward of Bolt3Attn.forward on the HIP path.

The reference differentiates its forward with autograd (vsa_lm/config/bolt3.py:194-276); its
slot decisions run under no_grad (:98-112, :121-135, :165-180), so the gradient is that of a
forward whose decisions are constants.  This module computes the same gradients from what the
HIP forward keeps:

* the attention over [sinks | slots | window] and the M_res readout of every chunk are
  differentiated by ``bolt3_attn_bwd`` (three HIP kernels, fp32), which returns the gradients
  of the roped queries, the un-roped queries (readout), eta, every key field, every slot
  snapshot, the slot bias, M_res of every step, res_norm's weight and gamma;
* the consolidation chain is differentiated by replaying the forward's decision log (the chain
  kernel's per-step record of fills, merges, evictions and delta-rule writes) backwards over
  the steps: the slots' keys and values are copies and mass-weighted means of token keys and
  values (:121-155, :182-191), M_res follows the Gershgorin-scaled delta rule (:157-166);
* RoPE, the q/k RMSNorm, the gates' sigmoid / tanh, gamma's clamp and the projections close the
  chain back to x and the parameters.

The replay is a fixed sequence of batched products over all (batch, kv head) rows per step,
run on the forward's device and stream.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _abi as A

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


def chain_backward_hip(mod, tr: dict, o: dict, gam: torch.Tensor, b: int, n_steps: int):
    """bolt3_chain_bwd on the forward's trace and the attention backward's outputs: returns
    (d_kr, d_v, d_beta, d_gamma) like chain_backward."""
    HKV, HD, S, C = mod.HKV, mod.HD, mod.S, mod.C
    k_raw = tr["k_raw"]
    T = k_raw.shape[2]
    bh = b * HKV
    dev = k_raw.device
    ns = min(mod.n_sinks, C)
    f32 = dict(device=dev, dtype=torch.float32)
    d_kr, d_v = torch.zeros(bh, T, HD, **f32), torch.zeros(bh, T, HD, **f32)
    d_beta = torch.zeros(bh, T, **f32)
    d_gamma = torch.empty(n_steps, bh, HD // 32, **f32)
    work = torch.empty(A.chain_bwd_workspace_bytes(b, HKV, HD, n_steps), dtype=torch.uint8, device=dev)
    a = A.ChainBwdArgs()
    a.dtype, a.B, a.HKV, a.HD, a.S, a.T = A.dtype_code(k_raw.dtype), b, HKV, HD, S, T
    a.n_steps, a.off0, a.len0, a.step_stride, a.step_len = n_steps, ns, C - ns, C, C
    a.kr, a.v, a.beta, a.log = k_raw.data_ptr(), tr["v"].data_ptr(), tr["beta"].data_ptr(), tr["log"].data_ptr()
    a.snap_mass, a.snap_pm, a.snap_m = tr["snap_mass"].data_ptr(), tr["snap_pm"].data_ptr(), tr["snap_m"].data_ptr()
    a.gamma, a.inv_freq = gam.data_ptr(), mod._packed(k_raw.dtype, dev)[2]["inv_freq"].data_ptr()
    a.d_slot_k, a.d_slot_v, a.d_m = o["d_slot_k"].data_ptr(), o["d_slot_v"].data_ptr(), o["d_m"].data_ptr()
    a.d_kr, a.d_v, a.d_beta, a.d_gamma = d_kr.data_ptr(), d_v.data_ptr(), d_beta.data_ptr(), d_gamma.data_ptr()
    a.work, a.work_bytes = work.data_ptr(), work.numel()
    A.call("bolt3_chain_bwd", a, dev)
    return d_kr, d_v, d_beta, d_gamma.view(n_steps, b, HKV, -1).sum(dim=(0, 1, 3))


def native_chain_ok(mod, dt: torch.dtype) -> bool:
    """Whether bolt3_chain_bwd takes this layer's chain (bf16 storage, HD = S = 128, C <= 128)."""
    return dt == torch.bfloat16 and mod.HD == 128 and mod.S == 128 and mod.C <= 128


def attn_backward(mod, tr: dict, dy: torch.Tensor, dt: torch.dtype, n_steps: int):
    """bolt3_attn_bwd on the forward's tensors: returns its output buffers by name."""
    q_rope, q_raw, k_rope, v, eta = tr["q_rope"], tr["q_raw"], tr["k_rope"], tr["v"], tr["eta"]
    b, H, T, HD = q_rope.shape
    HKV, S, C = mod.HKV, mod.S, mod.C
    dev = q_rope.device
    bh = b * HKV
    n_chunks = (T + C - 1) // C
    n_qt = (C + 31) // 32
    ns = min(mod.n_sinks, C)
    f32 = dict(device=dev, dtype=torch.float32)
    sdt = dict(device=dev, dtype=dt)   # the row gradients of storage-dtype tensors
    o = dict(d_rows=torch.empty(b, H, T, **f32), lse=torch.empty(b, H, T, **f32),
             d_q_rope=torch.empty(b, H, T, HD, **sdt), d_q_raw=torch.empty(b, H, T, HD, **sdt),
             d_eta=torch.empty(b, H, T, **f32), d_res_w=torch.zeros(bh, n_chunks, HD, **f32),
             d_gamma=torch.zeros(bh, n_chunks, **f32),
             d_k_own=torch.empty(b, HKV, T, HD, **sdt), d_v_own=torch.empty(b, HKV, T, HD, **sdt),
             d_k_next=torch.empty(b, HKV, T, HD, **sdt), d_v_next=torch.empty(b, HKV, T, HD, **sdt))
    # rows no kernel writes are zero: the q_raw and eta gradients of chunks without a readout
    # (0 and 1, or all when nothing was consolidated), the next-chunk key / value gradients of
    # the last chunk's keys
    t_m = min(T, 2 * C) if n_steps > 0 else T
    o["d_q_raw"][:, :, :t_m].zero_()
    o["d_eta"][:, :, :t_m].zero_()
    o["d_k_next"][:, :, (n_chunks - 1) * C:].zero_()
    o["d_v_next"][:, :, (n_chunks - 1) * C:].zero_()
    a = A.AttnBwdArgs()
    a.dtype, a.B, a.T, a.H, a.HKV, a.HD, a.S, a.C = A.dtype_code(dt), b, T, H, HKV, HD, S, C
    a.n_sinks, a.n_chunks, a.n_qtiles, a.n_steps, a.score_round = mod.n_sinks, n_chunks, n_qt, n_steps, 1
    a.q_rope, a.q_raw, a.q_sb, a.q_sh = q_rope.data_ptr(), q_raw.data_ptr(), q_rope.stride(0), q_rope.stride(1)
    a.win_k, a.win_v, a.w_sb, a.w_sh = k_rope.data_ptr(), v.data_ptr(), k_rope.stride(0), k_rope.stride(1)
    if n_steps > 0:
        o.update(d_m=torch.empty(n_steps, bh, HD, HD, **f32), d_bias=torch.zeros(n_steps, b * H, n_qt, S, **f32),
                 d_slot_k=torch.empty(n_steps, bh, S, HD, **f32), d_slot_v=torch.empty(n_steps, bh, S, HD, **f32),
                 d_sink_k=torch.zeros(n_chunks, bh, ns, HD, **f32), d_sink_v=torch.zeros(n_chunks, bh, ns, HD, **f32))
        a.slot_k, a.slot_v, a.slot_bias = tr["snap_k"].data_ptr(), tr["snap_v"].data_ptr(), tr["snap_bias"].data_ptr()
        a.slot_step = bh * S * HD
        a.m_res, a.m_step, a.m_split = tr["snap_m"].data_ptr(), bh * HD * HD, int(dt == torch.bfloat16)
    a.eta, a.e_sb, a.e_sh = eta.data_ptr(), eta.stride(0), eta.stride(1)
    side = mod._packed(dt, dev)[2]
    a.gamma, a.res_w, a.eps = side["gamma"].data_ptr(), side["res_w"].data_ptr(), float(mod.res_norm.eps)
    y = tr["y"]
    a.y, a.y_sb, a.y_st = y.data_ptr(), y.stride(0), y.stride(1)
    a.dy, a.dy_sb, a.dy_st = dy.data_ptr(), dy.stride(0), dy.stride(1)
    for name, t in o.items():
        setattr(a, name, t.data_ptr())
    A.call("bolt3_attn_bwd", a, dev)
    return o


def layer_backward(mod, x: torch.Tensor, tr: dict, d_out: torch.Tensor, dt: torch.dtype):
    """Gradients of Bolt3Attn.forward: (dx, {parameter name: gradient}); the projections'
    gradients (dx among them) in the storage dtype their products run in, the rest fp32."""
    b, T, D = x.shape
    H, HKV, HD, S, C = mod.H, mod.HKV, mod.HD, mod.S, mod.C
    G = H // HKV
    bh = b * HKV
    dev = x.device
    n_chunks = (T + C - 1) // C
    n_steps = max(0, n_chunks - 2)
    ns = min(mod.n_sinks, C)
    grads = {}
    # the projections' products run in the storage dtype, as the reference's linears do under
    # autocast (fp32 storage: fp32 products)
    W, _, side = mod._packed(dt, dev)
    if "wT" not in side:   # the weights' transposes, for products in F.linear's layout (cached with the pack)
        side["wT"], side["woT"] = W.t().contiguous(), side["wo"].t().contiguous()
    d_out = d_out.to(dt)
    # o_proj
    y = tr["y"]
    grads["o_proj.weight"] = d_out.reshape(-1, D).t() @ y.reshape(-1, H * HD)
    dy = F.linear(d_out, side["woT"])                               # [b, T, H*HD], storage dtype
    # attention and readout
    o = attn_backward(mod, tr, dy, dt, n_steps)
    inv_freq = mod.rope.inv_freq.to(dev).float()
    gam = mod.gamma_delta().detach().to(dev)
    d_gam = o["d_gamma"].view(b, HKV, n_chunks).sum(dim=(0, 2))
    d_kappa = torch.zeros(HKV, device=dev)
    if n_steps > 0:
        # kappa: the slot bias is kappa * log(max(mass, 1)) (vsa_lm/config/bolt3.py:238-241)
        dbias = o["d_bias"].sum(2).view(n_steps, b, HKV, G, S).sum(3)             # [step, b, HKV, S]
        logm = tr["snap_mass"].clamp_min(1.0).log().view(n_steps, b, HKV, S)
        d_kappa = (dbias * logm).sum(dim=(0, 1, 3))
        if native_chain_ok(mod, dt):
            dk_c, dv_c, db_c, dg_c = chain_backward_hip(mod, tr, o, gam, b, n_steps)
        else:
            pos = torch.arange(T, device=dev, dtype=torch.float32)
            steps, _, pms = replay_slots(tr["log"], pos, S, C, ns)
            dk_c, dv_c, db_c, dg_c = chain_backward(
                steps, o["d_slot_k"], o["d_slot_v"], o["d_m"], pms, inv_freq, tr["k_raw"].reshape(bh, T, HD),
                tr["v"].reshape(bh, T, HD), tr["beta"].reshape(bh, T), gam, tr["snap_m"], dt == torch.bfloat16, b,
                HKV)
        d_gam += dg_c
    # RoPE transposes, the q / k norms' backward and the gates' derivatives, one pass over the
    # token rows into dz, the gradient of the packed projection output [q | k | v | beta | eta | pad]
    f32 = dict(device=dev, dtype=torch.float32)
    dz = torch.empty(b * T, W.shape[0], dtype=dt, device=dev)
    has_norm = mod.q_norm is not None
    nb = A.heads_bwd_blocks(b, T)
    ha = A.HeadsBwdArgs()
    ha.dtype, ha.B, ha.T, ha.H, ha.HKV, ha.HD, ha.n_sinks, ha.n_chunks = A.dtype_code(dt), b, T, H, HKV, HD, ns, \
        n_chunks
    ha.d_q_raw, ha.d_q_rope = o["d_q_raw"].data_ptr(), o["d_q_rope"].data_ptr()
    ha.d_k_own, ha.d_k_next = o["d_k_own"].data_ptr(), o["d_k_next"].data_ptr()
    ha.d_v_own, ha.d_v_next = o["d_v_own"].data_ptr(), o["d_v_next"].data_ptr()
    if n_steps > 0:
        ha.d_sink_k, ha.d_sink_v = o["d_sink_k"].data_ptr(), o["d_sink_v"].data_ptr()
        ha.d_k_chain, ha.d_v_chain, ha.d_beta = dk_c.data_ptr(), dv_c.data_ptr(), db_c.data_ptr()
    ha.d_eta, ha.beta, ha.eta = o["d_eta"].data_ptr(), tr["beta"].data_ptr(), tr["eta"].data_ptr()
    if has_norm:
        lin_q, lin_kv = tr["lin_q"], tr["lin_kv"]
        qn_w, kn_w = mod.q_norm.weight.detach().float().contiguous(), mod.k_norm.weight.detach().float().contiguous()
        d_qn, d_kn = torch.empty(nb, HD, **f32), torch.empty(nb, HD, **f32)
        ha.lin_q, ha.lin_q_row_stride = lin_q.data_ptr(), lin_q.shape[-1]
        ha.lin_k, ha.lin_k_row_stride = lin_kv.data_ptr(), lin_kv.shape[-1]
        ha.qn_w, ha.kn_w, ha.has_qk_norm = qn_w.data_ptr(), kn_w.data_ptr(), 1
        ha.q_eps, ha.k_eps = float(mod.q_norm.eps), float(mod.k_norm.eps)
        ha.d_qn_w, ha.d_kn_w = d_qn.data_ptr(), d_kn.data_ptr()
    inv_f = inv_freq.contiguous()
    ha.inv_freq = inv_f.data_ptr()
    ha.dz, ha.dz_row_stride, ha.dz_cols = dz.data_ptr(), dz.shape[1], dz.shape[1]
    A.call("bolt3_heads_bwd", ha, dev)
    if has_norm:
        grads["q_norm.weight"], grads["k_norm.weight"] = d_qn.sum(0), d_kn.sum(0)
    widths = [H * HD, HKV * HD, HKV * HD, HKV, H]
    # one product each for dx and for the packed weight's gradient: rows q | k | v | beta | eta
    dx = F.linear(dz, side["wT"])
    dW = dz.t() @ x.reshape(b * T, D)
    lins = (mod.q_proj, mod.k_proj, mod.v_proj, mod.beta_proj, mod.eta_proj)
    off = 0
    for name, lin, width in zip(("q_proj", "k_proj", "v_proj", "beta_proj", "eta_proj"), lins, widths):
        grads[f"{name}.weight"] = dW[off:off + width]
        if lin.bias is not None:   # column sums of dz, accumulated in fp32 (no fp32 copy of dz)
            grads[f"{name}.bias"] = dz[:, off:off + width].sum(0, dtype=torch.float32)
        off += width
    grads["kappa"] = d_kappa
    # gamma = clamp(0.999 * sigmoid(log_gamma), 1e-3, 0.999); clamp passes its bounds inclusive
    sg = torch.sigmoid(mod.log_gamma.detach().float().to(dev))
    g0 = 0.999 * sg
    inside = ((g0 >= 1e-3) & (g0 <= 0.999)).float()
    grads["log_gamma"] = d_gam * 0.999 * sg * (1.0 - sg) * inside
    grads["res_norm.weight"] = o["d_res_w"].sum(dim=(0, 1))
    return dx.view(b, T, D), grads


class Bolt3Function(torch.autograd.Function):
    """Bolt3Attn.forward as one autograd node: the HIP forward keeps its trace, the backward is
    layer_backward.  Inputs: (module, x in the storage dtype, *parameters in named order)."""

    @staticmethod
    def forward(ctx, mod, x, *params):
        tr = {}
        out = mod._forward_hip(x, tr)
        ctx.mod, ctx.tr, ctx.dt = mod, tr, x.dtype
        ctx.names = [n for n, _ in mod.named_parameters()]
        ctx.save_for_backward(x)
        return out

    @staticmethod
    def backward(ctx, d_out):
        (x,) = ctx.saved_tensors
        dx, grads = layer_backward(ctx.mod, x, ctx.tr, d_out, ctx.dt)
        ctx.tr = None
        out = [None, dx.to(x.dtype)]
        for name, prm in zip(ctx.names, ctx.mod.parameters()):
            g = grads.get(name)
            out.append(None if g is None else g.to(prm.dtype).view_as(prm))
        return tuple(out)
