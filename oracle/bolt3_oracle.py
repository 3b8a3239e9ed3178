"""Bolt-3 Dual-Field attention: CPU restatement used as the parity oracle.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product (``vsa-lm_amd/bolt3_amd``) never imports it and has no CPU
path of its own.

What it restates
----------------
The reference implements Bolt-3 as plain PyTorch in
``vsa_lm/config/bolt3.py`` (reference tree).  This module re-expresses the
same arithmetic on CPU tensors, per (batch, kv-head) row ``bh``:

* ``rms_norm``            -- vsa_lm/surgery.py:43-53
* ``rope_inv_freq``       -- vsa_lm/surgery.py:56-72
* ``rope_at``             -- vsa_lm/config/bolt3.py:12-20, vsa_lm/surgery.py:86-93
* ``gamma_delta``         -- vsa_lm/config/bolt3.py:56-57
* ``project``             -- vsa_lm/config/bolt3.py:59-66, 196-199
* ``consolidate``         -- vsa_lm/config/bolt3.py:68-192 (fill and steady branches)
* ``forward``             -- vsa_lm/config/bolt3.py:194-276
* ``layer_step``          -- vsa_lm/config/bolt3.py:343-425 (Bolt-3 branch of Bolt3Decoder.step)
* ``HybridRef``           -- vsa_lm/config/bolt3.py:335-457 (model-level step/prefill) with the
                             softmax-anchor branch vsa_lm/config/bolt3.py:426-445 and
                             StaticKV vsa_lm/decode.py:88-106

Numerics
--------
The oracle is the reference's CPU semantics (no autocast).  To stay
bit-identical to the reference in fp32, every floating-point reduction is
issued as the same torch op on the same shapes as the reference (batched
``matmul`` over query heads after expanding kv heads, one-hot ``bmm`` for the
merge sums, ``F.normalize`` / ``F.cosine_similarity`` for cosines, ``topk``
for the two orderings).  Index bookkeeping (which slot/token goes where) is
written independently.  For a module whose linear weights have a different
dtype than the activations (bf16 projections + fp32 Bolt-3 parameters, the
layout real checkpoints use) the linears run in the activation dtype, which is
what the reference's bf16 autocast does to them; every other op keeps its
CPU dtype.

Pinning: tests/test_oracle_closed_form.py (closed forms, invariants, brute
force on small inputs) and tests/test_oracle_golden.py (vectors written by
tests/golden/make_golden.py from the reference itself).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

N_SINKS = 4
SIM_K = 0.88
SIM_V = 0.80
UTIL_DECAY = 0.995


# ----------------------------------------------------------------- primitives

def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """LlamaRMSNorm (vsa_lm/surgery.py:49-53): fp32 statistics, cast back to x's dtype."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * w.float()).to(x.dtype)


def rope_inv_freq(head_dim: int, theta: float, rope_scaling: dict | None = None) -> torch.Tensor:
    """Inverse RoPE frequencies theta^(-2i/HD) with the optional llama3 band scaling
    (vsa_lm/surgery.py:56-72)."""
    expo = torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim
    inv = 1.0 / (theta ** expo)
    if rope_scaling and rope_scaling.get("rope_type") == "llama3":
        ctx = float(rope_scaling["original_max_position_embeddings"])
        factor = float(rope_scaling["factor"])
        lo = float(rope_scaling["low_freq_factor"])
        hi = float(rope_scaling["high_freq_factor"])
        wl = 2.0 * math.pi / inv
        scaled = torch.where(wl > ctx / lo, inv / factor, inv)
        blend = (ctx / wl - lo) / (hi - lo)
        mixed = (1.0 - blend) * scaled / factor + blend * scaled
        mid = ~(wl < ctx / hi) & ~(wl > ctx / lo)
        inv = torch.where(mid, mixed, scaled)
    return inv


def rope_at(x: torch.Tensor, pos: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    """Rotate the last dim of ``x`` by angles pos*inv_freq.

    ``pos`` broadcasts against x.shape[:-1] and is taken as fp32; the angle is an
    fp32 product; cos/sin are rounded to x's dtype before use and the two
    products and the sum are separate ops (vsa_lm/config/bolt3.py:17-20,
    vsa_lm/surgery.py:86-93).
    """
    ang = pos.float().unsqueeze(-1) * inv_freq
    ang = torch.cat((ang, ang), dim=-1)
    half = x.shape[-1] // 2
    swapped = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * ang.cos().to(x.dtype) + swapped * ang.sin().to(x.dtype)


def gamma_delta(log_gamma: torch.Tensor) -> torch.Tensor:
    """M_res decay (vsa_lm/config/bolt3.py:56-57), evaluated in log_gamma's dtype."""
    return (0.999 * torch.sigmoid(log_gamma)).clamp(1e-3, 0.999).float()


def _select(x: torch.Tensor, k: int, largest: bool, ties: str):
    """Top-k along the last dim.  ties="torch": torch.topk, the reference's own call, whose
    order among exactly equal values is implementation-defined (introsort / nth_element on
    CPU).  ties="index": exact ties resolved by the lower index (a stable sort) -- the rule the
    HIP kernel uses.  Both put NaN first when largest and last otherwise."""
    if ties == "torch":
        return torch.topk(x, k=k, dim=-1, largest=largest)
    if ties != "index":
        raise ValueError(ties)
    v, i = torch.sort(x, dim=-1, descending=largest, stable=True)
    return v[..., :k], i[..., :k]


def _expand_kv(t: torch.Tensor, groups: int) -> torch.Tensor:
    """[b, hkv, n, d] -> [b, hkv*groups, n, d]; query head h reads kv head h // groups."""
    return t if groups == 1 else t.repeat_interleave(groups, dim=1)


# ----------------------------------------------------------------- parameters

@dataclass
class Bolt3Params:
    """Plain tensors of one Bolt-3 layer (state-dict names of vsa_lm/config/bolt3.py:33-54)."""
    D: int
    H: int
    HKV: int
    HD: int
    eps: float
    S: int
    C: int
    wq: torch.Tensor
    wk: torch.Tensor
    wv: torch.Tensor
    wo: torch.Tensor
    wb: torch.Tensor
    bb: torch.Tensor
    we: torch.Tensor
    be: torch.Tensor
    kappa: torch.Tensor
    log_gamma: torch.Tensor
    res_w: torch.Tensor
    inv_freq: torch.Tensor
    bq: torch.Tensor | None = None
    bk: torch.Tensor | None = None
    bv: torch.Tensor | None = None
    qn_w: torch.Tensor | None = None
    kn_w: torch.Tensor | None = None

    @property
    def G(self) -> int:
        return self.H // self.HKV

    @classmethod
    def from_module(cls, m) -> "Bolt3Params":
        """Read any module exposing the reference's Bolt3Attn attribute names."""
        sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
        eps = float(m.res_norm.eps)
        return cls(
            D=m.q_proj.weight.shape[1], H=m.H, HKV=m.HKV, HD=m.HD, eps=eps, S=m.S, C=m.C,
            wq=sd["q_proj.weight"], wk=sd["k_proj.weight"], wv=sd["v_proj.weight"],
            wo=sd["o_proj.weight"], wb=sd["beta_proj.weight"], bb=sd["beta_proj.bias"],
            we=sd["eta_proj.weight"], be=sd["eta_proj.bias"], kappa=sd["kappa"],
            log_gamma=sd["log_gamma"], res_w=sd["res_norm.weight"],
            inv_freq=m.rope.inv_freq.detach().cpu(),
            bq=sd.get("q_proj.bias"), bk=sd.get("k_proj.bias"), bv=sd.get("v_proj.bias"),
            qn_w=sd.get("q_norm.weight"), kn_w=sd.get("k_norm.weight"),
        )


def _lin(x, w, b=None):
    """Linear in the activation dtype (autocast rule for mixed-dtype checkpoints)."""
    return F.linear(x, w.to(x.dtype), None if b is None else b.to(x.dtype))


def project(p: Bolt3Params, x: torch.Tensor):
    """Heads and gates: q_raw [b,H,T,HD], k_raw/v [b,HKV,T,HD], beta [b,HKV,T], eta [b,H,T,1]
    (vsa_lm/config/bolt3.py:59-66, 198-199)."""
    b, t, _ = x.shape
    q = _lin(x, p.wq, p.bq).view(b, t, p.H, p.HD)
    k = _lin(x, p.wk, p.bk).view(b, t, p.HKV, p.HD)
    v = _lin(x, p.wv, p.bv).view(b, t, p.HKV, p.HD)
    if p.qn_w is not None:
        q, k = rms_norm(q, p.qn_w, p.eps), rms_norm(k, p.kn_w, p.eps)
    beta = torch.sigmoid(_lin(x, p.wb, p.bb)).transpose(1, 2)
    eta = torch.tanh(_lin(x, p.we, p.be)).transpose(1, 2).unsqueeze(-1)
    return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), beta, eta


# ----------------------------------------------------------------- slot state

@dataclass
class SlotState:
    """Attractor slots and M_res of every bh row; ak/av in the storage dtype (un-roped keys)."""
    ak: torch.Tensor      # [bh, S, HD]
    av: torch.Tensor      # [bh, S, HD]
    mass: torch.Tensor    # [bh, S] fp32
    util: torch.Tensor    # [bh, S] fp32
    pm: torch.Tensor      # [bh, S] fp32 (mean position of a slot)
    act: torch.Tensor     # [bh, S] bool
    m_res: torch.Tensor   # [bh, HD, HD] fp32
    n_filled: int = 0

    @classmethod
    def empty(cls, bh: int, S: int, HD: int, dtype) -> "SlotState":
        z = lambda *s, dt=torch.float32: torch.zeros(*s, dtype=dt)
        return cls(z(bh, S, HD, dt=dtype), z(bh, S, HD, dt=dtype), torch.ones(bh, S), z(bh, S),
                   z(bh, S), torch.zeros(bh, S, dtype=torch.bool), z(bh, HD, HD), 0)

    def clone(self) -> "SlotState":
        return SlotState(self.ak.clone(), self.av.clone(), self.mass.clone(), self.util.clone(),
                         self.pm.clone(), self.act.clone(), self.m_res.clone(), self.n_filled)


def slot_bias(p: Bolt3Params, st: SlotState, b: int) -> torch.Tensor:
    """Attention bias of the slots, kappa*log(max(mass,1)), -inf when inactive: [bh, S] fp32
    (vsa_lm/config/bolt3.py:238-241)."""
    kap = p.kappa.float().repeat(b).view(-1, 1)
    return (kap * torch.log(st.mass.clamp_min(1.0))).masked_fill(~st.act, float("-inf"))


def slot_keys(p: Bolt3Params, st: SlotState, b: int) -> torch.Tensor:
    return _slot_keys(p, st, b)


def _slot_keys(p: Bolt3Params, st: SlotState, b: int) -> torch.Tensor:
    """Attractor keys roped at their mean positions, [bh, S, HD] in storage dtype."""
    ak = st.ak.view(b, p.HKV, p.S, p.HD)
    return rope_at(ak, st.pm.view(b, p.HKV, p.S), p.inv_freq.view(1, 1, 1, -1)).view(b * p.HKV, p.S, p.HD)


def _retrieval(p, st, b, kp, v32, dt, bias, mask_inactive):
    """Softmax read of the slots by the chunk's roped keys -> rel_err per token
    (vsa_lm/config/bolt3.py:100-103 and :170-174)."""
    k_read = _slot_keys(p, st, b)
    sc = torch.bmm(kp, k_read.transpose(-1, -2)).float() * (p.HD ** -0.5) + bias
    if mask_inactive:
        sc.masked_fill_(~st.act.unsqueeze(1), -1e9)
    v_hat = torch.bmm(F.softmax(sc, dim=-1).to(dt), st.av).float()
    return (v32 - v_hat).norm(dim=-1) / (v32.norm(dim=-1) + 1e-6)


def consolidate(p: Bolt3Params, st: SlotState | None, kr, kp, v, pos, beta, gam, b: int,
                log: dict | None = None, ties: str = "torch", force: dict | None = None) -> SlotState:
    """One consolidation of a chunk that left the window (vsa_lm/config/bolt3.py:68-192).

    kr/kp/v: [bh, l, HD] storage dtype (un-roped, roped keys, values); pos: [l] or
    [bh, l] fp32 positions; beta: [bh, l]; gam: [HKV] fp32.  Returns the new state.
    ``log`` (optional dict) receives the per-token / per-slot decisions; ``ties`` selects
    the order among exactly equal scores (see ``_select``).

    ``force`` imposes another implementation's decisions (see ``decisions_from_log``): fill
    ``picked`` [bh, m] (slot n_filled + i takes token picked[:, i]); steady ``slot``, ``merge``
    [bh, l] and the replacements ``top_toks``, ``bot_slots``, ``win`` [bh, min(l, S)] (token
    top_toks[:, i] replaces slot bot_slots[:, i] where win[:, i]).  Every value is still computed
    here; only which tokens go where is taken from ``force``.  ``log`` then holds this oracle's
    own decisions from the same state, each stage given the forced stages before it: the merge
    decisions from the state before the step, the replacements from the state after the forced
    merges.
    """
    bh, l, hd = kr.shape
    dt = kr.dtype
    S = p.S
    posf = pos.float().expand(bh, l) if pos.dim() == 1 else pos.float().reshape(bh, l)
    if st is None:
        st = SlotState.empty(bh, S, hd, dt)
    else:
        st = st.clone()
    st.util = st.util * UTIL_DECAY
    v32 = v.float()
    rows = torch.arange(bh).unsqueeze(1)

    if st.n_filled < S:
        # ---- fill: copy the best tokens into the next free slots
        with torch.no_grad():
            m = min(S - st.n_filled, l)
            if st.n_filled > 0:
                bias = torch.log(st.mass.clamp_min(1.0)).unsqueeze(1)
                rel = _retrieval(p, st, b, kp, v32, dt, bias, mask_inactive=True)
                cos = torch.bmm(F.normalize(kr.float(), dim=-1),
                                F.normalize(st.ak.float(), dim=-1).transpose(-1, -2))
                cos.masked_fill_(~st.act.unsqueeze(1), 0.0)
                score = rel * (1.0 - cos.max(dim=-1).values.clamp(0.0, 1.0))
                init_u = rel
            else:
                score = F.normalize(v32, dim=-1).var(dim=-1)
                init_u = torch.full((bh, l), 0.15)
            picked = _select(score, m, True, ties)[1]                          # [bh, m]
        own_picked = picked
        if force is not None:
            picked = force["picked"][:, :m].long()
        slots = torch.arange(st.n_filled, st.n_filled + m).expand(bh, m)
        st.ak[rows, slots] = kr[rows, picked]
        st.av[rows, slots] = v[rows, picked]
        st.pm[rows, slots] = posf[rows, picked]
        st.mass[rows, slots] = 1.0
        st.util[rows, slots] = init_u[rows, picked]
        st.act[rows, slots] = True
        if log is not None:
            log.update(kind="fill", picked=own_picked.clone(), score=score.clone())
        st.n_filled += m
        return st

    # ---- steady: score -> merge -> evict/replace -> delta-rule write of the rest
    kap = p.kappa.float().repeat(b).view(bh, 1, 1)
    with torch.no_grad():
        rel = _retrieval(p, st, b, kp, v32, dt, kap * torch.log(st.mass.clamp_min(1.0)).unsqueeze(1),
                         mask_inactive=False)
        kn = F.normalize(kr.float(), dim=-1)
        cos = torch.bmm(kn, F.normalize(st.ak.float(), dim=-1).transpose(-1, -2))
        best, slot = cos.max(dim=-1)
        partner = st.av.float()[rows, slot]
        sim_v = F.cosine_similarity(v32, partner, dim=-1)
        score = rel * (1.0 - best.clamp(0.0, 1.0))
        merge = (best >= SIM_K) & (sim_v >= SIM_V)
        own = dict(slot=slot, merge=merge)
        if force is not None:
            slot, merge = force["slot"][:, :l].long(), force["merge"][:, :l].bool()

    # merge: mass-weighted means of the slot and the tokens assigned to it
    onehot = F.one_hot(slot, num_classes=S).float() * merge.float().unsqueeze(-1)   # [bh, l, S]
    cnt = onehot.sum(dim=1)
    sel = onehot.transpose(1, 2)
    k_acc = torch.bmm(sel, kr.float())
    v_acc = torch.bmm(sel, v32)
    p_acc = torch.bmm(sel, posf.unsqueeze(-1)).squeeze(-1)
    hit = cnt > 0
    m_new = st.mass + cnt
    mk = st.mass.unsqueeze(-1)
    st.ak = torch.where(hit.unsqueeze(-1), ((mk * st.ak.float() + k_acc) / m_new.unsqueeze(-1)).to(dt), st.ak)
    st.av = torch.where(hit.unsqueeze(-1), ((mk * st.av.float() + v_acc) / m_new.unsqueeze(-1)).to(dt), st.av)
    st.pm = torch.where(hit, (st.mass * st.pm + p_acc) / m_new, st.pm)
    st.mass = torch.where(hit, m_new, st.mass)

    # eviction: best non-merged tokens against the least useful (most redundant) slots
    with torch.no_grad():
        an = F.normalize(st.ak.float(), dim=-1)
        pair = torch.bmm(an, an.transpose(-1, -2))
        pair.diagonal(dim1=1, dim2=2).fill_(-1.0)
        keep = st.util * (1.0 - pair.max(dim=-1).values.clamp(0.0, 0.98))
        cand = torch.where(merge, torch.full_like(score, -1e9), score)
        kc = min(l, S)
        tv, tj = _select(cand, kc, True, ties)
        bv, bs = _select(keep, kc, False, ties)
        win = (tv > bv) & (tv > -1e8)
        own.update(top_toks=tj, bot_slots=bs, win=win)
        if force is not None:
            tj, bs, win = force["top_toks"][:, :kc].long(), force["bot_slots"][:, :kc].long(), force["win"][:, :kc].bool()
        inserted = torch.zeros(bh, l, dtype=torch.bool)
        inserted[rows, tj] = win
        to_delta = (~merge) & (~inserted)

    r_w, s_w = rows.expand_as(bs)[win], bs[win]
    t_w = tj[win]
    st.ak[r_w, s_w] = kr[r_w, t_w]
    st.av[r_w, s_w] = v[r_w, t_w]
    st.pm[r_w, s_w] = posf[r_w, t_w]
    st.mass[r_w, s_w] = 1.0
    st.util[r_w, s_w] = rel[r_w, t_w]

    # Gershgorin-safe delta rule into M_res; the normalised keys are taken again outside no_grad,
    # as the reference does (vsa_lm/config/bolt3.py:157): gradients reach kr through this rule
    kn = F.normalize(kr.float(), dim=-1)
    w = beta.float() * to_delta.float()
    gram = torch.bmm(kn, kn.transpose(-1, -2)).abs()
    rowsum = torch.bmm(gram, w.unsqueeze(-1)).squeeze(-1).clamp_min(1.0)
    bsafe = (w / rowsum).unsqueeze(-1)
    err = (v32 - torch.bmm(kn, st.m_res)) * bsafe
    st.m_res = gam.repeat(b).view(bh, 1, 1) * st.m_res + torch.bmm(kn.transpose(1, 2), err)

    if log is not None:
        own_ins = torch.zeros(bh, l, dtype=torch.bool)
        own_ins[rows, own["top_toks"]] = own["win"]
        log.update(kind="steady", best=best.clone(), slot=own["slot"].clone(), sim_v=sim_v.clone(),
                   best2=cos.topk(2, dim=-1).values[..., 1].clone(),
                   rel=rel.clone(), score=score.clone(), merge=own["merge"].clone(), keep=keep.clone(),
                   top_vals=tv.clone(), top_toks=own["top_toks"].clone(), bot_vals=bv.clone(),
                   bot_slots=own["bot_slots"].clone(), win=own["win"].clone(),
                   delta=((~merge) & (~own_ins)).clone(), delta_applied=to_delta.clone())
    return st


# ----------------------------------------------------------------- attention

def _readout(p, q_raw_c, m_res, eta_c, gam, b, tc):
    """η ⊙ RMSNorm(normalize(q_raw)·M_res·(1-γ)/√HD) (vsa_lm/config/bolt3.py:251-256)."""
    qn = F.normalize(q_raw_c.reshape(b, p.HKV, p.G, tc, p.HD).float(), dim=-1)
    ym = torch.einsum("bhgtc,bhcd->bhgtd", qn, m_res.view(b, p.HKV, p.HD, p.HD))
    ym = ym * ((1.0 - gam).view(1, p.HKV, 1, 1, 1) / (p.HD ** 0.5))
    return eta_c * rms_norm(ym.reshape(b, p.H, tc, p.HD), p.res_w, p.eps)


def _fields(p, qp, scale, sinks, st, b, win_k, win_v, mask, fp32_scores):
    """Joint softmax over [sinks | attractors | window] and the value read.

    fp32_scores=False: scores are rounded to the storage dtype before scaling
    (forward, vsa_lm/config/bolt3.py:226-249); True: scores computed in fp32
    (decoder step, vsa_lm/config/bolt3.py:372-396).
    """
    G = p.G
    qs = qp.float() if fp32_scores else qp

    def score(keys):
        kk = _expand_kv(keys, G)
        kk = kk.float() if fp32_scores else kk
        s = torch.matmul(qs, kk.transpose(-1, -2))
        return (s if fp32_scores else s.float()) * scale

    parts, vals = [], []
    if sinks is not None:
        parts.append(score(sinks[0]))
        vals.append(_expand_kv(sinks[1], G))
    if st is not None:
        keys = _slot_keys(p, st, b).view(b, p.HKV, p.S, p.HD)
        s_att = score(keys)
        kap = p.kappa.float().view(1, p.HKV, 1, 1)
        bias = _expand_kv(kap * torch.log(st.mass.view(b, p.HKV, 1, p.S).clamp_min(1.0)), G)
        act = _expand_kv(st.act.view(b, p.HKV, 1, p.S), G)
        parts.append((s_att + bias).masked_fill(~act, float("-inf")))
        vals.append(_expand_kv(st.av.view(b, p.HKV, p.S, p.HD), G))
    s_win = score(win_k)
    if mask is not None:
        s_win = s_win.masked_fill(~mask, float("-inf"))
    parts.append(s_win)
    vals.append(_expand_kv(win_v, G))
    sc = torch.cat(parts, dim=-1) if len(parts) > 1 else parts[0]
    vv = torch.cat(vals, dim=2) if len(vals) > 1 else vals[0]
    return torch.matmul(F.softmax(sc, dim=-1).to(vv.dtype), vv)


@dataclass
class ForwardTrace:
    states: list = field(default_factory=list)   # SlotState after each consolidation
    logs: list = field(default_factory=list)     # decision log of each consolidation
    chunks: list = field(default_factory=list)   # (kr, kp, v, pos, beta) consolidated, [bh, l, HD]
    y_pre: torch.Tensor | None = None            # attention + readout before o_proj, [b, H, T, HD]
    heads: tuple | None = None                   # (q_raw, q_rope, k_raw, k_rope, v, beta, eta)


def forward(p: Bolt3Params, x: torch.Tensor, trace: ForwardTrace | None = None, ties: str = "torch",
            decisions=None) -> torch.Tensor:
    """Bolt3Attn.forward (vsa_lm/config/bolt3.py:194-276).  Returns [b, T, D].

    ``decisions``: optional sequence, one entry per consolidation step (``force`` of
    ``consolidate``, or None to decide freely), imposing another implementation's slot decisions
    so that its whole output can be compared with this arithmetic along its own trajectory."""
    b, T, _ = x.shape
    q_raw, k_raw, v_all, beta_all, eta_all = project(p, x)
    q_rope = rope_at(q_raw, torch.arange(T, dtype=torch.float32), p.inv_freq)
    k_rope = rope_at(k_raw, torch.arange(T, dtype=torch.float32), p.inv_freq)
    gam = gamma_delta(p.log_gamma)
    scale = p.HD ** -0.5
    bh = b * p.HKV
    flat = lambda t: t.reshape(bh, t.shape[2], -1) if t.dim() == 4 else t.reshape(bh, t.shape[2])

    sinks = st = None
    prev = None            # (start, end) of the chunk held as "prev"
    ys = []
    n_done = 0
    for s0 in range(0, T, p.C):
        e0 = min(T, s0 + p.C)
        tc = e0 - s0
        lo = prev[0] if prev is not None else s0
        plen = s0 - lo
        qi = torch.arange(tc)[:, None]
        kj = torch.arange(e0 - lo)[None, :]
        mask = (kj <= plen + qi).view(1, 1, tc, -1)
        yc = _fields(p, q_rope[:, :, s0:e0], scale, sinks, st, b, k_rope[:, :, lo:e0],
                     v_all[:, :, lo:e0], mask, fp32_scores=False)
        if st is not None:
            yc = yc + _readout(p, q_raw[:, :, s0:e0], st.m_res, eta_all[:, :, s0:e0], gam, b, tc).to(yc.dtype)
        ys.append(yc)

        if tc == p.C and e0 < T:
            if prev is not None:
                a, z = prev
                if sinks is None:
                    ns = min(N_SINKS, z - a)
                    sinks = (k_rope[:, :, a:a + ns], v_all[:, :, a:a + ns])
                    a += ns
                chunk = (flat(k_raw[:, :, a:z]), flat(k_rope[:, :, a:z]), flat(v_all[:, :, a:z]),
                         torch.arange(a, z, dtype=torch.float32), flat(beta_all[:, :, a:z]))
                log = {} if trace is not None else None
                force = decisions[n_done] if decisions is not None else None
                st = consolidate(p, st, *chunk, gam, b, log=log, ties=ties, force=force)
                n_done += 1
                if trace is not None:
                    trace.states.append(st.clone())
                    trace.logs.append(log)
                    trace.chunks.append(chunk)
            prev = (s0, e0)

    y = torch.cat(ys, dim=2)
    if trace is not None:
        trace.y_pre = y
        trace.heads = (q_raw, q_rope, k_raw, k_rope, v_all, beta_all, eta_all)
    return F.linear(y.transpose(1, 2).reshape(b, T, p.H * p.HD), p.wo.to(y.dtype))


# Reference parameter names of the Bolt3Params fields (vsa_lm/config/bolt3.py:24-54)
PARAM_NAMES = dict(wq="q_proj.weight", bq="q_proj.bias", wk="k_proj.weight", bk="k_proj.bias",
                   wv="v_proj.weight", bv="v_proj.bias", wo="o_proj.weight", wb="beta_proj.weight",
                   bb="beta_proj.bias", we="eta_proj.weight", be="eta_proj.bias", kappa="kappa",
                   log_gamma="log_gamma", res_w="res_norm.weight", qn_w="q_norm.weight", kn_w="k_norm.weight")


def forward_grads(p: Bolt3Params, x: torch.Tensor, upstream: torch.Tensor, ties: str = "torch"):
    """Gradients of sum(forward(x) * upstream) with respect to x and every parameter, by autograd
    through this restatement of the forward (the reference's own backward: its slot selection
    runs under no_grad, vsa_lm/config/bolt3.py:98-112, :121-135, :165-180, and the gradients
    follow the forward's decisions).  Returns (y, {"x": dx, reference name: grad}); parameters
    the forward does not reach get zeros, like the reference's zero-weighted term (:257-258)."""
    leaves = {}
    for f_name in PARAM_NAMES:
        t = getattr(p, f_name)
        if t is not None:
            leaves[f_name] = t.detach().clone().requires_grad_(True)
    q = Bolt3Params(**{**p.__dict__, **leaves})
    xg = x.detach().clone().requires_grad_(True)
    y = forward(q, xg, ties=ties)
    (y * upstream.to(y.dtype)).sum().backward()
    out = {"x": xg.grad}
    for f_name, t in leaves.items():
        out[PARAM_NAMES[f_name]] = t.grad if t.grad is not None else torch.zeros_like(t)
    return y.detach(), out


# ----------------------------------------------------------------- decoder

@dataclass
class LayerCache:
    """Per-layer decoder state of one Bolt-3 layer (vsa_lm/config/bolt3.py:310-315)."""
    st: SlotState | None = None
    sinks: tuple | None = None
    prev: tuple | None = None   # (kr, kp, v, pos[1,1,n], beta) along dim 2
    cur: tuple | None = None


def layer_step(p: Bolt3Params, h: torch.Tensor, pos_start: int, m_state: torch.Tensor, cache: LayerCache,
               log: list | None = None, ties: str = "torch", force=None):
    """Bolt-3 branch of Bolt3Decoder.step for one layer (vsa_lm/config/bolt3.py:343-425).

    h: normed input [b, t, D].  m_state: M_res [b, HKV, HD, HD] fp32.  Returns
    (attention output before o_proj [b, H, t, HD], o_proj output [b, t, D], new m_state).
    ``cache`` is updated in place.  ``force``: a callable returning the decisions to impose on
    the consolidation this step runs (``force`` of ``consolidate``), called only when one runs.
    """
    b, t, _ = h.shape
    q_r, k_r, v_n, beta_n, eta_n = project(p, h)
    pos_n = torch.arange(pos_start, pos_start + t, dtype=torch.float32)
    q_p = rope_at(q_r, pos_n, p.inv_freq)
    k_p = rope_at(k_r, pos_n, p.inv_freq)
    gam = gamma_delta(p.log_gamma)
    scale = p.HD ** -0.5
    new = (k_r, k_p, v_n, pos_n[None, None, :], beta_n)
    before = 0 if cache.cur is None else cache.cur[1].shape[2]
    cache.cur = new if cache.cur is None else tuple(torch.cat([a, c], dim=2) for a, c in zip(cache.cur, new))
    if cache.prev is not None:
        wk = torch.cat([cache.prev[1], cache.cur[1]], dim=2)
        wv = torch.cat([cache.prev[2], cache.cur[2]], dim=2)
        plen = cache.prev[1].shape[2]
    else:
        wk, wv, plen = cache.cur[1], cache.cur[2], 0
    mask = None
    if t > 1:
        qi = torch.arange(t)[:, None]
        kj = torch.arange(wk.shape[2])[None, :]
        mask = (kj <= plen + before + qi).view(1, 1, t, -1)
    y = _fields(p, q_p, scale, cache.sinks, cache.st, b, wk, wv, mask, fp32_scores=True)
    y = y + _readout(p, q_r, m_state.view(b * p.HKV, p.HD, p.HD), eta_n, gam, b, t).to(y.dtype)
    out = F.linear(y.transpose(1, 2).reshape(b, t, p.H * p.HD), p.wo.to(y.dtype))

    if cache.cur[1].shape[2] >= p.C:
        if cache.prev is not None:
            kr_, kp_, v_, pos_, b_ = cache.prev
            if cache.sinks is None:
                ns = min(N_SINKS, kp_.shape[2])
                cache.sinks = (kp_[:, :, :ns].clone(), v_[:, :, :ns].clone())
                kr_, kp_, v_, pos_, b_ = kr_[:, :, ns:], kp_[:, :, ns:], v_[:, :, ns:], pos_[:, :, ns:], b_[:, :, ns:]
            bh, n = b * p.HKV, kr_.shape[2]
            st_in = cache.st
            if st_in is not None:
                st_in = st_in.clone()
                st_in.m_res = m_state.reshape(bh, p.HD, p.HD).clone()
            lg = {} if log is not None else None
            cache.st = consolidate(p, st_in, kr_.reshape(bh, n, p.HD), kp_.reshape(bh, n, p.HD),
                                   v_.reshape(bh, n, p.HD), pos_.reshape(n), b_.reshape(bh, n), gam, b, log=lg,
                                   ties=ties, force=None if force is None else force())
            if log is not None:
                log.append(lg)
            m_state = cache.st.m_res.view(b, p.HKV, p.HD, p.HD)
        cache.prev, cache.cur = cache.cur, None
    return y, out, m_state


class HybridRef:
    """Model-level decoder step over a hybrid stack of Bolt-3 and softmax-anchor layers
    (vsa_lm/config/bolt3.py:335-457).  ``model`` is any object with the reference's
    UniversalVSALM attribute names (embed_tokens, blocks[i].{norm1,norm2,mlp,vsa|attn},
    norm, lm_head)."""

    def __init__(self, model, C: int = 128, ties: str = "torch", logs: dict | None = None,
                 decisions: dict | None = None):
        self.model = model
        self.C = C
        self.ties = ties
        self.logs = logs            # optional {layer: [decision log of each consolidation]}
        # optional {layer: [decisions to impose on each consolidation, in order]} (consolidate's
        # ``force``): the oracle then follows another implementation's trajectory
        self.decisions = decisions
        self._n_forced: dict = {}
        self.params = {}
        for li, blk in enumerate(model.blocks):
            if hasattr(blk, "vsa"):
                self.params[li] = Bolt3Params.from_module(blk.vsa)

    def _next_forced(self, li: int):
        i = self._n_forced.get(li, 0)
        self._n_forced[li] = i + 1
        seq = self.decisions[li]
        if i >= len(seq):
            raise IndexError(f"layer {li}: consolidation {i} has no decisions to impose ({len(seq)} given)")
        return seq[i]

    def blank(self, b: int):
        st = {}
        for li, blk in enumerate(self.model.blocks):
            if li in self.params:
                p = self.params[li]
                st[li] = [torch.zeros(b, p.HKV, p.HD, p.HD), LayerCache()]
            else:
                st[li] = [None, None]       # softmax anchor: (k, v) concatenated along time
        return st

    @torch.no_grad()
    def step(self, tokens: torch.Tensor, pos_start: int, state: dict):
        m = self.model
        b, t = tokens.shape
        x = m.embed_tokens(tokens)
        for li, blk in enumerate(m.blocks):
            h = blk.norm1(x)
            if li in self.params:
                ms, cache = state[li]
                lg = None if self.logs is None else self.logs.setdefault(li, [])
                fc = None
                if self.decisions is not None and li in self.decisions:
                    fc = (lambda li=li: self._next_forced(li))
                _, out, ms = layer_step(self.params[li], h, pos_start, ms, cache, log=lg, ties=self.ties, force=fc)
                state[li][0] = ms
                x = x + out
            else:
                ly = blk.attn
                q, k, v = ly.head_qkv(h)
                q, k = ly.rope(q, pos_start=pos_start), ly.rope(k, pos_start=pos_start)
                kc, vc = state[li]
                n_prev = 0 if kc is None else kc.shape[2]
                kc = k if kc is None else torch.cat([kc, k], dim=2)
                vc = v if vc is None else torch.cat([vc, v], dim=2)
                state[li] = [kc, vc]
                if t > 1:
                    qi = torch.arange(t)[:, None]
                    kj = torch.arange(n_prev + t)[None, :]
                    msk = (kj <= (n_prev + qi)).view(1, 1, t, n_prev + t)
                    y = F.scaled_dot_product_attention(q, kc.to(q.dtype), vc.to(q.dtype), attn_mask=msk,
                                                       enable_gqa=(ly.G > 1))
                else:
                    y = F.scaled_dot_product_attention(q, kc.to(q.dtype), vc.to(q.dtype), enable_gqa=(ly.G > 1))
                x = x + ly.o_proj(y.transpose(1, 2).reshape(b, t, ly.H * ly.HD))
            x = x + blk.mlp(blk.norm2(x))
        return m.norm(x)

    @torch.no_grad()
    def prefill(self, ids: torch.Tensor):
        state = self.blank(ids.shape[0])
        h = None
        for s0 in range(0, ids.shape[1], self.C):
            h = self.step(ids[:, s0:s0 + self.C], s0, state)
        return h, state

    # -------------------------------------------------------------- generation and memory (checkers)

    @torch.no_grad()
    def logits(self, h: torch.Tensor) -> torch.Tensor:
        return self.model.lm_head(h[:, -1])

    @torch.no_grad()
    def generate_greedy(self, ids: torch.Tensor, n_new: int, eos_ids=None, close_think_ids=None):
        """Bolt3Decoder.generate_batch at temperature 0 (vsa_lm/config/bolt3.py:459-500), one token at a
        time with the reference's per-row rules: eos rows keep their first eos position as length;
        from the budget point max(64, n_new - 64) every row still thinking (not closed, not done)
        is forced through close_think_ids; a row counts as closed after the forced sequence or when
        it emits close_think_ids[1]; every 16 tokens the loop stops if all rows are done.
        Returns (tokens [B, n], lengths [B], the top-2 logit gap of each step [n])."""
        B, T = ids.shape
        h, state = self.prefill(ids)
        lg = self.logits(h)
        close = list(close_think_ids or ())
        eos = set(eos_ids or ())
        done, closed = [False] * B, [False] * B
        lengths, cursor = [n_new] * B, [-1] * B
        budget = max(64, n_new - 64)
        toks, gaps = [], []
        for i in range(n_new):
            top2 = lg.float().topk(2, dim=-1).values
            gaps.append(float((top2[:, 0] - top2[:, 1]).min()))
            nxt = lg.argmax(dim=-1).tolist()
            if close:
                if i == budget:
                    for r in range(B):
                        if not closed[r] and not done[r] and cursor[r] < 0:
                            cursor[r] = 0
                for r in range(B):
                    if cursor[r] >= 0:
                        nxt[r] = close[cursor[r]]
                        cursor[r] += 1
                        if cursor[r] >= len(close):
                            cursor[r], closed[r] = -1, True
                if len(close) > 1:
                    for r in range(B):
                        closed[r] = closed[r] or nxt[r] == close[1]
            toks.append(nxt)
            if eos:
                for r in range(B):
                    if not done[r] and nxt[r] in eos:
                        lengths[r], done[r] = i + 1, True
                if i % 16 == 15 and all(done):
                    break
            h = self.step(torch.tensor(nxt).view(B, 1), T + i, state)
            lg = self.logits(h)
        return torch.tensor(toks).T.contiguous(), torch.tensor(lengths), gaps

    @torch.no_grad()
    def memorize(self, ids: torch.Tensor, state: dict, start_pos: int):
        """Bolt3Decoder.memorize (vsa_lm/config/bolt3.py:528-546): feed ids in chunks of C, then per
        Bolt-3 layer the trace (end position, M_after - gamma^(len // C) * M_before)."""
        before = {li: st[0].clone() for li, st in state.items() if li in self.params}
        pos = start_pos
        for s0 in range(0, ids.shape[1], self.C):
            part = ids[:, s0:s0 + self.C]
            self.step(part, pos, state)
            pos += part.shape[1]
        traces = {}
        for li, m0 in before.items():
            g = gamma_delta(self.params[li].log_gamma).view(1, -1, 1, 1)
            traces[li] = (pos, state[li][0] - g ** (ids.shape[1] // self.C) * m0)
        return pos, traces

    def forget(self, traces: dict, state: dict, next_pos: int):
        """Bolt3Decoder.forget (vsa_lm/config/bolt3.py:548-557): subtract each trace decayed by gamma
        once per C positions since its end."""
        for li, (end, delta) in traces.items():
            g = gamma_delta(self.params[li].log_gamma).view(1, -1, 1, 1)
            state[li][0] = state[li][0] - g ** max(0, (next_pos - end) // self.C) * delta

