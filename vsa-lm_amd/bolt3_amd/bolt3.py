"""Bolt-3 Dual-Field attention on MI355X: drop-in ``Bolt3Attn`` / ``Bolt3Decoder``.

Mirrors the Python interface of vsa_lm/config/bolt3.py (reference tree):
constructor signatures, parameter / state-dict names, ``gamma_delta``,
``head_qkv``, ``_consolidate_functional`` and the decoder's ``step`` /
``prefill`` / ``generate_batch`` / ``generate`` / ``continue_generate`` /
``memorize`` / ``forget`` / ``blank_state`` / ``state_bytes`` / ``_sample``.

Everything between the input projections and ``o_proj`` runs in the HIP
kernels of libbolt3_amd.so (include/bolt3_amd.h), and so does the backward of
the attention and readout (backward.py replays the consolidation chain's
decisions for the rest of the gradient).  The projections are one
packed GEMM (q | k | v | beta | eta) through torch.  There is no CPU or eager
fallback: a CPU tensor or a missing library raises.

Numerics are those of the reference evaluated on CPU without autocast; when
the projection weights and the activations differ in dtype (bf16 projections
with fp32 Bolt-3 parameters) the projections run in the activation dtype, as
the reference's bf16 autocast runs them.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _abi as A
from .backward import Bolt3Function
from .layers import RMSNorm, RoPE

N_SINKS = 4


def _require_gpu(t: torch.Tensor, what: str):
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the Bolt-3 HIP path needs a ROCm device tensor (got {t.device}); "
                           f"there is no CPU implementation")


_N_CUS: dict = {}


def _n_cus(dev: torch.device) -> int:
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _N_CUS:
        _N_CUS[key] = torch.cuda.get_device_properties(key).multi_processor_count
    return _N_CUS[key]


# Per device: a counter that the slot-decision workgroups of the forward's first step group bump
# when they start, and the number of bumps issued so far.  The main stream waits on it
# (bolt3_wait_count) before the q projection, so that those workgroups, each needing a whole
# compute unit's LDS, are resident first instead of waiting for the GEMM's end.
_STARTED: dict = {}
WAIT_POLLS = 20000


def _started_counter(dev: torch.device) -> list:
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _STARTED:
        _STARTED[key] = [torch.zeros(1, dtype=torch.int32, device=dev), 0]
    return _STARTED[key]


def _wait_started(dev: torch.device, counter: torch.Tensor, target: int) -> None:
    rc = A.load().bolt3_wait_count(counter.data_ptr(), target & 0xFFFFFFFF, WAIT_POLLS, A.stream_of(dev))
    if rc != 0:
        raise RuntimeError(f"bolt3_wait_count failed with code {rc}")


# The forward's consolidation steps are issued in this many groups, so that the slot field and
# readout of early chunks run while the chain still decides later steps.
CHAIN_GROUPS = 3
# ... and at least one group per this many steps, so that the work left after the last group's
# slot decisions (its M_res updates, attention and o_proj) stays short on long sequences
GROUP_STEPS = 32


# The bf16 forward without a trace prepares the query heads (q RMSNorm, RoPE, the eta gate)
# inside the attention kernel from the q projection output (b3_attn_args.q_lin) instead of in a
# head-preparation pass of its own; both give the same bits.
FUSED_Q_PREP = True


def _n_groups(n_steps: int) -> int:
    return max(CHAIN_GROUPS, round(n_steps / GROUP_STEPS))


def _step_groups(n: int, k: int) -> list[tuple[int, int]]:
    """Split steps [0, n) into at most k contiguous ranges: a short first one (about
    n / (2k - 2) + 1 steps and at most n / k, so that the attention starts soon after the q
    projection, which runs beside it), the rest nearly equal."""
    k = max(1, min(k, n))
    if k == 1:
        return [(0, n)]
    first = max(1, min(n // k, (n + 1) // (2 * k - 2) + 1))
    rest = n - first
    bounds = [0, first] + [first + rest * i // (k - 1) for i in range(1, k)]
    return [(bounds[i], bounds[i + 1]) for i in range(k) if bounds[i + 1] > bounds[i]]


class _storage_dtype:
    """The dtype the kernels store activations in: the input's, or under autocast the autocast
    dtype (the projections then produce it, as the reference's linears do under autocast).
    Autocast is switched off inside, so every projection output has exactly this dtype."""

    def __init__(self, x: torch.Tensor):
        dev = x.device.type
        self.auto = torch.is_autocast_enabled(dev)
        self.dt = torch.get_autocast_dtype(dev) if self.auto else x.dtype
        self.ctx = torch.autocast(dev, enabled=False) if self.auto else None

    def __enter__(self):
        if self.ctx is not None:
            self.ctx.__enter__()
        return self.dt

    def __exit__(self, *exc):
        if self.ctx is not None:
            return self.ctx.__exit__(*exc)
        return False


def _check_dtype(t: torch.Tensor, dt: torch.dtype, what: str):
    if t.dtype != dt:
        raise TypeError(f"{what} is {t.dtype}, the kernels were told {dt}")


def _tout(t: torch.Tensor | None, offset: int = 0) -> A.TensorOut:
    """[B][heads][cap][HD] view with the token axis starting at ``offset``."""
    if t is None:
        return A.TensorOut(None, 0, 0)
    es = t.element_size()
    return A.TensorOut(t.data_ptr() + offset * t.shape[-1] * es, t.stride(0), t.stride(1))


def _gout(t: torch.Tensor | None, offset: int = 0) -> A.GateOut:
    if t is None:
        return A.GateOut(None, 0, 0)
    return A.GateOut(t.data_ptr() + offset * 4, t.stride(0), t.stride(1))


class Bolt3Attn(nn.Module):
    """Bolt-3 attention layer (vsa_lm/config/bolt3.py:23-276)."""

    def __init__(self, cfg: dict, max_T: int = 2048, S: int = 128, C: int = 128):
        super().__init__()
        D, H, HKV = int(cfg["dim"]), int(cfg["num_heads"]), int(cfg["num_kv_heads"])
        HD = int(cfg.get("head_dim") or (D // H))
        bias = bool(cfg.get("qkv_bias", False))
        self.H, self.HKV, self.HD, self.G = H, HKV, HD, H // HKV
        self.S, self.C, self.n_sinks = S, C, N_SINKS
        self.sim_k, self.sim_v, self.gamma_u = 0.88, 0.80, 0.995
        self.q_proj = nn.Linear(D, H * HD, bias=bias)
        self.k_proj = nn.Linear(D, HKV * HD, bias=bias)
        self.v_proj = nn.Linear(D, HKV * HD, bias=bias)
        self.o_proj = nn.Linear(H * HD, D, bias=False)
        if cfg.get("qk_norm", False):
            self.q_norm, self.k_norm = RMSNorm(HD, cfg["eps"]), RMSNorm(HD, cfg["eps"])
        else:
            self.q_norm = self.k_norm = None
        self.rope = RoPE(HD, cfg["rope_theta"], cfg.get("rope_scaling"))
        self.kappa = nn.Parameter(torch.ones(HKV))
        self.log_gamma = nn.Parameter(torch.full((HKV,), 3.5))
        self.beta_proj = nn.Linear(D, HKV, bias=True)
        nn.init.zeros_(self.beta_proj.weight)
        nn.init.constant_(self.beta_proj.bias, -1.0)
        self.eta_proj = nn.Linear(D, H, bias=True)
        nn.init.zeros_(self.eta_proj.weight)
        nn.init.zeros_(self.eta_proj.bias)
        self.res_norm = RMSNorm(HD, cfg["eps"])
        with torch.no_grad():
            self.res_norm.weight.fill_(0.05)
        self._pack_key = None
        self._pack = None

    # ------------------------------------------------------------ reference API

    def gamma_delta(self) -> torch.Tensor:
        return (0.999 * torch.sigmoid(self.log_gamma)).clamp(1e-3, 0.999).float()

    def head_qkv(self, x: torch.Tensor):
        """q, k, v heads after the optional q/k RMSNorm: [b,H,T,HD], [b,HKV,T,HD] x2."""
        b, t, _ = x.shape
        q = self.q_proj(x).view(b, t, self.H, self.HD)
        k = self.k_proj(x).view(b, t, self.HKV, self.HD)
        v = self.v_proj(x).view(b, t, self.HKV, self.HD)
        if self.q_norm is not None:
            q, k = self.q_norm(q), self.k_norm(k)
        return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)

    # ------------------------------------------------------------ packed parameters

    def _packed(self, dt: torch.dtype, device: torch.device):
        """(W_all, b_all, side) cached until a parameter changes.  W_all packs q | k | v | beta | eta
        rows (the decoder's one projection); side holds W_o, the split projections q, k | v and
        beta | eta used by the forward, and the fp32 tensors the kernels read."""
        # the parameters straight from the module dicts (one level of submodules), cheaper than
        # self.parameters() on the decode path, where this runs once per layer and token
        params = [q for q in self._parameters.values() if q is not None]
        params += [q for m in self._modules.values() if m is not None for q in m._parameters.values() if q is not None]
        key = (dt, device, tuple([(q.data_ptr(), q._version) for q in params]), self.rope.inv_freq.data_ptr())
        if key == self._pack_key:
            return self._pack
        with torch.no_grad():
            lins = (self.q_proj, self.k_proj, self.v_proj, self.beta_proj, self.eta_proj)
            # zero rows pad the packed output width to a multiple of 16 columns, so every row of
            # the projection output starts 16-byte aligned (the head kernels move 16-byte vectors)
            n_out = sum(m.out_features for m in lins)
            pad = (-n_out) % 16
            W = torch.cat([m.weight.to(device=device, dtype=dt) for m in lins] +
                          [torch.zeros(pad, self.q_proj.in_features, device=device, dtype=dt)], dim=0).contiguous()
            if any(m.bias is not None for m in lins):
                b = torch.cat([(m.bias if m.bias is not None else torch.zeros(m.out_features, device=device))
                               .to(device=device, dtype=dt) for m in lins] +
                              [torch.zeros(pad, device=device, dtype=dt)]).contiguous()
            else:
                b = None
            def pack(ms):
                w = [m.weight.to(device=device, dtype=dt) for m in ms]
                pd = (-sum(m.out_features for m in ms)) % 16
                w.append(torch.zeros(pd, self.q_proj.in_features, device=device, dtype=dt))
                bb = None
                if any(m.bias is not None for m in ms):
                    bb = torch.cat([(m.bias if m.bias is not None else torch.zeros(m.out_features, device=device))
                                    .to(device=device, dtype=dt) for m in ms] +
                                   [torch.zeros(pd, device=device, dtype=dt)]).contiguous()
                return torch.cat(w, dim=0).contiguous(), bb
            # the forward projects q, k | v and the gates beta | eta separately: q and k | v then
            # have 4096 and 2048 columns, widths the GEMM tiles divide
            wq, bq = pack((self.q_proj,))
            wkv, bkv = pack((self.k_proj, self.v_proj))
            wg, bg = pack((self.beta_proj, self.eta_proj))
            side = dict(
                wq=wq, bq=bq, wkv=wkv, bkv=bkv, wg=wg, bg=bg,
                wo=self.o_proj.weight.to(device=device, dtype=dt).contiguous(),
                inv_freq=self.rope.inv_freq.to(device).float().contiguous(),
                kappa=self.kappa.detach().to(device).float().contiguous(),
                res_w=self.res_norm.weight.detach().to(device).float().contiguous(),
                qn=None if self.q_norm is None else self.q_norm.weight.detach().to(device).float().contiguous(),
                kn=None if self.k_norm is None else self.k_norm.weight.detach().to(device).float().contiguous(),
                gamma=self.gamma_delta().detach().to(device).contiguous(),
            )
        self._pack = (W, b, side)
        self._pack_key = key
        return self._pack

    def _heads(self, lin, B, T, dt, side, pos0, q_raw, q_rope, k_raw, k_rope, v, beta, eta, pos_out=None,
               kv_offset=0, lin_kv=None, parts=0, gates=None, rope_cs=None):
        a = A.HeadsArgs()
        a.dtype, a.B, a.T, a.H, a.HKV, a.HD = A.dtype_code(dt), B, T, self.H, self.HKV, self.HD
        if lin is not None:
            a.lin, a.lin_row_stride = lin.data_ptr(), lin.shape[-1]
        if lin_kv is not None:
            a.lin_kv, a.lin_kv_row_stride = lin_kv.data_ptr(), lin_kv.shape[-1]
        a.parts = parts
        if gates is not None:
            a.gates, a.gates_row_stride = gates.data_ptr(), gates.shape[-1]
        a.qn_w, a.kn_w = A.ptr(side["qn"]), A.ptr(side["kn"])
        a.has_qk_norm = int(side["qn"] is not None)
        a.eps = float(self.res_norm.eps)
        a.inv_freq, a.pos0 = side["inv_freq"].data_ptr(), int(pos0)
        a.q_raw, a.q_rope = _tout(q_raw), _tout(q_rope)
        a.k_raw, a.k_rope, a.v = _tout(k_raw, kv_offset), _tout(k_rope, kv_offset), _tout(v, kv_offset)
        a.beta, a.eta = _gout(beta, kv_offset), _gout(eta)
        a.pos_out = None if pos_out is None else pos_out.data_ptr() + kv_offset * 4
        a.rope_cs = None if rope_cs is None else rope_cs.data_ptr()
        A.call("bolt3_heads", a, (lin if lin is not None else lin_kv).device)

    def _chain(self, dt, device, B, kr, kp, v, tok_bh_stride, pos, beta, beta_bh_stride, n_steps, off0, len0,
               step_stride, step_len, n_filled, st: dict, m_res, gam, side, snap_k=None, snap_v=None,
               snap_bias=None, snap_m=None, log=None, kp_exact=False, phase=0, work=None, started=None,
               snap_mass=None, snap_pm=None):
        if work is None:
            work = torch.empty(A.chain_workspace_bytes(dt, B, self.HKV, self.HD, self.S, n_steps),
                               dtype=torch.uint8, device=device)
        a = A.ChainArgs()
        a.dtype, a.B, a.HKV, a.HD, a.S = A.dtype_code(dt), B, self.HKV, self.HD, self.S
        a.kr, a.kp, a.v, a.tok_bh_stride = kr, kp, v, tok_bh_stride
        a.pos, a.beta, a.beta_bh_stride = pos, beta, beta_bh_stride
        a.n_steps, a.off0, a.len0, a.step_stride, a.step_len = n_steps, off0, len0, step_stride, step_len
        a.n_filled, a.kp_exact = n_filled, int(kp_exact)
        a.ak, a.av = st["ak"].data_ptr(), st["av"].data_ptr()
        a.mass, a.util, a.pm = st["mass"].data_ptr(), st["util"].data_ptr(), st["pm"].data_ptr()
        a.act, a.m_res = st["act"].data_ptr(), m_res.data_ptr()
        a.kappa, a.gamma, a.inv_freq = side["kappa"].data_ptr(), gam.data_ptr(), side["inv_freq"].data_ptr()
        a.snap_k, a.snap_v, a.snap_bias, a.snap_m = A.ptr(snap_k), A.ptr(snap_v), A.ptr(snap_bias), A.ptr(snap_m)
        a.log = A.ptr(log)
        a.snap_mass, a.snap_pm = A.ptr(snap_mass), A.ptr(snap_pm)
        a.work, a.work_bytes = work.data_ptr(), work.numel()
        a.phase, a.started = phase, started
        A.call("bolt3_chain", a, device)

    def _empty_slots(self, bh, dt, device):
        return dict(
            ak=torch.zeros(bh, self.S, self.HD, dtype=dt, device=device),
            av=torch.zeros(bh, self.S, self.HD, dtype=dt, device=device),
            mass=torch.ones(bh, self.S, device=device),
            util=torch.zeros(bh, self.S, device=device),
            pm=torch.zeros(bh, self.S, device=device),
            act=torch.zeros(bh, self.S, dtype=torch.uint8, device=device),
        )

    # ------------------------------------------------------------ forward

    def forward(self, x: torch.Tensor, _trace: dict | None = None) -> torch.Tensor:
        _require_gpu(x, "Bolt3Attn.forward")
        need_grad = torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))
        with _storage_dtype(x) as dt:
            if need_grad:
                # one autograd node: the forward keeps its trace, the backward runs bolt3_attn_bwd
                # and replays the consolidation chain (backward.py)
                return Bolt3Function.apply(self, x.to(dt), *self.parameters())
            return self._forward_hip(x.to(dt), _trace)

    @torch.no_grad()
    def _forward_hip(self, x: torch.Tensor, trace: dict | None, score_round: int = 1,
                     keep_log: bool = True) -> torch.Tensor:
        """The forward on the HIP path.  ``trace`` (a dict) receives the head tensors, the chain's
        final state and snapshots, the attention output and (keep_log) the decision log.
        score_round 1: q.k rounded to the storage dtype before scaling (the forward); 0: fp32
        scores (the decoder's step, used by its prefill)."""
        b, T, _ = x.shape
        dt, dev = x.dtype, x.device
        H, HKV, HD, S, C = self.H, self.HKV, self.HD, self.S, self.C
        x = x.contiguous()
        _, _, side = self._packed(dt, dev)
        gam = side["gamma"]
        main = torch.cuda.current_stream(dev)
        # k | v and the gates first: the consolidation chain needs only k, v and beta, so it runs
        # on side streams while the q projection, the q head preparation and the attention
        # proceed on this one.  The q projection is issued once the first step group's slot
        # decisions hold their compute units (bolt3_wait_count) and runs on the rest of the chip.
        lin_kv = F.linear(x, side["wkv"], side["bkv"])
        gates = F.linear(x, side["wg"], side["bg"])
        _check_dtype(lin_kv, dt, "k|v projection")
        _check_dtype(gates, dt, "gate projection")
        k_raw = torch.empty(b, HKV, T, HD, dtype=dt, device=dev)
        k_rope, v = torch.empty_like(k_raw), torch.empty_like(k_raw)
        beta = torch.empty(b, HKV, T, device=dev)
        pos = torch.empty(T, device=dev)
        n_chunks = (T + C - 1) // C
        n_cons = max(0, n_chunks - 2)
        bh = b * HKV
        snaps = (None, None, None, None)
        split = n_cons > 0 and dt == torch.bfloat16
        # bf16 without a trace: the attention prepares the query heads itself, from the q
        # projection output and the (cos, sin) table that the k head preparation writes
        fuse_q = split and trace is None and FUSED_Q_PREP and S == 128 and H // HKV in (1, 2, 4, 8)
        rope_cs = torch.empty(T, HD // 2, dtype=torch.int32, device=dev) if fuse_q else None
        self._heads(None, b, T, dt, side, 0, None, None, k_raw, k_rope, v, beta, None, pos_out=pos,
                    lin_kv=lin_kv, parts=2, gates=gates, rope_cs=rope_cs)

        # bf16: the chain's steps go out in groups; the slot decisions of a group run on one side
        # stream, its Gershgorin scales and M_res updates on another, and the main stream adds the
        # slot field and readout of a group's chunks as soon as that group is done
        groups = _step_groups(n_cons, _n_groups(n_cons) if split else 1) if n_cons > 0 else []
        done = []   # per group: event after its M_res updates
        # the first group's slot decisions hold their compute units before the q projection, a
        # GEMM whose grid covers the whole chip, is issued: otherwise most of them wait for its end
        ctr = _started_counter(dev) if split and 2 * b * HKV <= _n_cus(dev) else None
        first_started = None
        if n_cons > 0:
            s_dec = A.side_stream(dev, 0)
            s_m = A.side_stream(dev, 1) if split else s_dec
            # n_filled = 0: the chain builds the empty state itself, these are outputs only
            st = dict(ak=torch.empty(bh, S, HD, dtype=dt, device=dev), av=torch.empty(bh, S, HD, dtype=dt, device=dev),
                      mass=torch.empty(bh, S, device=dev), util=torch.empty(bh, S, device=dev),
                      pm=torch.empty(bh, S, device=dev), act=torch.empty(bh, S, dtype=torch.uint8, device=dev))
            m_res = torch.empty(bh, HD, HD, device=dev)
            snaps = (torch.empty(n_cons, bh, S, HD, dtype=dt, device=dev),
                     torch.empty(n_cons, bh, S, HD, dtype=dt, device=dev),
                     torch.empty(n_cons, bh, S, device=dev),
                     torch.empty(n_cons, bh, HD, HD, device=dev))
            ns = min(self.n_sinks, C)
            log = None
            if trace is not None and keep_log:
                log = torch.zeros(n_cons, bh, A.LOG_ROWS, A.LOG_COLS, device=dev)
            # the slots' mass and mean position after every step, for the backward
            snap_mp = (torch.empty(n_cons, bh, S, device=dev), torch.empty(n_cons, bh, S, device=dev)) \
                if trace is not None else None
            works = [torch.empty(A.chain_workspace_bytes(dt, b, HKV, HD, S, s1 - s0), dtype=torch.uint8, device=dev)
                     for s0, s1 in groups]
            s_dec.wait_stream(main)   # after the head preparation and the allocations above
            esz = k_raw.element_size()
            # filled slots before each group (they depend only on the token counts)
            nf_at, nf = [], 0
            for s0, s1 in groups:
                nf_at.append(nf)
                for i in range(s0, s1):
                    nf = min(S, nf + (C - ns if i == 0 else C))

            def issue_group(gi):
                s0, s1 = groups[gi]
                # step 0 takes the first chunk after its sinks; step i > 0 takes chunk i
                tok = s0 * C
                off0, len0 = (ns, C - ns) if s0 == 0 else (0, C)
                args = (dt, dev, b, k_raw.data_ptr() + tok * HD * esz, k_rope.data_ptr() + tok * HD * esz,
                        v.data_ptr() + tok * HD * esz, T * HD, pos.data_ptr() + tok * 4, beta.data_ptr() + tok * 4,
                        T, s1 - s0, off0, len0, C, C, nf_at[gi], st, m_res, gam, side,
                        *(t[s0:s1] for t in snaps))
                kw = dict(log=None if log is None else log[s0:s1], kp_exact=True, work=works[gi])
                if snap_mp is not None:
                    kw.update(snap_mass=snap_mp[0][s0:s1], snap_pm=snap_mp[1][s0:s1])
                started = None
                if split:
                    count = ctr is not None and s0 == 0
                    with torch.cuda.stream(s_dec):
                        self._chain(*args, phase=1, started=ctr[0].data_ptr() if count else None, **kw)
                    if count:
                        ctr[1] += bh
                        started = ctr[1]
                    s_m.wait_stream(s_dec)
                    with torch.cuda.stream(s_m):
                        self._chain(*args, phase=2, **kw)
                else:
                    with torch.cuda.stream(s_dec):
                        self._chain(*args, **kw)
                ev = torch.cuda.Event()
                ev.record(s_m)
                done.append(ev)
                return started

            # the first group goes out before the q projection and its head preparation, the
            # others after them (the main stream has work while the host issues them)
            first_started = issue_group(0)
            if trace is not None:
                trace.update(state=st, m_res=m_res, snap_k=snaps[0], snap_v=snaps[1], snap_bias=snaps[2],
                             snap_m=snaps[3], log=log, n_filled=nf, snap_mass=snap_mp[0], snap_pm=snap_mp[1])
        if first_started is not None:
            _wait_started(dev, ctr[0], first_started)
        lin_q = F.linear(x, side["wq"], side["bq"])
        _check_dtype(lin_q, dt, "q projection")
        if not fuse_q:
            q_raw = torch.empty(b, H, T, HD, dtype=dt, device=dev)
            q_rope = torch.empty_like(q_raw)
            eta = torch.empty(b, H, T, device=dev)
            self._heads(lin_q, b, T, dt, side, 0, q_raw, q_rope, None, None, None, None, eta, lin_kv=lin_kv,
                        parts=1, gates=gates)
        for gi in range(1, len(groups)):
            issue_group(gi)
        if trace is not None:
            trace.update(q_raw=q_raw, q_rope=q_rope, k_raw=k_raw, k_rope=k_rope, v=v, beta=beta, eta=eta, pos=pos,
                         lin_q=lin_q, lin_kv=lin_kv)

        K = H * HD
        a = A.AttnArgs()
        a.dtype, a.B, a.H, a.HKV, a.HD, a.S, a.C, a.n_sinks = A.dtype_code(dt), b, H, HKV, HD, S, C, self.n_sinks
        a.mode, a.n_q, a.score_round = 0, T, int(score_round)
        if fuse_q:
            a.q_lin, a.q_lin_stride = lin_q.data_ptr(), lin_q.shape[-1]
            a.qn_w, a.qn_eps = A.ptr(side["qn"]), float(self.res_norm.eps)
            a.rope_cs = rope_cs.data_ptr()
            a.gates, a.gates_stride, a.gates_col = gates.data_ptr(), gates.shape[-1], HKV
        else:
            a.q_rope, a.q_raw, a.q_sb, a.q_sh = q_rope.data_ptr(), q_raw.data_ptr(), q_rope.stride(0), q_rope.stride(1)
            a.eta, a.e_sb, a.e_sh = eta.data_ptr(), eta.stride(0), eta.stride(1)
        a.win_k, a.win_v, a.w_sb, a.w_sh = k_rope.data_ptr(), v.data_ptr(), k_rope.stride(0), k_rope.stride(1)
        if n_cons > 0:
            a.slot_k, a.slot_v, a.slot_bias = snaps[0].data_ptr(), snaps[1].data_ptr(), snaps[2].data_ptr()
            a.slot_step = bh * S * HD
            a.m_res, a.m_step = snaps[3].data_ptr(), bh * HD * HD
            a.m_split = int(dt == torch.bfloat16)
        a.gamma, a.res_w, a.eps = gam.data_ptr(), side["res_w"].data_ptr(), float(self.res_norm.eps)
        if split and trace is None:
            # Group by group, as soon as the chain has produced a group's snapshots: the attention
            # over all key fields of the group's chunks (the first group also takes chunks 0 and
            # 1) into one [B * rows, H * HD] block (the group's token range of every batch row),
            # then o_proj of that block as one GEMM, copied into place.  Only the last group's
            # attention and o_proj follow the chain's end.
            spans = [(0, min(T, (groups[0][1] + 2) * C))] + \
                    [(min(T, (s0 + 2) * C), min(T, (s1 + 2) * C)) for s0, s1 in groups[1:]]
            y_all = torch.empty(b * T * K, dtype=dt, device=dev)
            out = torch.empty(b, T, side["wo"].shape[0], dtype=dt, device=dev)
            esz, off = y_all.element_size(), 0
            a.part = 0
            for gi, ((s0, s1), ev) in enumerate(zip(groups, done)):
                t0, t1 = spans[gi]
                blk = y_all[off:off + b * (t1 - t0) * K].view(b * (t1 - t0), K)
                off += b * (t1 - t0) * K
                main.wait_event(ev)
                a.chunk_begin, a.chunk_end = (0 if gi == 0 else s0 + 2), s1 + 2
                # element (b, t) of the block at its base + (b * rows + t - t0) * K (the kernel
                # writes rows t >= t0 only)
                a.y, a.y_sb, a.y_st = blk.data_ptr() - t0 * K * esz, (t1 - t0) * K, K
                A.call("bolt3_chunk_attn", a, dev)
                if b == 1:   # the group's output rows are one contiguous slab of the result
                    torch.mm(blk, side["wo"].t(), out=out[0, t0:t1])
                else:
                    out[:, t0:t1].copy_(F.linear(blk, side["wo"]).view(b, t1 - t0, -1))
            return out
        # One [B, T, H * HD] attention output (the backward reads it), o_proj as one GEMM.  bf16:
        # group by group, as soon as the chain has produced a group's snapshots, one launch over
        # the group's chunks (the first group also takes chunks 0 and 1).
        y = torch.empty(b, T, K, dtype=dt, device=dev)
        a.y, a.y_sb, a.y_st = y.data_ptr(), y.stride(0), y.stride(1)
        if trace is not None:   # every query row's softmax normaliser, which the backward reuses
            trace["lse"] = torch.empty(b, H, T, device=dev)
            a.lse = trace["lse"].data_ptr()
        if not split:
            for ev in done:
                main.wait_event(ev)
            A.call("bolt3_chunk_attn", a, dev)
        else:
            a.part = 0
            for gi, ((s0, s1), ev) in enumerate(zip(groups, done)):
                main.wait_event(ev)
                a.chunk_begin, a.chunk_end = (0 if gi == 0 else s0 + 2), s1 + 2
                A.call("bolt3_chunk_attn", a, dev)
        if trace is not None:
            trace["y"] = y
        return F.linear(y, side["wo"])

    # ------------------------------------------------------------ consolidation (reference internal API)

    @torch.no_grad()
    def _consolidate_functional(self, ak, av, mass, util, pm, act, m_res, k_raw, k_rope, v_old, pos_old, beta_old,
                                inv_freq, diag_eye, gam, n_filled: int = 0):
        """One consolidation of the chunk (k_raw, k_rope, v_old, pos_old, beta_old) into the slot state;
        same arguments and 8-tuple result as vsa_lm/config/bolt3.py:68-192 (diag_eye is unused)."""
        _require_gpu(k_raw, "Bolt3Attn._consolidate_functional")
        b, hkv, l, hd = k_raw.shape
        bh, dt, dev = b * hkv, k_raw.dtype, k_raw.device
        if pos_old.dim() == 3 and (pos_old.shape[0] != 1 or pos_old.shape[1] != 1):
            if not torch.equal(pos_old, pos_old[:1, :1].expand_as(pos_old)):
                raise NotImplementedError("per-row token positions are not supported by the chain kernel")
        if ak is None:
            st = self._empty_slots(bh, dt, dev)
            m = torch.zeros(bh, hd, hd, device=dev)
            n_filled = 0
        else:
            st = dict(ak=ak.reshape(bh, self.S, hd).to(dt).contiguous().clone(),
                      av=av.reshape(bh, self.S, hd).to(dt).contiguous().clone(),
                      mass=mass.reshape(bh, self.S).float().contiguous().clone(),
                      util=util.reshape(bh, self.S).float().contiguous().clone(),
                      pm=pm.reshape(bh, self.S).float().contiguous().clone(),
                      act=act.reshape(bh, self.S).to(torch.uint8).contiguous().clone())
            m = m_res.reshape(bh, hd, hd).float().contiguous().clone()
        kr = k_raw.reshape(bh, l, hd).contiguous()
        kp = k_rope.reshape(bh, l, hd).to(dt).contiguous()
        vv = v_old.reshape(bh, l, hd).to(dt).contiguous()
        pos = pos_old.reshape(-1)[:l].float().contiguous() if pos_old.numel() == l else \
            pos_old.reshape(-1, l)[0].float().contiguous()
        bet = beta_old.reshape(bh, l).float().contiguous()
        side = dict(kappa=self.kappa.detach().to(dev).float().contiguous(),
                    inv_freq=inv_freq.to(dev).float().contiguous())
        self._chain(dt, dev, b, kr.data_ptr(), kp.data_ptr(), vv.data_ptr(), l * hd, pos.data_ptr(),
                    bet.data_ptr(), l, 1, 0, l, l, l, int(n_filled), st, m, gam.to(dev).float().contiguous(), side)
        nf = int(n_filled) + min(self.S - int(n_filled), l) if n_filled < self.S else int(n_filled)
        return st["ak"], st["av"], st["mass"], st["util"], st["pm"], st["act"].bool(), m, nf


def __getattr__(name):
    # the reference imports the decoder from the layer's module (vsa_lm.config.bolt3)
    if name in ("Bolt3Decoder", "Bolt3LayerState", "StaticKV", "AnchorCache"):
        from . import decoder
        return getattr(decoder, name)
    raise AttributeError(name)
