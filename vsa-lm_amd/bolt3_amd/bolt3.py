"""Bolt-3 Dual-Field attention on MI355X: drop-in ``Bolt3Attn`` / ``Bolt3Decoder``.

Mirrors the Python interface of vsa_lm/config/bolt3.py (reference tree):
constructor signatures, parameter / state-dict names, ``gamma_delta``,
``head_qkv``, ``_consolidate_functional`` and the decoder's ``step`` /
``prefill`` / ``generate_batch`` / ``generate`` / ``continue_generate`` /
``memorize`` / ``forget`` / ``blank_state`` / ``state_bytes`` / ``_sample``.

Everything between the input projections and ``o_proj`` runs in the HIP
kernels of libbolt3_amd.so (include/bolt3_amd.h).  The projections are one
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
from .layers import RMSNorm, RoPE

N_SINKS = 4


def _require_gpu(t: torch.Tensor, what: str):
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the Bolt-3 HIP path needs a ROCm device tensor (got {t.device}); "
                           f"there is no CPU implementation")


_SIDE_STREAMS: dict = {}
_N_CUS: dict = {}


def _n_cus(dev: torch.device) -> int:
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _N_CUS:
        _N_CUS[key] = torch.cuda.get_device_properties(key).multi_processor_count
    return _N_CUS[key]


def _side_stream(dev: torch.device, i: int = 0) -> torch.cuda.Stream:
    """Extra streams per device (default priority): 0 for the chain's slot decisions, 1 for its
    M_res updates."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), i)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=dev)
    return _SIDE_STREAMS[key]


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


class _NoBackward(torch.autograd.Function):
    """Keeps autograd edges to the inputs but refuses to differentiate the HIP path."""

    @staticmethod
    def forward(ctx, out, *inputs):
        return out.view_as(out)

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError("Bolt3Attn backward is not implemented in the HIP path yet")


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
               kv_offset=0, lin_kv=None, parts=0, gates=None):
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
        A.call("bolt3_heads", a, (lin if lin is not None else lin_kv).device)

    def _chain(self, dt, device, B, kr, kp, v, tok_bh_stride, pos, beta, beta_bh_stride, n_steps, off0, len0,
               step_stride, step_len, n_filled, st: dict, m_res, gam, side, snap_k=None, snap_v=None,
               snap_bias=None, snap_m=None, log=None, kp_exact=False, phase=0, work=None, started=None):
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
        out = self._forward_hip(x, _trace)
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            out = _NoBackward.apply(out, x, *[p for p in self.parameters() if p.requires_grad])
        return out

    @torch.no_grad()
    def _forward_hip(self, x: torch.Tensor, trace: dict | None) -> torch.Tensor:
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
        k_raw = torch.empty(b, HKV, T, HD, dtype=dt, device=dev)
        k_rope, v = torch.empty_like(k_raw), torch.empty_like(k_raw)
        beta = torch.empty(b, HKV, T, device=dev)
        pos = torch.empty(T, device=dev)
        self._heads(None, b, T, dt, side, 0, None, None, k_raw, k_rope, v, beta, None, pos_out=pos,
                    lin_kv=lin_kv, parts=2, gates=gates)

        n_chunks = (T + C - 1) // C
        n_cons = max(0, n_chunks - 2)
        bh = b * HKV
        snaps = (None, None, None, None)
        split = n_cons > 0 and dt == torch.bfloat16
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
            s_dec = _side_stream(dev, 0)
            s_m = _side_stream(dev, 1) if split else s_dec
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
            if trace is not None:
                log = torch.zeros(n_cons, bh, A.LOG_ROWS, A.LOG_COLS, device=dev)
            works = [torch.empty(A.chain_workspace_bytes(dt, b, HKV, HD, S, s1 - s0), dtype=torch.uint8, device=dev)
                     for s0, s1 in groups]
            s_dec.wait_stream(main)   # after the head preparation and the allocations above
            esz = k_raw.element_size()
            nf = 0
            for (s0, s1), work in zip(groups, works):
                # step 0 takes the first chunk after its sinks; step i > 0 takes chunk i
                tok = s0 * C
                off0, len0 = (ns, C - ns) if s0 == 0 else (0, C)
                args = (dt, dev, b, k_raw.data_ptr() + tok * HD * esz, k_rope.data_ptr() + tok * HD * esz,
                        v.data_ptr() + tok * HD * esz, T * HD, pos.data_ptr() + tok * 4, beta.data_ptr() + tok * 4,
                        T, s1 - s0, off0, len0, C, C, nf, st, m_res, gam, side,
                        *(t[s0:s1] for t in snaps))
                kw = dict(log=None if log is None else log[s0:s1], kp_exact=True, work=work)
                if split:
                    count = ctr is not None and s0 == 0
                    with torch.cuda.stream(s_dec):
                        self._chain(*args, phase=1, started=ctr[0].data_ptr() if count else None, **kw)
                    if count:
                        ctr[1] += bh
                        first_started = ctr[1]
                    s_m.wait_stream(s_dec)
                    with torch.cuda.stream(s_m):
                        self._chain(*args, phase=2, **kw)
                else:
                    with torch.cuda.stream(s_dec):
                        self._chain(*args, **kw)
                ev = torch.cuda.Event()
                ev.record(s_m)
                done.append(ev)
                for i in range(s0, s1):   # filled slots after each step depend only on the token counts
                    nf = min(S, nf + (C - ns if i == 0 else C))
            if trace is not None:
                trace.update(state=st, m_res=m_res, snap_k=snaps[0], snap_v=snaps[1], snap_bias=snaps[2],
                             snap_m=snaps[3], log=log)
        if first_started is not None:
            _wait_started(dev, ctr[0], first_started)
        lin_q = F.linear(x, side["wq"], side["bq"])
        q_raw = torch.empty(b, H, T, HD, dtype=dt, device=dev)
        q_rope = torch.empty_like(q_raw)
        eta = torch.empty(b, H, T, device=dev)
        self._heads(lin_q, b, T, dt, side, 0, q_raw, q_rope, None, None, None, None, eta, lin_kv=lin_kv, parts=1,
                    gates=gates)
        if trace is not None:
            trace.update(q_raw=q_raw, q_rope=q_rope, k_raw=k_raw, k_rope=k_rope, v=v, beta=beta, eta=eta, pos=pos)

        K = H * HD
        a = A.AttnArgs()
        a.dtype, a.B, a.H, a.HKV, a.HD, a.S, a.C, a.n_sinks = A.dtype_code(dt), b, H, HKV, HD, S, C, self.n_sinks
        a.mode, a.n_q, a.score_round = 0, T, 1
        a.q_rope, a.q_raw, a.q_sb, a.q_sh = q_rope.data_ptr(), q_raw.data_ptr(), q_rope.stride(0), q_rope.stride(1)
        a.eta, a.e_sb, a.e_sh = eta.data_ptr(), eta.stride(0), eta.stride(1)
        a.win_k, a.win_v, a.w_sb, a.w_sh = k_rope.data_ptr(), v.data_ptr(), k_rope.stride(0), k_rope.stride(1)
        if n_cons > 0:
            a.slot_k, a.slot_v, a.slot_bias = snaps[0].data_ptr(), snaps[1].data_ptr(), snaps[2].data_ptr()
            a.slot_step = bh * S * HD
            a.m_res, a.m_step = snaps[3].data_ptr(), bh * HD * HD
            a.m_split = int(dt == torch.bfloat16)
        a.gamma, a.res_w, a.eps = gam.data_ptr(), side["res_w"].data_ptr(), float(self.res_norm.eps)
        if not split:
            y = torch.empty(b, T, K, dtype=dt, device=dev)
            a.y, a.y_sb, a.y_st = y.data_ptr(), y.stride(0), y.stride(1)
            for ev in done:
                main.wait_event(ev)
            A.call("bolt3_chunk_attn", a, dev)
            if trace is not None:
                trace["y"] = y
            return F.linear(y, side["wo"])

        # Group by group, as soon as the chain has produced a group's snapshots: the attention
        # over all key fields of the group's chunks (the first group also takes chunks 0 and 1),
        # the readout and o_proj.  The attention output of a group of chunks is one
        # [B * rows, H * HD] block (token ranges of all batch rows together), so o_proj of a
        # group is one GEMM.
        spans = [(0, min(T, (groups[0][1] + 2) * C))] + \
                [(min(T, (s0 + 2) * C), min(T, (s1 + 2) * C)) for s0, s1 in groups[1:]]
        y_all = torch.empty(b * T * K, dtype=dt, device=dev)
        blocks, off = [], 0
        for t0, t1 in spans:
            blocks.append(y_all[off:off + b * (t1 - t0) * K].view(b * (t1 - t0), K))
            off += b * (t1 - t0) * K
        out = torch.empty(b, T, self.o_proj.out_features, dtype=dt, device=dev)
        esz = y_all.element_size()
        a.part = 0
        for gi, ((s0, s1), ev) in enumerate(zip(groups, done)):
            t0, t1 = spans[gi]
            main.wait_event(ev)
            a.chunk_begin, a.chunk_end = (0 if gi == 0 else s0 + 2), s1 + 2
            # element (b, t) of block gi at block + (b * rows + t - t0) * K
            a.y, a.y_sb, a.y_st = blocks[gi].data_ptr() - t0 * K * esz, (t1 - t0) * K, K
            A.call("bolt3_chunk_attn", a, dev)
            out[:, t0:t1].copy_(F.linear(blocks[gi], side["wo"]).view(b, t1 - t0, -1))
        if trace is not None:
            trace["y"] = torch.cat([blk.view(b, t1 - t0, K) for blk, (t0, t1) in zip(blocks, spans)], dim=1)
        return out

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


# ==================================================================== decoder

class StaticKV:
    """Growing key/value cache of a softmax-anchor layer (vsa_lm/decode.py:88-106)."""

    def __init__(self, B: int, HKV: int, Tmax: int, HD: int, dev, dt=torch.bfloat16):
        self.k = torch.empty(B, HKV, Tmax, HD, device=dev, dtype=dt)
        self.v = torch.empty_like(self.k)
        self.n = 0

    def append(self, k_new, v_new):
        L = k_new.shape[2]
        if self.n + L > self.k.shape[2]:
            cap = max(self.n + L + 1024, self.k.shape[2] * 2)
            nk = torch.empty(*self.k.shape[:2], cap, self.k.shape[3], device=self.k.device, dtype=self.k.dtype)
            nv = torch.empty_like(nk)
            nk[:, :, :self.n] = self.k[:, :, :self.n]
            nv[:, :, :self.n] = self.v[:, :, :self.n]
            self.k, self.v = nk, nv
        self.k[:, :, self.n:self.n + L] = k_new
        self.v[:, :, self.n:self.n + L] = v_new
        self.n += L
        return self.k[:, :, :self.n], self.v[:, :, :self.n]


class Bolt3LayerState:
    """Decoder state of one Bolt-3 layer in preallocated device buffers.

    The window is a ring of two halves of 2C tokens each: the previous chunk
    ("prev") in one half, the chunk being filled ("cur") in the other.  Slot
    state keeps the un-roped keys (ak) plus a cache of the keys roped at their
    mean positions (slot_k) and the attention bias (slot_bias), refreshed by
    every consolidation.  Reads with the reference's key names are served by
    ``__getitem__`` (vsa_lm/config/bolt3.py:310-315).
    """

    def __init__(self, ly: Bolt3Attn, B: int, device, dtype):
        C, S, HKV, HD = ly.C, ly.S, ly.HKV, ly.HD
        self.B, self.C, self.S, self.HKV, self.HD, self.dtype = B, C, S, HKV, HD, dtype
        self.cap = 4 * C
        self.win_kr = torch.zeros(B, HKV, self.cap, HD, dtype=dtype, device=device)
        self.win_kp = torch.zeros_like(self.win_kr)
        self.win_v = torch.zeros_like(self.win_kr)
        self.win_b = torch.zeros(B, HKV, self.cap, device=device)
        self.win_pos = torch.zeros(self.cap, device=device)
        self.sink_k = torch.zeros(B, HKV, N_SINKS, HD, dtype=dtype, device=device)
        self.sink_v = torch.zeros_like(self.sink_k)
        self.n_sink = 0
        bh = B * HKV
        self.slots = ly._empty_slots(bh, dtype, device)
        self.slot_k = torch.zeros(bh, S, HD, dtype=dtype, device=device)
        self.slot_bias = torch.zeros(bh, S, device=device)
        self.has_slots = False
        self.n_filled = 0
        self.prev = (0, 0)          # (start, length) in the ring
        self.cur = (2 * C, 0)
        self._dec_work = None
        self._dec = None   # the one-token step: key, argument blocks, output and projection workspace

    def decode_workspace(self, H: int) -> torch.Tensor:
        """Scratch of the one-token decode kernels (partial softmax state per key range)."""
        n = A.decode_workspace_bytes(self.B, H, self.HKV, self.HD) // 4
        if self._dec_work is None or self._dec_work.numel() < n:
            self._dec_work = torch.empty(n, device=self.win_kr.device)
        return self._dec_work

    def _seg(self, name, seg):
        s, n = seg
        if n == 0:
            return None
        if name == "pos":
            return self.win_pos[s:s + n].view(1, 1, n)
        if name == "b":
            return self.win_b[:, :, s:s + n]
        return {"kr": self.win_kr, "kp": self.win_kp, "v": self.win_v}[name][:, :, s:s + n]

    def __getitem__(self, key):
        B, HKV = self.B, self.HKV
        if key in ("ak", "av"):
            return self.slots[key].view(B, HKV, self.S, self.HD) if self.has_slots else None
        if key in ("mass", "util", "pm"):
            return self.slots[key].view(B * HKV, self.S) if self.has_slots else None
        if key == "act":
            return self.slots["act"].bool() if self.has_slots else None
        if key in ("sink_k", "sink_v"):
            return getattr(self, key)[:, :, :self.n_sink] if self.n_sink else None
        if key == "n_filled":
            return self.n_filled
        for pre, seg in (("prev_", self.prev), ("cur_", self.cur)):
            if key.startswith(pre):
                return self._seg(key[len(pre):], seg)
        raise KeyError(key)

    def get(self, key, default=None):
        try:
            v = self[key]
        except KeyError:
            return default
        return default if v is None else v


class Bolt3Decoder:
    """Constant-memory decoder over a hybrid Bolt-3 / softmax stack (vsa_lm/config/bolt3.py:279-557)."""

    def __init__(self, model, wrap_positions: bool = False, max_cache_pos: int = 65536, **kwargs):
        self.model = model.eval()
        self.max_T = model.config["max_T"]
        self.max_cache_pos = max_cache_pos
        self.C = int(model.config.get("bolt3_C", 128))
        # bf16 one-token steps run as one bolt3_decode_layer call (projections included); False
        # keeps the projections in torch around bolt3_decode (the tests compare the two)
        self.fuse_projections = True

    def _graph_runner(self, B: int, need_len: int, device):
        return None

    @staticmethod
    def state_bytes(model):
        flat, per_tok = 0, 0
        for blk in model.blocks:
            if hasattr(blk, "vsa"):
                ly = blk.vsa
                flat += ly.HKV * ly.HD * ly.HD * 4 + 2 * ly.S * ly.HKV * ly.HD * 2 + 4 * ly.C * ly.HKV * ly.HD * 2
            else:
                s = blk.attn
                per_tok += 2 * s.HKV * s.HD * 2
        return flat, per_tok

    @staticmethod
    def blank_state(model, batch_size: int, device, max_kv_len: int = 4096, state_dtype=torch.float32,
                    dtype=None, **kwargs):
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("Bolt3Decoder.blank_state: the Bolt-3 HIP path needs a ROCm device")
        dt = dtype or next(model.parameters()).dtype
        states, kv = [None] * len(model.blocks), [None] * len(model.blocks)
        for li, blk in enumerate(model.blocks):
            if hasattr(blk, "vsa"):
                ly = blk.vsa
                states[li] = torch.zeros(batch_size, ly.HKV, ly.HD, ly.HD, device=device, dtype=state_dtype)
                kv[li] = Bolt3LayerState(ly, batch_size, device, dt)
            else:
                s = blk.attn
                kv[li] = StaticKV(batch_size, s.HKV, max_kv_len, s.HD, device, dt=dt)
        return states, kv

    @staticmethod
    def _sample(logits, temperature: float, top_k: int = 40, top_p: float = 0.95):
        if temperature <= 1e-5:
            return logits.argmax(-1, keepdim=True)
        probs = F.softmax(logits.float() / temperature, dim=-1)
        if top_p < 1.0:
            sp, si = torch.sort(probs, descending=True, dim=-1)
            cp = torch.cumsum(sp, dim=-1)
            sp[cp - sp > top_p] = 0.0
            sp.div_(sp.sum(dim=-1, keepdim=True).clamp_min(1e-12))
            return si.gather(-1, torch.multinomial(sp, 1))
        tv, ti = torch.topk(logits.float() / temperature, min(top_k, logits.size(-1)), dim=-1)
        return ti.gather(-1, torch.multinomial(F.softmax(tv, -1), 1))

    # ------------------------------------------------------------ one Bolt-3 layer

    def _bolt3_layer(self, ly: Bolt3Attn, h, pos_start: int, m_state: torch.Tensor, st: Bolt3LayerState,
                     record=None):
        B, t, _ = h.shape
        dt, dev = h.dtype, h.device
        if dt != st.dtype:
            raise TypeError(f"activation dtype {dt} differs from the decoder state dtype {st.dtype}")
        if t > ly.C:
            raise NotImplementedError(f"step takes at most C={ly.C} tokens per call (got {t})")
        H, HKV, HD, S = ly.H, ly.HKV, ly.HD, ly.S
        W, bias, side = ly._packed(dt, dev)
        gam = side["gamma"]
        cs, cl = st.cur
        ps, pl = st.prev
        h = h if h.is_contiguous() else h.contiguous()
        if t == 1:
            # The argument block, the projection row and the attention output are kept in the
            # layer state; a step only refreshes the position, the ring segments and the input
            # and output rows.  bf16 runs the whole step (both projections included) in one
            # bolt3_decode_layer call.
            fused = self.fuse_projections and dt == torch.bfloat16 and h.shape[-1] % 32 == 0 and \
                side["wo"].shape[0] % 16 == 0
            key = (id(side), m_state.data_ptr(), W.data_ptr(), fused)
            if st._dec is None or st._dec[0] != key:
                y = torch.empty(B, H * HD, dtype=dt, device=dev)
                n_out = side["wo"].shape[0]
                pw = torch.empty(A.decode_layer_workspace_bytes(B, h.shape[-1], W.shape[0], H * HD, n_out) // 4,
                                 device=dev) if fused else None
                la = A.DecodeLayerArgs() if fused else None
                a = la.dec if fused else A.DecodeArgs()   # la.dec shares la's memory
                a.dtype, a.B, a.H, a.HKV, a.HD, a.S = A.dtype_code(dt), B, H, HKV, HD, S
                a.lin_row_stride = W.shape[0]
                a.qn_w, a.kn_w, a.has_qk_norm = A.ptr(side["qn"]), A.ptr(side["kn"]), int(side["qn"] is not None)
                a.eps, a.inv_freq = float(ly.res_norm.eps), side["inv_freq"].data_ptr()
                a.win_kr, a.win_kp, a.win_v = st.win_kr.data_ptr(), st.win_kp.data_ptr(), st.win_v.data_ptr()
                a.w_sb, a.w_sh = st.win_kr.stride(0), st.win_kr.stride(1)
                a.win_beta, a.wb_sb, a.wb_sh = st.win_b.data_ptr(), st.win_b.stride(0), st.win_b.stride(1)
                a.win_pos = st.win_pos.data_ptr()
                a.sink_k, a.sink_v = st.sink_k.data_ptr(), st.sink_v.data_ptr()
                a.s_sb, a.s_sh = st.sink_k.stride(0), st.sink_k.stride(1)
                a.slot_k, a.slot_v, a.slot_bias = st.slot_k.data_ptr(), st.slots["av"].data_ptr(), \
                    st.slot_bias.data_ptr()
                a.m_res, a.gamma, a.res_w, a.y = m_state.data_ptr(), gam.data_ptr(), side["res_w"].data_ptr(), \
                    y.data_ptr()
                work = st.decode_workspace(H)
                a.work, a.work_bytes = work.data_ptr(), work.numel() * 4
                if fused:
                    la.proj_work, la.proj_work_bytes = pw.data_ptr(), pw.numel() * 4
                    la.x_row_stride, la.d_model = h.shape[-1], h.shape[-1]
                    la.w_in, la.b_in, la.n_in = W.data_ptr(), A.ptr(bias), W.shape[0]
                    la.w_out, la.b_out, la.n_out = side["wo"].data_ptr(), None, side["wo"].shape[0]
                    la.out_row_stride = side["wo"].shape[0]
                st._dec = (key, la if fused else a, a, y, pw, side, W, bias)
            _, call_args, a, y, _, _, _, _ = st._dec
            a.pos = int(pos_start)
            a.a_start, a.a_len, a.b_start, a.b_len = ps, pl, cs, cl
            a.n_sink_keys, a.has_slots = st.n_sink, int(st.has_slots)
            if fused:
                out = torch.empty(B, 1, side["wo"].shape[0], dtype=dt, device=dev)
                call_args.x, call_args.out = h.data_ptr(), out.data_ptr()
                A.call("bolt3_decode_layer", call_args, dev)
                st.cur = (cs, cl + 1)
                if st.cur[1] >= ly.C:
                    self._consolidate(ly, st, m_state, gam, side, record)
                return out
            lin = F.linear(h, W, bias)
            a.lin = lin.data_ptr()
            A.call("bolt3_decode", a, dev)
            y = y.view(B, 1, H * HD)
        else:
            lin = F.linear(h, W, bias)
            q_raw = torch.empty(B, H, t, HD, dtype=dt, device=dev)
            q_rope = torch.empty_like(q_raw)
            eta = torch.empty(B, H, t, device=dev)
            ly._heads(lin, B, t, dt, side, pos_start, q_raw, q_rope, st.win_kr, st.win_kp, st.win_v, st.win_b, eta,
                      pos_out=st.win_pos, kv_offset=cs + cl)
            y = torch.empty(B, t, H * HD, dtype=dt, device=dev)
            a = A.AttnArgs()
            a.dtype, a.B, a.H, a.HKV, a.HD, a.S, a.C, a.n_sinks = A.dtype_code(dt), B, H, HKV, HD, S, ly.C, ly.n_sinks
            a.mode, a.n_q, a.score_round = 1, t, 0
            a.q_rope, a.q_raw, a.q_sb, a.q_sh = q_rope.data_ptr(), q_raw.data_ptr(), q_rope.stride(0), q_rope.stride(1)
            a.eta, a.e_sb, a.e_sh = eta.data_ptr(), eta.stride(0), eta.stride(1)
            a.win_k, a.win_v, a.w_sb, a.w_sh = st.win_kp.data_ptr(), st.win_v.data_ptr(), st.win_kp.stride(0), \
                st.win_kp.stride(1)
            a.a_start, a.a_len, a.b_start, a.b_len = ps, pl, cs, cl + t
            a.sink_k, a.sink_v = st.sink_k.data_ptr(), st.sink_v.data_ptr()
            a.s_sb, a.s_sh, a.n_sink_keys = st.sink_k.stride(0), st.sink_k.stride(1), st.n_sink
            a.slot_k, a.slot_v, a.slot_bias = st.slot_k.data_ptr(), st.slots["av"].data_ptr(), st.slot_bias.data_ptr()
            a.slot_step, a.has_slots = 0, int(st.has_slots)
            a.m_res, a.m_step = m_state.data_ptr(), 0
            a.gamma, a.res_w, a.eps = gam.data_ptr(), side["res_w"].data_ptr(), float(ly.res_norm.eps)
            a.y, a.y_sb, a.y_st = y.data_ptr(), y.stride(0), y.stride(1)
            A.call("bolt3_chunk_attn", a, dev)
        st.cur = (cs, cl + t)
        out = F.linear(y, side["wo"])
        if st.cur[1] >= ly.C:
            self._consolidate(ly, st, m_state, gam, side, record)
        return out

    def _consolidate(self, ly: Bolt3Attn, st: Bolt3LayerState, m_state, gam, side, record=None):
        ps, pl = st.prev
        if pl > 0:
            off, l = ps, pl
            if st.n_sink == 0:
                ns = min(ly.n_sinks, l)
                st.sink_k[:, :, :ns].copy_(st.win_kp[:, :, off:off + ns])
                st.sink_v[:, :, :ns].copy_(st.win_v[:, :, off:off + ns])
                st.n_sink = ns
                off, l = off + ns, l - ns
            if st.n_filled == 0:
                for k, v in ly._empty_slots(st.B * st.HKV, st.dtype, m_state.device).items():
                    st.slots[k].copy_(v)
                m_state.zero_()
            log = None
            if record is not None:
                log = torch.zeros(1, st.B * st.HKV, A.LOG_ROWS, A.LOG_COLS, device=m_state.device)
                record.append(dict(log=log[0], n_filled=st.n_filled, tokens=l))
            ly._chain(st.dtype, m_state.device, st.B, st.win_kr.data_ptr(), st.win_kp.data_ptr(),
                      st.win_v.data_ptr(), st.cap * st.HD, st.win_pos.data_ptr(), st.win_b.data_ptr(), st.cap,
                      1, off, l, l, l, st.n_filled, st.slots, m_state, gam, side,
                      snap_k=st.slot_k, snap_bias=st.slot_bias, kp_exact=True, log=log)
            if st.n_filled < ly.S:
                st.n_filled += min(ly.S - st.n_filled, l)
            st.has_slots = True
        cs, cl = st.cur
        st.prev = (cs, cl)
        st.cur = (0 if cs == 2 * ly.C else 2 * ly.C, 0)

    # ------------------------------------------------------------ model-level API

    @torch.no_grad()
    def step(self, tokens: torch.Tensor, pos_start: int, states, kv_caches, record=None):
        m = self.model
        b, t = tokens.shape
        x = m.embed_tokens(tokens)
        for li, blk in enumerate(m.blocks):
            h = blk.norm1(x)
            if hasattr(blk, "vsa"):
                rec = None
                if record is not None:
                    rec = record.setdefault(li, []) if isinstance(record, dict) else record
                x = x + self._bolt3_layer(blk.vsa, h, pos_start, states[li], kv_caches[li], rec)
            else:
                ly = blk.attn
                q, k, v = ly.head_qkv(h)
                q, k = ly.rope(q, pos_start=pos_start), ly.rope(k, pos_start=pos_start)
                n_prev = kv_caches[li].n
                pk, pv = kv_caches[li].append(k, v)
                if t > 1:
                    qi = torch.arange(t, device=tokens.device)[:, None]
                    kj = torch.arange(n_prev + t, device=tokens.device)[None, :]
                    cmask = (kj <= (n_prev + qi)).view(1, 1, t, n_prev + t)
                    y = F.scaled_dot_product_attention(q, pk.to(q.dtype), pv.to(q.dtype), attn_mask=cmask,
                                                       enable_gqa=ly.G > 1)
                else:
                    y = F.scaled_dot_product_attention(q, pk.to(q.dtype), pv.to(q.dtype), enable_gqa=ly.G > 1)
                x = x + ly.o_proj(y.transpose(1, 2).reshape(b, t, ly.H * ly.HD))
            x = x + blk.mlp(blk.norm2(x))
        return m.norm(x), states, kv_caches

    @torch.no_grad()
    def prefill(self, ids: torch.Tensor, max_kv_len: int = 4096):
        b, t = ids.shape
        states, kv = self.blank_state(self.model, b, ids.device, max_kv_len=max(max_kv_len, t + 1024))
        h = None
        for s in range(0, t, self.C):
            h, states, kv = self.step(ids[:, s:min(t, s + self.C)], s, states, kv)
        return h, states, kv

    @torch.no_grad()
    def generate_batch(self, ids: torch.Tensor, max_new_tokens: int, temperature: float = 0.6, top_k: int = 40,
                       top_p: float = 0.95, eos_ids: set[int] | None = None,
                       close_think_ids: list[int] | None = None):
        B, T = ids.shape
        h, states, kv = self.prefill(ids, max_kv_len=T + max_new_tokens + 64)
        logits = self.model.lm_head(h[:, -1, :])
        eos = torch.tensor(sorted(eos_ids or ()), device=ids.device, dtype=torch.long)
        done = torch.zeros(B, dtype=torch.bool, device=ids.device)
        lengths = torch.full((B,), max_new_tokens, dtype=torch.long, device=ids.device)
        end_think = close_think_ids[1] if (close_think_ids and len(close_think_ids) > 1) else None
        closed = torch.zeros(B, dtype=torch.bool, device=ids.device)
        q_pos = torch.full((B,), -1, dtype=torch.long, device=ids.device)
        trigger = max(64, max_new_tokens - 64)
        out, pos = [], T
        for i in range(max_new_tokens):
            nxt = self._sample(logits, temperature, top_k=top_k, top_p=top_p)
            if close_think_ids:
                if i == trigger:
                    q_pos[(~closed) & (~done) & (q_pos < 0)] = 0
                active = q_pos >= 0
                if bool(active.any()):
                    for r in torch.nonzero(active, as_tuple=False).view(-1).tolist():
                        nxt[r, 0] = close_think_ids[int(q_pos[r])]
                        q_pos[r] += 1
                        if q_pos[r] >= len(close_think_ids):
                            q_pos[r] = -1
                            closed[r] = True
                if end_think is not None:
                    closed |= nxt[:, 0] == end_think
            out.append(nxt)
            if eos.numel():
                hit = torch.isin(nxt[:, 0], eos) & ~done
                lengths[hit] = i + 1
                done |= hit
                if i % 16 == 15 and bool(done.all()):
                    break
            h, states, kv = self.step(nxt, pos, states, kv)
            logits = self.model.lm_head(h[:, -1, :])
            pos += 1
        return torch.cat(out, dim=1), lengths

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, max_new_tokens: int, temperature: float = 0.0, top_k: int = 40,
                 top_p: float = 0.95, eos_ids: set[int] | None = None, close_think_ids: list[int] | None = None):
        toks, n = self.generate_batch(prompt, max_new_tokens, temperature, top_k, top_p, eos_ids, close_think_ids)
        return torch.cat([prompt, toks[:, : int(n[0].item())]], dim=1)

    @torch.no_grad()
    def continue_generate(self, ids: torch.Tensor, states, kv_caches, start_pos: int, max_new_tokens: int,
                          temperature: float = 0.0, top_k: int = 40, top_p: float = 0.95,
                          eos_ids: set[int] | None = None):
        out, pos, h = [], start_pos, None
        for s in range(0, ids.shape[1], self.C):
            e = min(ids.shape[1], s + self.C)
            h, states, kv_caches = self.step(ids[:, s:e], pos, states, kv_caches)
            pos += e - s
        logits = self.model.lm_head(h[:, -1, :])
        for _ in range(max_new_tokens):
            nxt = self._sample(logits, temperature, top_k=top_k, top_p=top_p)
            out.append(nxt)
            if eos_ids and int(nxt[0, 0].item()) in eos_ids:
                break
            h, states, kv_caches = self.step(nxt, pos, states, kv_caches)
            logits = self.model.lm_head(h[:, -1, :])
            pos += 1
        toks = torch.cat(out, dim=1) if out else torch.empty(ids.shape[0], 0, dtype=torch.long, device=ids.device)
        return toks, states, kv_caches, pos

    @torch.no_grad()
    def memorize(self, ids: torch.Tensor, states, kv_caches, start_pos: int):
        pre = [s.clone() if s is not None else None for s in states]
        pos = start_pos
        for s in range(0, ids.shape[1], self.C):
            e = min(ids.shape[1], s + self.C)
            _, states, kv_caches = self.step(ids[:, s:e], pos, states, kv_caches)
            pos += e - s
        n_tok = ids.shape[1]
        traces = []
        for li, blk in enumerate(self.model.blocks):
            if hasattr(blk, "vsa"):
                gam = blk.vsa.gamma_delta().view(1, -1, 1, 1).to(states[li].device)
                traces.append((pos, states[li] - (gam ** (n_tok // blk.vsa.C)) * pre[li]))
            else:
                traces.append(None)
        return states, kv_caches, pos, traces

    @torch.no_grad()
    def forget(self, traces, states, next_pos: int, kv_caches=None, pre_kv_lens=None):
        for li, tr in enumerate(traces):
            if tr is not None and states[li] is not None:
                end_p, delta = tr
                blk = self.model.blocks[li]
                gam = blk.vsa.gamma_delta().view(1, -1, 1, 1).to(states[li].device)
                states[li] = states[li] - (gam ** max(0, (next_pos - end_p) // blk.vsa.C)) * delta
        return states
