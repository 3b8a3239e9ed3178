"""Backward of Bolt3Attn.forward on the HIP path.

The reference differentiates its forward with autograd (vsa_lm/config/bolt3.py:194-276); its
slot decisions run under no_grad (:98-112, :121-135, :165-180), so the gradient is that of a
forward whose decisions are constants.  This module computes the same gradients from what the
HIP forward keeps, in four C calls and the projections' products:

* ``bolt3_attn_bwd``: the attention over [sinks | slots | window] and the M_res readout of every
  chunk -- the gradients of the roped queries, the un-roped queries (readout), eta, every key
  field, every slot snapshot, the slot bias, M_res of every step, res_norm's weight and gamma;
* ``bolt3_chain_bwd``: the consolidation chain walked backwards from the forward's decision log
  and per-step snapshots -- the slots' keys and values are copies and mass-weighted means of
  token keys and values (:121-155, :182-191), M_res follows the Gershgorin-scaled delta rule
  (:157-166);
* ``bolt3_heads_bwd``: RoPE, the q/k RMSNorm and the gates' sigmoid / tanh back to the packed
  projection output; gamma's clamp and the projections close the chain back to x and the
  parameters.

There is no second path: a shape the kernels do not take (more than 128 tokens per chunk, S other
than 128, head_dim other than 64 or 128) raises.

``Bolt3Function`` keeps the forward's trace through ``save_for_backward``, so activation
checkpointing (the heal trainer wraps every block in ``torch.utils.checkpoint``,
vsa_lm/converter.py:698-700) frees it between the forward and the backward and recomputes it.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _abi as A


def chain_backward_args(mod, tr: dict, o: dict, gam: torch.Tensor, b: int, n_steps: int, zeros: dict):
    """bolt3_chain_bwd's arguments on the forward's trace and the attention backward's outputs,
    and its buffers: the gradients of the un-roped keys and the values [bh, T, HD] and of beta
    [bh, T] (fp32, taken zero-filled from ``zeros``), the per-step gamma partial sums and the
    workspace.  The caller runs the phases (1 and 2 may go on different streams, 3 after both)."""
    HKV, HD, S, C = mod.HKV, mod.HD, mod.S, mod.C
    k_raw = tr["k_raw"]
    T = k_raw.shape[2]
    bh = b * HKV
    dev = k_raw.device
    ns = min(mod.n_sinks, C)
    buf = dict(d_kr=zeros["d_kr"], d_v=zeros["d_v"], d_beta=zeros["d_beta"],
               d_gamma=torch.empty(n_steps, bh, HD // 32, device=dev, dtype=torch.float32),
               work=torch.empty(max(1, A.chain_bwd_workspace_bytes(b, HKV, HD, n_steps)), dtype=torch.uint8,
                                device=dev))
    a = A.ChainBwdArgs()
    a.dtype, a.B, a.HKV, a.HD, a.S, a.T = A.dtype_code(k_raw.dtype), b, HKV, HD, S, T
    a.n_steps, a.off0, a.len0, a.step_stride, a.step_len = n_steps, ns, C - ns, C, C
    a.kr, a.v, a.beta, a.log = k_raw.data_ptr(), tr["v"].data_ptr(), tr["beta"].data_ptr(), tr["log"].data_ptr()
    a.snap_mass, a.snap_pm, a.snap_m = tr["snap_mass"].data_ptr(), tr["snap_pm"].data_ptr(), tr["snap_m"].data_ptr()
    inv_freq = mod._packed(k_raw.dtype, dev)[2]["inv_freq"]
    a.gamma, a.inv_freq = gam.data_ptr(), inv_freq.data_ptr()
    a.d_slot_k, a.d_slot_v, a.d_m = o["d_slot_k"].data_ptr(), o["d_slot_v"].data_ptr(), o["d_m"].data_ptr()
    for k in ("d_kr", "d_v", "d_beta", "d_gamma"):
        setattr(a, k, buf[k].data_ptr())
    a.work, a.work_bytes = buf["work"].data_ptr(), buf["work"].numel()
    return a, buf


def chain_backward_hip(mod, tr: dict, o: dict, gam: torch.Tensor, b: int, n_steps: int):
    """bolt3_chain_bwd in one call: the gradients of the un-roped keys and the values [bh, T, HD],
    of beta [bh, T] (all fp32) and of gamma [HKV]."""
    k_raw = tr["k_raw"]
    bh, T, HD = b * mod.HKV, k_raw.shape[2], mod.HD
    f32 = dict(device=k_raw.device, dtype=torch.float32)
    zeros = dict(d_kr=torch.zeros(bh, T, HD, **f32), d_v=torch.zeros(bh, T, HD, **f32), d_beta=torch.zeros(bh, T, **f32))
    a, buf = chain_backward_args(mod, tr, o, gam, b, n_steps, zeros)
    A.call("bolt3_chain_bwd", a, k_raw.device)
    return buf["d_kr"], buf["d_v"], buf["d_beta"], buf["d_gamma"].view(n_steps, b, mod.HKV, -1).sum(dim=(0, 1, 3))


def _zero_arena(dev, shapes: dict) -> dict:
    """fp32 tensors of the given shapes, zero-filled by one fill over one allocation."""
    sizes = {k: int(torch.Size(v).numel()) for k, v in shapes.items()}
    arena = torch.zeros(max(1, sum(sizes.values())), device=dev, dtype=torch.float32)
    out, off = {}, 0
    for k, shp in shapes.items():
        out[k] = arena[off:off + sizes[k]].view(shp)
        off += sizes[k]
    return out


def attn_backward_args(mod, tr: dict, dy: torch.Tensor, dt: torch.dtype, n_steps: int, extra_zeros=None):
    """bolt3_attn_bwd's arguments on the forward's tensors and its output buffers by name (the
    caller runs the parts: 1, the readout; 2, the attention).  ``extra_zeros``: further fp32
    buffers {name: shape} to take zero-filled from the same fill (returned among the outputs)."""
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
    zshapes = dict(d_res_w=(bh, n_chunks, HD), d_gamma=(bh, n_chunks))
    if n_steps > 0:
        zshapes.update(d_bias=(n_steps, b * H, n_qt, S), d_sink_k=(n_chunks, bh, ns, HD),
                       d_sink_v=(n_chunks, bh, ns, HD))
    zshapes.update(extra_zeros or {})
    o = _zero_arena(dev, zshapes)
    o.update(d_rows=torch.empty(b, H, T, **f32), lse=tr["lse"],
             d_q_rope=torch.empty(b, H, T, HD, **sdt), d_q_raw=torch.empty(b, H, T, HD, **sdt),
             d_eta=torch.empty(b, H, T, **f32),
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
        o.update(d_m=torch.empty(n_steps, bh, HD, HD, **f32),
                 d_slot_k=torch.empty(n_steps, bh, S, HD, **f32), d_slot_v=torch.empty(n_steps, bh, S, HD, **f32))
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
        if hasattr(a, name):
            setattr(a, name, t.data_ptr())
    # the readout's du / |q_raw| rows between its two kernels: d_q_rope's memory, which the
    # attention kernels (part 2) overwrite afterwards
    a.rd_rows = o["d_q_rope"].data_ptr()
    return a, o


def layer_backward(mod, x: torch.Tensor, tr: dict, d_out: torch.Tensor, dt: torch.dtype):
    """Gradients of Bolt3Attn.forward: (dx, {parameter name: gradient}); the projections'
    gradients (dx among them) in the storage dtype their products run in, the rest fp32.

    Two streams.  This one: the o_proj products, the readout's backward, the chain's token
    statistics, the attention's backward, the chain's slot recursion and token gradients, the
    key / value part of the head backward and the projections' products.  The side stream: the
    chain's M_res recursion, a few long-lived workgroups that run beside the attention's backward
    (this stream holds the attention until they are resident, bolt3_wait_count), then the query
    part of the head backward beside the chain's slot recursion and token gradients, and the
    reductions to the small parameters.  Every buffer the side stream touches is allocated on this stream and held here
    until this stream has waited for the side stream's last kernel; the side stream's own results
    are marked as used on this stream."""
    from .bolt3 import WAIT_POLLS, _n_cus, _started_counter   # (bolt3 imports this module)
    b, T, D = x.shape
    H, HKV, HD, S, C = mod.H, mod.HKV, mod.HD, mod.S, mod.C
    G = H // HKV
    bh = b * HKV
    dev = x.device
    n_chunks = (T + C - 1) // C
    n_steps = max(0, n_chunks - 2)
    ns = min(mod.n_sinks, C)
    grads = {}
    main = torch.cuda.current_stream(dev)
    aux = A.side_stream(dev, 0)
    # the projections' products run in the storage dtype, as the reference's linears do under
    # autocast (fp32 storage: fp32 products)
    W, _, side = mod._packed(dt, dev)
    if "wT" not in side:
        # the weights' transposes, for products in F.linear's layout (cached with the pack).  The
        # packed weight's transpose takes zero columns up to a multiple of 64: dz gets as many
        # (the head backward zeroes them), and dx = dz W, whose reduction runs over them, takes a
        # faster GEMM (cfg2: 0.38 against 0.50 ms at 6208 against 6192 columns)
        kp = -(-W.shape[0] // 64) * 64
        side["wT"] = F.pad(W, (0, 0, 0, kp - W.shape[0])).t().contiguous()
        side["woT"] = side["wo"].t().contiguous()
    d_out = d_out.to(dt)
    y = tr["y"]
    grads["o_proj.weight"] = d_out.reshape(-1, D).t() @ y.reshape(-1, H * HD)
    dy = F.linear(d_out, side["woT"])                               # [b, T, H*HD], storage dtype
    # attention and readout; the chain's key / value / beta gradients come zero-filled with the
    # attention's own zero-filled outputs
    extra = dict(d_kr=(bh, T, HD), d_v=(bh, T, HD), d_beta=(bh, T)) if n_steps > 0 else None
    aa, o = attn_backward_args(mod, tr, dy, dt, n_steps, extra)
    aa.part = 1
    A.call("bolt3_attn_bwd", aa, dev)
    if n_steps > 0:
        ca, cbuf = chain_backward_args(mod, tr, o, side["gamma"], b, n_steps, o)
        ca.kernels = A.CBWD_STATS
        A.call("bolt3_chain_bwd", ca, dev)
        # (the hold only where the recursion's workgroups fit on the chip at once)
        ctr = _started_counter(dev) if bh * (HD // 32) <= _n_cus(dev) else None
        aux.wait_stream(main)
        with torch.cuda.stream(aux):
            ca.kernels, ca.started = A.CBWD_M_REC, None if ctr is None else ctr[0].data_ptr()
            A.call("bolt3_chain_bwd", ca, dev)
            ca.started = None
        ev_m = torch.cuda.Event()
        ev_m.record(aux)
        if ctr is not None:
            ctr[1] += bh * (HD // 32)
            rc = A.load().bolt3_wait_count(ctr[0].data_ptr(), ctr[1] & 0xFFFFFFFF, WAIT_POLLS, A.stream_of(dev))
            if rc != 0:
                raise RuntimeError(f"bolt3_wait_count failed with code {rc}")
    aa.part = 2
    A.call("bolt3_attn_bwd", aa, dev)
    # RoPE transposes, the q / k norms' backward and the gates' derivatives, one pass over the
    # token rows into dz, the gradient of the packed projection output [q | k | v | beta | eta | pad]:
    # the query heads (part 1) on the side stream beside the chain's slot recursion and token
    # gradients, the key / value heads (part 2) here once the chain is done
    f32 = dict(device=dev, dtype=torch.float32)
    dz = torch.empty(b * T, side["wT"].shape[1], dtype=dt, device=dev)
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
        ha.d_k_chain, ha.d_v_chain, ha.d_beta = cbuf["d_kr"].data_ptr(), cbuf["d_v"].data_ptr(), \
            cbuf["d_beta"].data_ptr()
    ha.d_eta, ha.beta, ha.eta = o["d_eta"].data_ptr(), tr["beta"].data_ptr(), tr["eta"].data_ptr()
    if has_norm:
        lin_q, lin_kv = tr["lin_q"], tr["lin_kv"]
        d_qn, d_kn = torch.empty(nb, HD, **f32), torch.empty(nb, HD, **f32)
        ha.lin_q, ha.lin_q_row_stride = lin_q.data_ptr(), lin_q.shape[-1]
        ha.lin_k, ha.lin_k_row_stride = lin_kv.data_ptr(), lin_kv.shape[-1]
        ha.qn_w, ha.kn_w, ha.has_qk_norm = side["qn"].data_ptr(), side["kn"].data_ptr(), 1
        ha.q_eps, ha.k_eps = float(mod.q_norm.eps), float(mod.k_norm.eps)
        ha.d_qn_w, ha.d_kn_w = d_qn.data_ptr(), d_kn.data_ptr()
    ha.inv_freq = side["inv_freq"].data_ptr()
    ha.dz, ha.dz_row_stride, ha.dz_cols = dz.data_ptr(), dz.shape[1], dz.shape[1]
    aux.wait_stream(main)
    with torch.cuda.stream(aux):
        ha.parts = 1
        A.call("bolt3_heads_bwd", ha, dev)
        small = {}
        d_gam = o["d_gamma"].view(b, HKV, n_chunks).sum(dim=(0, 2))
        if n_steps > 0:
            d_gam = d_gam + cbuf["d_gamma"].view(n_steps, b, HKV, -1).sum(dim=(0, 1, 3))
            # kappa: the slot bias is kappa * log(max(mass, 1)) (vsa_lm/config/bolt3.py:238-241)
            dbias = o["d_bias"].sum(2).view(n_steps, b, HKV, G, S).sum(3)             # [step, b, HKV, S]
            logm = tr["snap_mass"].clamp_min(1.0).log().view(n_steps, b, HKV, S)
            small["kappa"] = (dbias * logm).sum(dim=(0, 1, 3))
        else:
            small["kappa"] = torch.zeros(HKV, device=dev)
        # gamma = clamp(0.999 * sigmoid(log_gamma), 1e-3, 0.999); clamp passes its bounds inclusive
        sg = torch.sigmoid(mod.log_gamma.detach().float().to(dev))
        g0 = 0.999 * sg
        inside = ((g0 >= 1e-3) & (g0 <= 0.999)).float()
        small["log_gamma"] = d_gam * 0.999 * sg * (1.0 - sg) * inside
        small["res_norm.weight"] = o["d_res_w"].sum(dim=(0, 1))
        if has_norm:
            small["q_norm.weight"] = d_qn.sum(0)
    if n_steps > 0:
        ca.kernels = A.CBWD_SLOT_REC
        A.call("bolt3_chain_bwd", ca, dev)
        main.wait_event(ev_m)
        ca.kernels = A.CBWD_TOK_GRAD
        A.call("bolt3_chain_bwd", ca, dev)
    ha.parts = 2
    A.call("bolt3_heads_bwd", ha, dev)
    main.wait_stream(aux)   # dz's query columns
    widths = [H * HD, HKV * HD, HKV * HD, HKV, H]
    lins = (mod.q_proj, mod.k_proj, mod.v_proj, mod.beta_proj, mod.eta_proj)
    names = ("q_proj", "k_proj", "v_proj", "beta_proj", "eta_proj")
    # the k norm's weight gradient and the biases' column sums of dz (accumulated in fp32, no fp32
    # copy of dz) on the side stream, beside the projections' products
    aux.wait_stream(main)
    with torch.cuda.stream(aux):
        if has_norm:
            small["k_norm.weight"] = d_kn.sum(0)
        off = 0
        for name, lin, width in zip(names, lins, widths):
            if lin.bias is not None:
                small[f"{name}.bias"] = dz[:, off:off + width].sum(0, dtype=torch.float32)
            off += width
    # one product each for dx and for the packed weight's gradient: rows q | k | v | beta | eta
    dx = F.linear(dz, side["wT"])
    dW = dz.t() @ x.reshape(b * T, D)
    off = 0
    for name, width in zip(names, widths):
        grads[f"{name}.weight"] = dW[off:off + width]
        off += width
    main.wait_stream(aux)
    for k, t in small.items():
        t.record_stream(main)
        grads[k] = t
    return dx.view(b, T, D), grads


# the forward's trace entries the backward reads (all tensors)
TRACE_KEYS = ("y", "lse", "q_rope", "q_raw", "k_raw", "k_rope", "v", "beta", "eta", "lin_q", "lin_kv", "snap_k", "snap_v",
              "snap_bias", "snap_m", "snap_mass", "snap_pm", "log")


class Bolt3Function(torch.autograd.Function):
    """Bolt3Attn.forward as one autograd node: the HIP forward keeps its trace, the backward is
    layer_backward.  Inputs: (module, x in the storage dtype, *parameters in named order).

    The trace goes through save_for_backward (the entries this forward made; one without a
    consolidation makes no snapshots or log), so saved-tensor hooks see all of it: under
    torch.utils.checkpoint(use_reentrant=False) nothing of it stays alive between the forward
    and the backward, and the backward's recomputation rebuilds it.  Saved tensors stay until
    the graph is freed, so a second backward with retain_graph=True gives the same gradients."""

    @staticmethod
    def forward(ctx, mod, x, *params):
        tr = {}
        out = mod._forward_hip(x, tr)
        ctx.mod, ctx.dt = mod, x.dtype
        ctx.names = [n for n, _ in mod.named_parameters()]
        ctx.present = tuple(k for k in TRACE_KEYS if tr.get(k) is not None)
        ctx.save_for_backward(x, *(tr[k] for k in ctx.present))
        return out

    @staticmethod
    def backward(ctx, d_out):
        x, *saved = ctx.saved_tensors
        tr = dict(zip(ctx.present, saved))
        dx, grads = layer_backward(ctx.mod, x, tr, d_out, ctx.dt)
        out = [None, dx.to(x.dtype)]
        for name, prm in zip(ctx.names, ctx.mod.parameters()):
            g = grads.get(name)
            out.append(None if g is None else g.to(prm.dtype).view_as(prm))
        return tuple(out)
