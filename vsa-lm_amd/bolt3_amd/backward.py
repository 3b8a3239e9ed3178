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


def chain_backward_hip(mod, tr: dict, o: dict, gam: torch.Tensor, b: int, n_steps: int):
    """bolt3_chain_bwd on the forward's trace and the attention backward's outputs: returns the
    gradients of the un-roped keys and the values [bh, T, HD], of beta [bh, T] (all fp32) and of
    gamma [HKV]."""
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
    work = torch.empty(max(1, A.chain_bwd_workspace_bytes(b, HKV, HD, n_steps)), dtype=torch.uint8, device=dev)
    a = A.ChainBwdArgs()
    a.dtype, a.B, a.HKV, a.HD, a.S, a.T = A.dtype_code(k_raw.dtype), b, HKV, HD, S, T
    a.n_steps, a.off0, a.len0, a.step_stride, a.step_len = n_steps, ns, C - ns, C, C
    a.kr, a.v, a.beta, a.log = k_raw.data_ptr(), tr["v"].data_ptr(), tr["beta"].data_ptr(), tr["log"].data_ptr()
    a.snap_mass, a.snap_pm, a.snap_m = tr["snap_mass"].data_ptr(), tr["snap_pm"].data_ptr(), tr["snap_m"].data_ptr()
    inv_freq = mod._packed(k_raw.dtype, dev)[2]["inv_freq"]
    a.gamma, a.inv_freq = gam.data_ptr(), inv_freq.data_ptr()
    a.d_slot_k, a.d_slot_v, a.d_m = o["d_slot_k"].data_ptr(), o["d_slot_v"].data_ptr(), o["d_m"].data_ptr()
    a.d_kr, a.d_v, a.d_beta, a.d_gamma = d_kr.data_ptr(), d_v.data_ptr(), d_beta.data_ptr(), d_gamma.data_ptr()
    a.work, a.work_bytes = work.data_ptr(), work.numel()
    A.call("bolt3_chain_bwd", a, dev)
    return d_kr, d_v, d_beta, d_gamma.view(n_steps, b, HKV, -1).sum(dim=(0, 1, 3))


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
        dk_c, dv_c, db_c, dg_c = chain_backward_hip(mod, tr, o, gam, b, n_steps)
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


# the forward's trace entries the backward reads (all tensors)
TRACE_KEYS = ("y", "q_rope", "q_raw", "k_raw", "k_rope", "v", "beta", "eta", "lin_q", "lin_kv", "snap_k", "snap_v",
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
