"""Small modules around the Bolt-3 path, with the reference's parameter names.

``RMSNorm`` and ``RoPE`` carry the state-dict names the reference uses
(``weight``; non-persistent buffer ``inv_freq``) so checkpoints load
unchanged.  ``SoftmaxAttn``, ``MLP`` and ``HybridLM`` are the caller side of the
path (the softmax-anchor layers and the model container that
``Bolt3Decoder`` walks); they run as PyTorch ops on the device, except
``RMSNorm``, whose device forward is the library's ``bolt3_rms_norm`` (one pass
per row instead of the torch ops' six; CPU tensors keep the torch ops).
  RMSNorm      -- vsa_lm/surgery.py:43-53
  rope_inv_freq-- vsa_lm/surgery.py:56-72
  RoPE         -- vsa_lm/surgery.py:80-93
  MLP          -- vsa_lm/surgery.py:202-211
  SoftmaxAttn  -- vsa_lm/config/standard.py:55-122 (plain, un-gated variant)
  HybridLM     -- vsa_lm/config/standard.py:341-404 (UniversalBlock / UniversalVSALM names)
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda and _hip_norm_ok(x, self.weight):
            return _rms_norm_hip(x, self.weight, self.eps)
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (xf * self.weight.float()).to(x.dtype)


def _hip_norm_ok(x: torch.Tensor, w: torch.Tensor) -> bool:
    """bolt3_rms_norm takes the device forward when nothing asks for a gradient (it has no
    backward) and the shape and dtypes are its own; CPU tensors keep the torch ops."""
    needs_grad = torch.is_grad_enabled() and (x.requires_grad or w.requires_grad)
    return (not needs_grad and x.dtype in (torch.float32, torch.bfloat16) and
            w.dtype in (torch.float32, torch.bfloat16) and x.shape[-1] % 8 == 0 and x.numel() > 0)


def _rms_norm_hip(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    from . import _abi as A
    D = x.shape[-1]
    x2 = x.reshape(-1, D)
    if x2.stride(-1) != 1 or (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    y = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    wc = w.detach().contiguous()
    a = A.RmsNormArgs()
    a.dtype, a.rows, a.dim = A.dtype_code(x.dtype), x2.shape[0], D
    a.x, a.x_row_stride, a.w, a.w_dtype = x2.data_ptr(), x2.stride(0), wc.data_ptr(), A.dtype_code(wc.dtype)
    a.y, a.y_row_stride, a.eps = y.data_ptr(), y.stride(0), float(eps)
    A.call("bolt3_rms_norm", a, x.device)
    return y.view(x.shape)


def rope_inv_freq(head_dim: int, theta: float, rope_scaling: dict | None = None) -> torch.Tensor:
    """theta^(-2i/HD), with the llama3 frequency-band rescaling when requested."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    if rope_scaling and rope_scaling.get("rope_type") == "llama3":
        ctx = float(rope_scaling["original_max_position_embeddings"])
        factor = float(rope_scaling["factor"])
        lo, hi = float(rope_scaling["low_freq_factor"]), float(rope_scaling["high_freq_factor"])
        wl = 2.0 * math.pi / inv
        scaled = torch.where(wl > ctx / lo, inv / factor, inv)
        blend = (ctx / wl - lo) / (hi - lo)
        mixed = (1.0 - blend) * scaled / factor + blend * scaled
        mid = ~(wl < ctx / hi) & ~(wl > ctx / lo)
        inv = torch.where(mid, mixed, scaled)
    return inv


class RoPE(nn.Module):
    def __init__(self, head_dim: int, theta: float, rope_scaling: dict | None = None):
        super().__init__()
        self.register_buffer("inv_freq", rope_inv_freq(head_dim, theta, rope_scaling), persistent=False)

    def forward(self, x: torch.Tensor, pos_start: int = 0) -> torch.Tensor:
        t = torch.arange(pos_start, pos_start + x.shape[2], device=x.device, dtype=torch.float32)
        ang = t[:, None] * self.inv_freq.to(x.device)
        ang = torch.cat((ang, ang), dim=-1)
        half = x.shape[-1] // 2
        rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return x * ang.cos().to(x.dtype)[None, None] + rot * ang.sin().to(x.dtype)[None, None]


class MLP(nn.Module):
    def __init__(self, cfg: dict):
        super().__init__()
        D, I = cfg["dim"], cfg["intermediate"]
        self.gate_proj = nn.Linear(D, I, bias=False)
        self.up_proj = nn.Linear(D, I, bias=False)
        self.down_proj = nn.Linear(I, D, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class SoftmaxAttn(nn.Module):
    """Causal softmax-anchor layer of a hybrid stack."""

    def __init__(self, cfg: dict):
        super().__init__()
        D, H, HKV = cfg["dim"], cfg["num_heads"], cfg["num_kv_heads"]
        HD = cfg.get("head_dim") or (D // H)
        bias = bool(cfg.get("qkv_bias", False))
        self.H, self.HKV, self.HD, self.G = H, HKV, HD, H // HKV
        self.q_proj = nn.Linear(D, H * HD, bias=bias)
        self.k_proj = nn.Linear(D, HKV * HD, bias=bias)
        self.v_proj = nn.Linear(D, HKV * HD, bias=bias)
        self.o_proj = nn.Linear(H * HD, D, bias=False)
        if cfg.get("qk_norm", False):
            self.q_norm, self.k_norm = RMSNorm(HD, cfg["eps"]), RMSNorm(HD, cfg["eps"])
        else:
            self.q_norm = self.k_norm = None
        self.rope = RoPE(HD, cfg["rope_theta"], cfg.get("rope_scaling"))

    def head_qkv(self, x):
        b, t, _ = x.shape
        q = self.q_proj(x).view(b, t, self.H, self.HD)
        k = self.k_proj(x).view(b, t, self.HKV, self.HD)
        v = self.v_proj(x).view(b, t, self.HKV, self.HD)
        if self.q_norm is not None:
            q, k = self.q_norm(q), self.k_norm(k)
        return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)

    def forward(self, x):
        b, t, _ = x.shape
        q, k, v = self.head_qkv(x)
        q, k = self.rope(q), self.rope(k)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=self.G > 1)
        return self.o_proj(y.transpose(1, 2).reshape(b, t, self.H * self.HD))


class Block(nn.Module):
    def __init__(self, cfg: dict, kind: str):
        super().__init__()
        from .bolt3 import Bolt3Attn
        self.norm1 = RMSNorm(cfg["dim"], cfg["eps"])
        if kind == "vsa":
            self.vsa = Bolt3Attn(cfg, max_T=cfg.get("max_T", 2048), S=int(cfg.get("bolt3_S", 128)),
                                 C=int(cfg.get("bolt3_C", 128)))
        else:
            self.attn = SoftmaxAttn(cfg)
        self.norm2 = RMSNorm(cfg["dim"], cfg["eps"])
        self.mlp = MLP(cfg)

    def forward(self, x):
        attn = self.vsa if hasattr(self, "vsa") else self.attn
        x = x + attn(self.norm1(x))
        return x + self.mlp(self.norm2(x))


class HybridLM(nn.Module):
    """Hybrid Bolt-3 / softmax language model with UniversalVSALM's attribute names."""

    def __init__(self, vocab_size: int, dim: int, num_layers: int, num_heads: int, num_kv_heads: int,
                 intermediate: int, layer_types: list[str] | None = None, hybrid_every: int = 4,
                 max_T: int = 2048, rope_theta: float = 10000.0, rope_scaling: dict | None = None,
                 eps: float = 1e-5, head_dim: int | None = None, qkv_bias: bool = False,
                 tie_word_embeddings: bool = True, **extra):
        super().__init__()
        head_dim = head_dim or dim // num_heads
        if layer_types is None:
            layer_types = ["softmax" if hybrid_every > 0 and (li + 1) % hybrid_every == 0 else "vsa"
                           for li in range(num_layers)]
        self.config = dict(vocab_size=vocab_size, dim=dim, num_layers=num_layers, num_heads=num_heads,
                           num_kv_heads=num_kv_heads, intermediate=intermediate, max_T=max_T,
                           rope_theta=rope_theta, rope_scaling=rope_scaling, eps=eps, head_dim=head_dim,
                           qkv_bias=qkv_bias, tie_word_embeddings=tie_word_embeddings, layer_types=layer_types,
                           hybrid_every=hybrid_every, **extra)
        self.config.setdefault("is_bolt3", True)
        self.embed_tokens = nn.Embedding(vocab_size, dim)
        self.blocks = nn.ModuleList(Block(self.config, k) for k in layer_types)
        self.norm = RMSNorm(dim, eps)
        self.lm_head = nn.Linear(dim, vocab_size, bias=False)
        if tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight

    def forward(self, input_ids):
        x = self.embed_tokens(input_ids)
        for blk in self.blocks:
            x = blk(x)
        return self.norm(x)
