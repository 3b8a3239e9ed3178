"""bolt3_amd: MI355X-native (gfx950) Bolt-3 Dual-Field attention.

Drop-in for vsa_lm.config.bolt3 (reference tree): ``Bolt3Attn`` and
``Bolt3Decoder`` keep the reference's constructor signatures, parameter names
and methods; the work between the projections and ``o_proj`` runs in the HIP
kernels of ``libbolt3_amd.so`` (C ABI: include/bolt3_amd.h).
"""
from .bolt3 import Bolt3Attn
from .decoder import AnchorCache, Bolt3Decoder, Bolt3LayerState, StaticKV, sample_tokens
from .layers import HybridLM, RMSNorm, RoPE, SoftmaxAttn, MLP

__all__ = ["Bolt3Attn", "Bolt3Decoder", "Bolt3LayerState", "AnchorCache", "StaticKV", "sample_tokens", "HybridLM",
           "RMSNorm", "RoPE", "SoftmaxAttn", "MLP"]
