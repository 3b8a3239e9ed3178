"""ctypes binding of the C ABI declared in include/bolt3_amd.h.

The library is loaded from ``libbolt3_amd.so`` next to this file.  There is no
fallback: if the library is missing or a call returns a non-zero status a
RuntimeError is raised.
"""
from __future__ import annotations

import ctypes as C
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libbolt3_amd.so")

B3_F32, B3_BF16 = 0, 1
ERRORS = {1001: "invalid argument", 1002: "unsupported shape or dtype", 1003: "workspace too small"}

LOG_ROWS, LOG_COLS = 14, 256
LOG_FIELDS = ("rel", "score", "best", "simv", "slot", "merge", "delta", "top_tok", "bot_slot", "win", "keep",
              "top_val", "bot_val", "info")
TIE_TOP, TIE_BOT, TIE_LIMIT = 1, 2, 4

p = C.c_void_p
i32 = C.c_int32
i64 = C.c_int64
f32 = C.c_float


class TensorOut(C.Structure):
    _fields_ = [("p", p), ("sb", i64), ("sh", i64)]


class GateOut(C.Structure):
    _fields_ = [("p", p), ("sb", i64), ("sh", i64)]


class HeadsArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("T", i32), ("H", i32), ("HKV", i32), ("HD", i32),
        ("lin", p), ("lin_row_stride", i64), ("lin_kv", p), ("lin_kv_row_stride", i64), ("parts", i32),
        ("qn_w", p), ("kn_w", p), ("has_qk_norm", i32), ("eps", f32),
        ("inv_freq", p), ("pos0", i32),
        ("q_raw", TensorOut), ("q_rope", TensorOut), ("k_raw", TensorOut), ("k_rope", TensorOut), ("v", TensorOut),
        ("beta", GateOut), ("eta", GateOut), ("pos_out", p), ("gates", p), ("gates_row_stride", i64),
        ("rope_cs", p),
    ]


class ChainArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("HKV", i32), ("HD", i32), ("S", i32),
        ("kr", p), ("kp", p), ("v", p), ("tok_bh_stride", i64), ("pos", p), ("beta", p), ("beta_bh_stride", i64),
        ("n_steps", i32), ("off0", i32), ("len0", i32), ("step_stride", i32), ("step_len", i32), ("n_filled", i32),
        ("kp_exact", i32),
        ("ak", p), ("av", p), ("mass", p), ("util", p), ("pm", p), ("act", p), ("m_res", p),
        ("kappa", p), ("gamma", p), ("inv_freq", p),
        ("snap_k", p), ("snap_v", p), ("snap_bias", p), ("snap_m", p), ("log", p),
        ("work", p), ("work_bytes", i64), ("phase", i32), ("started", p), ("snap_mass", p), ("snap_pm", p),
    ]


class AttnArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("H", i32), ("HKV", i32), ("HD", i32), ("S", i32), ("C", i32), ("n_sinks", i32),
        ("mode", i32), ("n_q", i32), ("score_round", i32),
        ("q_rope", p), ("q_raw", p), ("q_sb", i64), ("q_sh", i64),
        ("eta", p), ("e_sb", i64), ("e_sh", i64),
        ("win_k", p), ("win_v", p), ("w_sb", i64), ("w_sh", i64),
        ("a_start", i32), ("a_len", i32), ("b_start", i32), ("b_len", i32),
        ("sink_k", p), ("sink_v", p), ("s_sb", i64), ("s_sh", i64), ("n_sink_keys", i32),
        ("slot_k", p), ("slot_v", p), ("slot_bias", p), ("slot_step", i64), ("has_slots", i32),
        ("m_res", p), ("m_step", i64), ("m_split", i32),
        ("gamma", p), ("res_w", p), ("eps", f32),
        ("y", p), ("y_sb", i64), ("y_st", i64),
        ("part", i32), ("partial", p), ("chunk_begin", i32), ("chunk_end", i32), ("lse", p),
        ("q_lin", p), ("q_lin_stride", i64), ("qn_w", p), ("qn_eps", f32), ("rope_cs", p),
        ("gates", p), ("gates_stride", i64), ("gates_col", i32),
    ]


class DecodeArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("H", i32), ("HKV", i32), ("HD", i32), ("S", i32),
        ("lin", p), ("lin_row_stride", i64), ("qn_w", p), ("kn_w", p), ("has_qk_norm", i32), ("eps", f32),
        ("inv_freq", p), ("pos", i32),
        ("win_kr", p), ("win_kp", p), ("win_v", p), ("w_sb", i64), ("w_sh", i64),
        ("win_beta", p), ("wb_sb", i64), ("wb_sh", i64), ("win_pos", p),
        ("a_start", i32), ("a_len", i32), ("b_start", i32), ("b_len", i32),
        ("sink_k", p), ("sink_v", p), ("s_sb", i64), ("s_sh", i64), ("n_sink_keys", i32),
        ("slot_k", p), ("slot_v", p), ("slot_bias", p), ("has_slots", i32),
        ("m_res", p), ("gamma", p), ("res_w", p), ("y", p), ("work", p), ("work_bytes", i64),
        ("step_desc", p), ("ring_cap", i32),
    ]


class DecodeLayerArgs(C.Structure):
    _fields_ = [
        ("dec", DecodeArgs), ("x", p), ("x_row_stride", i64), ("d_model", i32),
        ("w_in", p), ("b_in", p), ("n_in", i32), ("w_out", p), ("b_out", p), ("n_out", i32),
        ("out", p), ("out_row_stride", i64), ("proj_work", p), ("proj_work_bytes", i64),
    ]


class SlotKeysArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("HKV", i32), ("HD", i32), ("S", i32),
        ("ak", p), ("pm", p), ("mass", p), ("act", p), ("kappa", p), ("inv_freq", p),
        ("slot_k", p), ("slot_bias", p),
    ]


class AttnBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("T", i32), ("H", i32), ("HKV", i32), ("HD", i32), ("S", i32), ("C", i32),
        ("n_sinks", i32), ("n_chunks", i32), ("n_qtiles", i32), ("n_steps", i32), ("score_round", i32),
        ("q_rope", p), ("q_raw", p), ("q_sb", i64), ("q_sh", i64),
        ("win_k", p), ("win_v", p), ("w_sb", i64), ("w_sh", i64),
        ("slot_k", p), ("slot_v", p), ("slot_bias", p), ("slot_step", i64),
        ("m_res", p), ("m_step", i64), ("m_split", i32),
        ("eta", p), ("e_sb", i64), ("e_sh", i64),
        ("gamma", p), ("res_w", p), ("eps", f32),
        ("y", p), ("y_sb", i64), ("y_st", i64),
        ("dy", p), ("dy_sb", i64), ("dy_st", i64),
        ("d_rows", p), ("lse", p), ("d_q_rope", p), ("d_q_raw", p), ("d_eta", p), ("d_m", p), ("d_res_w", p),
        ("d_gamma", p), ("d_bias", p), ("d_k_own", p), ("d_v_own", p), ("d_k_next", p), ("d_v_next", p),
        ("d_slot_k", p), ("d_slot_v", p), ("d_sink_k", p), ("d_sink_v", p), ("part", i32),
        ("rd_rows", p),
    ]


class RmsNormArgs(C.Structure):
    _fields_ = [("dtype", i32), ("rows", i64), ("dim", i32), ("x", p), ("x_row_stride", i64), ("w", p),
                ("w_dtype", i32), ("y", p), ("y_row_stride", i64), ("eps", f32)]


CHAIN_NOALLOC_SCRATCH_BYTES = 4 << 20   # B3_CHAIN_NOALLOC_SCRATCH_BYTES
# b3_chain_bwd_args.kernels bits (B3_CBWD_*)
CBWD_STATS, CBWD_M_REC, CBWD_SLOT_REC, CBWD_TOK_GRAD = 1, 2, 4, 8

class ChainBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("HKV", i32), ("HD", i32), ("S", i32), ("T", i32),
        ("n_steps", i32), ("off0", i32), ("len0", i32), ("step_stride", i32), ("step_len", i32),
        ("kr", p), ("v", p), ("beta", p), ("log", p), ("snap_mass", p), ("snap_pm", p), ("snap_m", p),
        ("gamma", p), ("inv_freq", p), ("d_slot_k", p), ("d_slot_v", p), ("d_m", p),
        ("d_kr", p), ("d_v", p), ("d_beta", p), ("d_gamma", p), ("work", p), ("work_bytes", i64), ("kernels", i32),
        ("started", p),
    ]


class HeadsBwdArgs(C.Structure):
    _fields_ = [
        ("dtype", i32), ("B", i32), ("T", i32), ("H", i32), ("HKV", i32), ("HD", i32), ("n_sinks", i32),
        ("n_chunks", i32),
        ("d_q_raw", p), ("d_q_rope", p), ("d_k_own", p), ("d_k_next", p), ("d_v_own", p), ("d_v_next", p),
        ("d_sink_k", p), ("d_sink_v", p), ("d_k_chain", p), ("d_v_chain", p), ("d_beta", p), ("d_eta", p),
        ("beta", p), ("eta", p), ("lin_q", p), ("lin_q_row_stride", i64), ("lin_k", p), ("lin_k_row_stride", i64),
        ("qn_w", p), ("kn_w", p), ("has_qk_norm", i32), ("q_eps", f32), ("k_eps", f32), ("inv_freq", p),
        ("dz", p), ("dz_row_stride", i64), ("dz_cols", i32), ("d_qn_w", p), ("d_kn_w", p), ("parts", i32),
    ]


EXPORTS = ("bolt3_attn_bwd", "bolt3_heads", "bolt3_heads_bwd", "bolt3_heads_bwd_blocks", "bolt3_chain",
           "bolt3_chain_bwd", "bolt3_chain_bwd_workspace_bytes",
           "bolt3_chain_noalloc", "bolt3_chain_workspace_bytes", "bolt3_chunk_attn",
           "bolt3_decode",
           "bolt3_decode_layer", "bolt3_decode_layer_workspace_bytes", "bolt3_decode_workspace_bytes",
           "bolt3_rms_norm", "bolt3_slot_keys", "bolt3_step_advance", "bolt3_version", "bolt3_wait_count")

_lib = None


def load():
    """Load the HIP library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                           f"(python -m bolt3_amd.build); there is no CPU implementation")
    lib = C.CDLL(LIB_PATH)
    for name, st in (("bolt3_heads", HeadsArgs), ("bolt3_chain", ChainArgs), ("bolt3_chain_noalloc", ChainArgs),
                     ("bolt3_chunk_attn", AttnArgs),
                     ("bolt3_decode", DecodeArgs), ("bolt3_decode_layer", DecodeLayerArgs),
                     ("bolt3_slot_keys", SlotKeysArgs), ("bolt3_attn_bwd", AttnBwdArgs),
                     ("bolt3_rms_norm", RmsNormArgs), ("bolt3_chain_bwd", ChainBwdArgs),
                     ("bolt3_heads_bwd", HeadsBwdArgs)):
        fn = getattr(lib, name)
        fn.argtypes = [C.POINTER(st), p]
        fn.restype = C.c_int
    lib.bolt3_chain_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32]
    lib.bolt3_chain_workspace_bytes.restype = i64
    lib.bolt3_chain_bwd_workspace_bytes.argtypes = [i32, i32, i32, i32]
    lib.bolt3_chain_bwd_workspace_bytes.restype = i64
    lib.bolt3_heads_bwd_blocks.argtypes = [i32, i32]
    lib.bolt3_heads_bwd_blocks.restype = i32
    lib.bolt3_decode_layer_workspace_bytes.argtypes = [i32, i32, i32, i32, i32]
    lib.bolt3_decode_layer_workspace_bytes.restype = i64
    lib.bolt3_decode_workspace_bytes.argtypes = [i32, i32, i32, i32]
    lib.bolt3_decode_workspace_bytes.restype = i64
    lib.bolt3_step_advance.argtypes = [p, i32, i32, i32, i32, i32, p]
    lib.bolt3_step_advance.restype = C.c_int
    lib.bolt3_wait_count.argtypes = [p, C.c_uint32, i32, p]
    lib.bolt3_wait_count.restype = C.c_int
    lib.bolt3_version.argtypes = []
    lib.bolt3_version.restype = C.c_char_p
    _lib = lib
    return lib


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return B3_F32
    if dt == torch.bfloat16:
        return B3_BF16
    raise TypeError(f"Bolt-3 HIP kernels take float32 or bfloat16 activations, got {dt}")


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_timers: dict | None = None


def set_timing(enabled: bool):
    """Record a HIP event pair around every entry-point launch (on the launch stream) when
    enabled; ``timings()`` then returns {entry point: [milliseconds per launch]}."""
    global _timers
    _timers = {} if enabled else None


_SIDE_STREAMS: dict = {}


def side_stream(dev: torch.device, i: int = 0) -> torch.cuda.Stream:
    """Extra streams per device, at the default priority.  The forward runs the chain's slot
    decisions on 0 and its M_res updates on 1; the backward runs the M_res recursion, the o_proj
    weight gradient and the parameter reductions on 0."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), i)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=dev)
    return _SIDE_STREAMS[key]


def timings() -> dict:
    if _timers is None:
        return {}
    torch.cuda.synchronize()
    return {k: [s.elapsed_time(e) for s, e in v] for k, v in _timers.items()}


def call(name: str, args, device: torch.device):
    stream = torch.cuda.current_stream(device)
    if _timers is not None:
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        ev[0].record(stream)
    rc = getattr(load(), name)(C.byref(args), C.c_void_p(stream.cuda_stream))
    if rc != 0:
        raise RuntimeError(f"{name} failed: {ERRORS.get(rc, f'hip error {rc}')}")
    if _timers is not None:
        ev[1].record(stream)
        _timers.setdefault(name, []).append(ev)


def decode_workspace_bytes(B: int, H: int, HKV: int, HD: int) -> int:
    return int(load().bolt3_decode_workspace_bytes(B, H, HKV, HD))


def decode_layer_workspace_bytes(B: int, d_model: int, n_in: int, hd_total: int, n_out: int) -> int:
    return int(load().bolt3_decode_layer_workspace_bytes(B, d_model, n_in, hd_total, n_out))


def chain_workspace_bytes(dt: torch.dtype, B: int, HKV: int, HD: int, S: int, n_steps: int) -> int:
    return int(load().bolt3_chain_workspace_bytes(dtype_code(dt), B, HKV, HD, S, n_steps))


def chain_bwd_workspace_bytes(B: int, HKV: int, HD: int, n_steps: int) -> int:
    return int(load().bolt3_chain_bwd_workspace_bytes(B, HKV, HD, n_steps))


def heads_bwd_blocks(B: int, T: int) -> int:
    return int(load().bolt3_heads_bwd_blocks(B, T))
