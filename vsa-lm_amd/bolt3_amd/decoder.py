"""Bolt-3 decoder on MI355X: constant-memory generation over a hybrid stack.

Drop-in for ``Bolt3Decoder`` of vsa_lm/config/bolt3.py:279-557 (reference
tree): same constructor, ``step`` / ``prefill`` / ``generate_batch`` /
``generate`` / ``continue_generate`` / ``memorize`` / ``forget`` /
``blank_state`` / ``state_bytes`` / ``_sample`` with the reference's argument
meaning and results.

Design (not the reference's):
  * Bolt-3 layers keep their whole state in preallocated device buffers
    (``Bolt3LayerState``: a window ring, sinks, slots with cached roped keys,
    M_res) and step through the HIP entry points: one ``bolt3_decode_layer``
    call per token in bf16 (both projections included), ``bolt3_chain`` when a
    chunk leaves the window.
  * Softmax-anchor layers keep keys and values in an ``AnchorCache`` that grows
    by whole pages.
  * ``generate_batch`` keeps its bookkeeping on the device (tokens, end of
    sequence, lengths, the forced close-of-thinking sequence) and never waits
    for the GPU inside the loop: the all-rows-done test the reference makes
    every 16 tokens is read back one period later from a copy taken then, and
    the output is cut where the reference would have stopped.
"""
from __future__ import annotations

from collections.abc import MutableMapping

import torch
import torch.nn.functional as F

from . import _abi as A
from .bolt3 import N_SINKS, Bolt3Attn, _check_dtype, _gout, _tout

DONE_CHECK_EVERY = 16      # tokens between the all-rows-done tests (the reference's period)


def _check_m_state(m: torch.Tensor, B: int, ly: Bolt3Attn):
    """The kernels read and write M_res as contiguous fp32 [B][HKV][HD][HD] on the device."""
    want = (B, ly.HKV, ly.HD, ly.HD)
    if m.dtype != torch.float32 or tuple(m.shape) != want or not m.is_contiguous() or not m.is_cuda:
        raise TypeError(f"M_res state must be a contiguous fp32 device tensor of shape {want}; "
                        f"got {m.dtype} {tuple(m.shape)} contiguous={m.is_contiguous()} on {m.device}")


def _check_step_len(ly: Bolt3Attn, st: "Bolt3LayerState", t: int):
    """A step's tokens join the current chunk, which the reference consolidates whole once it holds
    C or more (vsa_lm/config/bolt3.py:404-425): with the tokens already in it, at most 2C per
    chunk (a ring half; the chain takes at most 256 tokens per consolidation)."""
    if st.cur[1] + t > 2 * ly.C:
        raise NotImplementedError(
            f"a step of {t} tokens on a current chunk of {st.cur[1]} would make a chunk of more than 2C = "
            f"{2 * ly.C} tokens, which the reference consolidates as one (the chain takes at most {2 * ly.C}); "
            f"feed longer inputs through prefill or in pieces of at most C tokens")


def _fused_step_ok(dt: torch.dtype, d_model: int, hd_total: int, n_out: int) -> bool:
    """Whether bolt3_decode_layer takes this layer: bf16, input width a multiple of 32, output width
    a multiple of 16, and at most 8 K chunks of 512 in either projection."""
    return dt == torch.bfloat16 and d_model >= 32 and d_model % 32 == 0 and n_out % 16 == 0 and \
        (d_model + 511) // 512 <= 8 and (hd_total + 511) // 512 <= 8


class AnchorCache:
    """Key/value cache of one softmax-anchor layer.

    Same surface as the reference's StaticKV (vsa_lm/decode.py:88-106): tensors
    ``k`` / ``v`` of shape [B, HKV, capacity, HD], the count ``n`` of cached
    tokens, and ``append(k, v)`` returning the cached prefix.  Capacity is a
    whole number of PAGE-token pages and at least doubles when it grows.
    """

    PAGE = 256

    def __init__(self, B: int, HKV: int, Tmax: int, HD: int, dev, dt=torch.bfloat16):
        cap = -(-max(int(Tmax), 1) // self.PAGE) * self.PAGE
        self.k = torch.empty(B, HKV, cap, HD, device=dev, dtype=dt)
        self.v = torch.empty_like(self.k)
        self.n = 0

    @property
    def capacity(self) -> int:
        return self.k.shape[2]

    def reserve(self, tokens: int):
        if tokens <= self.capacity:
            return
        pages = -(-max(tokens, 2 * self.capacity) // self.PAGE)
        for name in ("k", "v"):
            old = getattr(self, name)
            new = old.new_empty(*old.shape[:2], pages * self.PAGE, old.shape[3])
            new.narrow(2, 0, self.n).copy_(old.narrow(2, 0, self.n))
            setattr(self, name, new)

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor):
        t = k_new.shape[2]
        self.reserve(self.n + t)
        self.k.narrow(2, self.n, t).copy_(k_new)
        self.v.narrow(2, self.n, t).copy_(v_new)
        self.n += t
        return self.k.narrow(2, 0, self.n), self.v.narrow(2, 0, self.n)


# the reference's name for the softmax layers' cache
StaticKV = AnchorCache


class Bolt3LayerState(MutableMapping):
    """Decoder state of one Bolt-3 layer in preallocated device buffers.

    The window is a ring of two halves of 2C tokens each: the previous chunk
    ("prev") in one half, the chunk being filled ("cur") in the other.  Slot
    state keeps the un-roped keys (ak) plus a cache of the keys roped at their
    mean positions (slot_k) and the attention bias (slot_bias), refreshed by
    every consolidation.  No tensor grows while decoding (the reference
    concatenates).

    It is a mapping with the keys of the reference's per-layer kv_caches dict
    (vsa_lm/config/bolt3.py:310-315): reading a key gives a view in the
    reference's shape (None for an empty part), assigning one rewrites the
    state, ``to_dict`` / ``from_dict`` convert both ways (the form the memory
    bank saves, vsa_lm/memory_bank.py:57-68).
    """

    KEYS = ("ak", "av", "mass", "util", "pm", "act", "sink_k", "sink_v", "prev_kr", "prev_kp", "prev_v",
            "prev_pos", "prev_b", "cur_kr", "cur_kp", "cur_v", "cur_pos", "cur_b", "n_filled")

    def __init__(self, ly: Bolt3Attn, B: int, device, dtype):
        C, S, HKV, HD = ly.C, ly.S, ly.HKV, ly.HD
        self.B, self.C, self.S, self.HKV, self.HD, self.dtype = B, C, S, HKV, HD, dtype
        self._ly = ly
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
        if key in ("ak", "av"):   # [bh, S, HD], as _consolidate_functional returns them
            return self.slots[key] if self.has_slots else None
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

    # ------------------------------------------------------------ mapping with the reference's keys

    def __iter__(self):
        return iter(self.KEYS)

    def __len__(self):
        return len(self.KEYS)

    def __setitem__(self, key, value):
        if key not in self.KEYS:
            raise KeyError(key)
        d = self.to_dict()
        d[key] = value
        self.load_dict(d)

    def __delitem__(self, key):
        raise TypeError("Bolt3LayerState has a fixed key set; assign None to clear a part")

    def to_dict(self) -> dict:
        """Snapshot in the reference's kv_caches form (tensors copied, n_filled an int)."""
        out = {}
        for k in self.KEYS:
            v = self[k]
            out[k] = v.clone() if torch.is_tensor(v) else v
        return out

    @classmethod
    def from_dict(cls, ly: "Bolt3Attn", d: dict, device=None, dtype=None) -> "Bolt3LayerState":
        """State of layer ``ly`` from a reference kv_caches dict (any device; tensors are copied)."""
        ref = next((v for v in d.values() if torch.is_tensor(v) and v.dim() == 4), None)
        if ref is None:
            raise ValueError("the dict holds no window, sink or slot tensors to size the state from")
        B = ref.shape[0] if d.get("ak") is None else d["ak"].numel() // (ly.HKV * ly.S * ly.HD)
        device = torch.device(device) if device is not None else ref.device
        dtype = dtype or (d["ak"].dtype if d.get("ak") is not None else ref.dtype)
        st = cls(ly, B, device, dtype)
        st.load_dict(d)
        return st

    def load_dict(self, d: dict):
        """Rewrite the whole state from a reference kv_caches dict.  The previous chunk goes to the
        ring's first half, the current one to its second; the roped slot keys and the slot bias are
        rebuilt from ak, pm, mass and act by the chain's own rotation (bolt3_slot_keys)."""
        B, HKV, HD, S, C, dt = self.B, self.HKV, self.HD, self.S, self.C, self.dtype
        dev = self.win_kr.device
        bh = B * HKV

        def put(dst, src, shape):
            dst.copy_(src.detach().reshape(shape).to(device=dev, dtype=dst.dtype))

        if d.get("ak") is None:
            for k, v in self._ly._empty_slots(bh, dt, dev).items():
                self.slots[k].copy_(v)
            self.has_slots = False
        else:
            for k in ("ak", "av"):
                put(self.slots[k], d[k], (bh, S, HD))
            for k in ("mass", "util", "pm"):
                put(self.slots[k], d[k], (bh, S))
            put(self.slots["act"], d["act"].to(torch.uint8), (bh, S))
            self.has_slots = True
            self._refresh_slot_keys()
        self.n_filled = int(d.get("n_filled") or 0)
        if d.get("sink_k") is None:
            self.n_sink = 0
        else:
            ns = d["sink_k"].shape[2]
            if ns > N_SINKS:
                raise ValueError(f"{ns} sink tokens; the state holds at most {N_SINKS}")
            put(self.sink_k[:, :, :ns], d["sink_k"], (B, HKV, ns, HD))
            put(self.sink_v[:, :, :ns], d["sink_v"], (B, HKV, ns, HD))
            self.n_sink = ns
        for pre, start in (("prev_", 0), ("cur_", 2 * C)):
            kp = d.get(pre + "kp")
            n = 0 if kp is None else kp.shape[2]
            if n > 2 * C:
                raise ValueError(f"{pre}* holds {n} tokens; a ring half holds at most {2 * C}")
            if n:
                put(self.win_kr[:, :, start:start + n], d[pre + "kr"], (B, HKV, n, HD))
                put(self.win_kp[:, :, start:start + n], kp, (B, HKV, n, HD))
                put(self.win_v[:, :, start:start + n], d[pre + "v"], (B, HKV, n, HD))
                put(self.win_b[:, :, start:start + n], d[pre + "b"], (B, HKV, n))
                put(self.win_pos[start:start + n], d[pre + "pos"], (n,))
            if pre == "prev_":
                self.prev = (start, n)
            else:
                self.cur = (start, n)

    def _refresh_slot_keys(self):
        ly = self._ly
        dev = self.win_kr.device
        a = A.SlotKeysArgs()
        a.dtype, a.B, a.HKV, a.HD, a.S = A.dtype_code(self.dtype), self.B, self.HKV, self.HD, self.S
        a.ak, a.pm, a.mass, a.act = (self.slots[k].data_ptr() for k in ("ak", "pm", "mass", "act"))
        # fp32 copies bound to names until the launch is queued: a bf16 module's kappa and
        # inv_freq are converted here, and a temporary freed before the launch could hand its
        # block to the next conversion
        kappa = ly.kappa.detach().to(device=dev, dtype=torch.float32).contiguous()
        inv_freq = ly.rope.inv_freq.to(device=dev, dtype=torch.float32).contiguous()
        a.kappa, a.inv_freq = kappa.data_ptr(), inv_freq.data_ptr()
        a.slot_k, a.slot_bias = self.slot_k.data_ptr(), self.slot_bias.data_ptr()
        A.call("bolt3_slot_keys", a, dev)
        del kappa, inv_freq





def sample_tokens(logits: torch.Tensor, temperature: float, top_k: int = 40, top_p: float = 0.95) -> torch.Tensor:
    """Next token per row, [B, 1] (vsa_lm/config/bolt3.py:321-333): greedy at temperature <= 1e-5;
    otherwise nucleus sampling of softmax(logits / temperature) when top_p < 1 (the smallest set of
    most likely tokens whose mass before the last one is at most top_p), else sampling among the
    top_k logits.  One multinomial draw per call, on the logits' device."""
    if temperature <= 1e-5:
        return logits.argmax(dim=-1, keepdim=True)
    z = logits.float() / temperature
    if top_p < 1.0:
        prob, order = torch.softmax(z, dim=-1).sort(dim=-1, descending=True)
        ahead = prob.cumsum(dim=-1) - prob           # probability mass ranked above each token
        prob = prob.masked_fill(ahead > top_p, 0.0)
        prob = prob / prob.sum(dim=-1, keepdim=True).clamp_min(1e-12)
        return torch.gather(order, -1, torch.multinomial(prob, 1))
    vals, idx = torch.topk(z, min(top_k, z.shape[-1]), dim=-1)
    return torch.gather(idx, -1, torch.multinomial(torch.softmax(vals, dim=-1), 1))


class _Bookkeeping:
    """Per-row generation state on the device (vsa_lm/config/bolt3.py:464-494): the tokens, which
    rows ended (eos) and after how many tokens, and the close-of-thinking sequence forced on rows
    still thinking once the budget point is reached."""

    def __init__(self, B: int, n_max: int, eos_ids, close_ids, dev):
        self.n_max = n_max
        self.toks = torch.zeros(B, n_max, dtype=torch.long, device=dev)
        self.lengths = torch.full((B,), n_max, dtype=torch.long, device=dev)
        self.done = torch.zeros(B, dtype=torch.bool, device=dev)
        self.eos = torch.tensor(sorted(eos_ids or ()), dtype=torch.long, device=dev)
        self.close = torch.tensor(list(close_ids or ()), dtype=torch.long, device=dev)
        self.end_think = int(close_ids[1]) if close_ids and len(close_ids) > 1 else None
        self.closed = torch.zeros(B, dtype=torch.bool, device=dev)
        self.cursor = torch.full((B,), -1, dtype=torch.long, device=dev)   # next forced index, -1: none
        self.budget = max(64, n_max - 64)
        self._flag = torch.zeros(1, dtype=torch.bool).pin_memory() if torch.cuda.is_available() else None
        self._flag_at = None
        self._flag_ev = None

    def take(self, i: int, nxt: torch.Tensor) -> torch.Tensor:
        """Record token i of every row ([B, 1]) after the forced sequence is applied."""
        n_close = self.close.numel()
        if n_close:
            if i == self.budget:
                start = ~self.closed & ~self.done & (self.cursor < 0)
                self.cursor = torch.where(start, torch.zeros_like(self.cursor), self.cursor)
            forcing = self.cursor >= 0
            forced = self.close[self.cursor.clamp(0, n_close - 1)]
            nxt = torch.where(forcing.unsqueeze(1), forced.unsqueeze(1), nxt)
            self.cursor = torch.where(forcing, self.cursor + 1, self.cursor)
            finished = forcing & (self.cursor >= n_close)
            self.cursor = torch.where(finished, torch.full_like(self.cursor, -1), self.cursor)
            self.closed = self.closed | finished
            if self.end_think is not None:
                self.closed = self.closed | (nxt[:, 0] == self.end_think)
        self.toks[:, i] = nxt[:, 0]
        if self.eos.numel():
            hit = torch.isin(nxt[:, 0], self.eos) & ~self.done
            self.lengths = torch.where(hit, torch.full_like(self.lengths, i + 1), self.lengths)
            self.done = self.done | hit
        return nxt

    def stop_at(self, i: int) -> int | None:
        """Token count at which the reference would have stopped, as far as known now.  At every
        DONE_CHECK_EVERY-th token the all-done flag is copied to host memory without waiting; it is
        read at the next check (or at the end), by which time the copy has long finished."""
        if not self.eos.numel():
            return None
        last = i == self.n_max - 1
        if i % DONE_CHECK_EVERY != DONE_CHECK_EVERY - 1 and not last:
            return None
        stop = None
        if self._flag_at is not None:
            self._flag_ev.synchronize()
            if bool(self._flag[0]):
                stop = self._flag_at + 1
            self._flag_at = None
        if stop is None and i % DONE_CHECK_EVERY == DONE_CHECK_EVERY - 1:
            self._flag.copy_(self.done.all().view(1), non_blocking=True)
            self._flag_ev = torch.cuda.Event()
            self._flag_ev.record()
            self._flag_at = i
            if last:                         # nothing runs after the last token: read it now
                self._flag_ev.synchronize()
                stop = i + 1 if bool(self._flag[0]) else None
        return stop


class Bolt3Decoder:
    """Constant-memory decoder over a hybrid Bolt-3 / softmax stack (vsa_lm/config/bolt3.py:279-557)."""

    def __init__(self, model, wrap_positions: bool = False, max_cache_pos: int = 65536, **kwargs):
        self.model = model.eval()
        self.max_T = model.config["max_T"]
        self.max_cache_pos = max_cache_pos
        self.wrap_positions = wrap_positions
        self.C = int(model.config.get("bolt3_C", 128))
        # bf16 one-token steps run as one bolt3_decode_layer call (projections included); False
        # keeps the projections in torch around bolt3_decode (the tests compare the two)
        self.fuse_projections = True
        # generate_batch replays a captured graph of the one-token step when the stack allows it
        self.use_graphs = True
        self._anchor_packs: dict = {}
        self._scratch_bufs: dict = {}

    def _graph_runner(self, B: int, need_len: int, device, states=None, kv_caches=None, pos: int = 0):
        """A DecodeGraph of the one-token step for this state (anchor caches sized for need_len
        tokens), or None when some layer cannot take it (not bf16, or outside the fused step's
        limits).  The reference has no graph (vsa_lm/config/bolt3.py:287-288)."""
        if states is None or not self.use_graphs or not self.fuse_projections:
            return None
        if not DecodeGraph.supported(self.model):
            return None
        return DecodeGraph(self, states, kv_caches, B, need_len, torch.device(device), pos)

    # ------------------------------------------------------------ state

    @staticmethod
    def state_bytes(model):
        """(bytes that do not grow with the context, bytes per cached token) of a decode state, counted
        as the reference counts them (vsa_lm/config/bolt3.py:290-300): M_res in fp32, slot keys and
        values, a window of two chunks of keys and values, anchor keys and values, all at 2 bytes."""
        fixed = per_token = 0
        for blk in model.blocks:
            if hasattr(blk, "vsa"):
                a = blk.vsa
                row = a.HKV * a.HD                    # one token's (or slot's) keys across kv heads
                fixed += row * a.HD * 4 + (2 * a.S + 4 * a.C) * row * 2
            else:
                per_token += 4 * blk.attn.HKV * blk.attn.HD
        return fixed, per_token

    @staticmethod
    def blank_state(model, batch_size: int, device, max_kv_len: int = 4096, state_dtype=torch.float32,
                    dtype=None, **kwargs):
        """Empty decode state: M_res per Bolt-3 layer (fp32 [B, HKV, HD, HD], None for anchors) and a
        cache per layer (Bolt3LayerState / AnchorCache) in the model's activation dtype."""
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError("Bolt3Decoder.blank_state: the Bolt-3 HIP path needs a ROCm device")
        if state_dtype != torch.float32:
            raise TypeError(f"M_res is kept in fp32 by the kernels (state_dtype={state_dtype} requested)")
        dt = dtype or next(model.parameters()).dtype
        states, caches = [], []
        for blk in model.blocks:
            if hasattr(blk, "vsa"):
                ly = blk.vsa
                states.append(torch.zeros(batch_size, ly.HKV, ly.HD, ly.HD, device=device))
                caches.append(Bolt3LayerState(ly, batch_size, device, dt))
            else:
                states.append(None)
                caches.append(AnchorCache(batch_size, blk.attn.HKV, max_kv_len, blk.attn.HD, device, dt))
        return states, caches

    @staticmethod
    def _sample(logits, temperature: float, top_k: int = 40, top_p: float = 0.95):
        return sample_tokens(logits, temperature, top_k, top_p)

    # ------------------------------------------------------------ one Bolt-3 layer

    def _bolt3_layer(self, ly: Bolt3Attn, h, pos_start: int, m_state: torch.Tensor, st: Bolt3LayerState,
                     record=None, desc: int | None = None):
        """One step of a Bolt-3 layer on t tokens.  ``desc``: device address of a step descriptor
        (graph capture): the fused one-token kernels then take the position and ring segments from
        it, and the ring bookkeeping and consolidation are left to the caller."""
        B, t, _ = h.shape
        dt, dev = h.dtype, h.device
        if dt != st.dtype:
            raise TypeError(f"activation dtype {dt} differs from the decoder state dtype {st.dtype}")
        _check_m_state(m_state, B, ly)
        _check_step_len(ly, st, t)
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
            fused = self.fuse_projections and _fused_step_ok(dt, h.shape[-1], H * HD, side["wo"].shape[0])
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
                a.step_desc, a.ring_cap = desc, st.cap
                A.call("bolt3_decode_layer", call_args, dev)
                a.step_desc = None
                if desc is None:
                    st.cur = (cs, cl + 1)
                    if st.cur[1] >= ly.C:
                        self._consolidate(ly, st, m_state, gam, side, record)
                return out
            if desc is not None:
                raise NotImplementedError("graph-captured steps need the fused bf16 layer step")
            lin = F.linear(h, W, bias)
            _check_dtype(lin, dt, "packed projection")
            a.lin = lin.data_ptr()
            A.call("bolt3_decode", a, dev)
            y = y.view(B, 1, H * HD)
        else:
            lin = F.linear(h, W, bias)
            _check_dtype(lin, dt, "packed projection")
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

    def _bolt3_prefill(self, ly: Bolt3Attn, h: torch.Tensor, m_state: torch.Tensor, st: Bolt3LayerState,
                       record=None):
        """A whole prompt through one Bolt-3 layer from an empty state, as the forward computes it
        (every chunk's attention at once, the chain in step groups beside it) with the decoder
        step's fp32 scores; then the state the reference's chunk-by-chunk prefill leaves
        (vsa_lm/config/bolt3.py:452-457): with n = T // C full chunks, chunks 0 .. n-2 consolidated,
        chunk n-1 as prev, the remaining tokens as cur.  The forward consolidates ceil(T/C) - 2
        chunks, one fewer when C divides T; that step runs here.  Returns the layer output.
        ``record`` (a list) receives the decision log of every consolidation, as ``step`` records."""
        B, T, _ = h.shape
        C, S, HD, HKV = ly.C, ly.S, ly.HD, ly.HKV
        dt, dev = h.dtype, h.device
        tr = {}
        out = ly._forward_hip(h, tr, score_round=0, keep_log=record is not None)
        side = ly._packed(dt, dev)[2]
        gam = side["gamma"]
        n_full = T // C
        n_steps = max(0, (T + C - 1) // C - 2)
        ns = min(ly.n_sinks, C)
        k_raw, k_rope, v, beta, pos = tr["k_raw"], tr["k_rope"], tr["v"], tr["beta"], tr["pos"]
        if n_steps > 0:
            slots, m_res, nf = tr["state"], tr["m_res"], tr["n_filled"]
            if record is not None:
                nf_i = 0
                for i in range(n_steps):
                    l_i = C - ns if i == 0 else C
                    record.append(dict(log=tr["log"][i], n_filled=nf_i, tokens=l_i))
                    nf_i = min(S, nf_i + l_i)
        else:
            slots, m_res, nf = ly._empty_slots(B * HKV, dt, dev), torch.zeros(B * HKV, HD, HD, device=dev), 0
        if T % C == 0 and n_full >= 2:
            i = n_full - 2                       # the step the forward leaves out
            off, l = (ns, C - ns) if i == 0 else (0, C)
            esz = k_raw.element_size()
            tok = i * C
            log = None
            if record is not None:
                log = torch.zeros(1, B * HKV, A.LOG_ROWS, A.LOG_COLS, device=dev)
                record.append(dict(log=log[0], n_filled=nf, tokens=l))
            ly._chain(dt, dev, B, k_raw.data_ptr() + tok * HD * esz, k_rope.data_ptr() + tok * HD * esz,
                      v.data_ptr() + tok * HD * esz, T * HD, pos.data_ptr() + tok * 4, beta.data_ptr() + tok * 4,
                      T, 1, off, l, C, C, nf, slots, m_res, gam, side, kp_exact=True, log=log)
            nf = min(S, nf + l)
            n_steps += 1
        m_state.copy_(m_res.view_as(m_state))
        # the reference's kv_caches form, loaded like any saved state
        d = dict.fromkeys(Bolt3LayerState.KEYS)
        d["n_filled"] = nf if n_steps > 0 else 0
        if n_steps > 0:
            d.update(ak=slots["ak"], av=slots["av"], mass=slots["mass"], util=slots["util"], pm=slots["pm"],
                     act=slots["act"].bool(), sink_k=k_rope[:, :, :ns], sink_v=v[:, :, :ns])
        for pre, (t0, t1) in (("prev_", ((n_full - 1) * C, n_full * C)), ("cur_", (n_full * C, T))):
            if t1 > t0 >= 0:
                d.update({pre + "kr": k_raw[:, :, t0:t1], pre + "kp": k_rope[:, :, t0:t1], pre + "v": v[:, :, t0:t1],
                          pre + "b": beta[:, :, t0:t1], pre + "pos": pos[t0:t1].view(1, 1, -1)})
        st.load_dict(d)
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

    # ------------------------------------------------------------ one softmax-anchor layer

    def _anchor_pack(self, ly, dt: torch.dtype, dev: torch.device):
        """(W_in rows q | k | v padded to 16, their bias or None, side tensors) of a softmax layer's
        fused one-token step, rebuilt when a parameter changes."""
        params = list(ly.parameters())
        key = (dt, dev, tuple((q.data_ptr(), q._version) for q in params))
        ent = self._anchor_packs.get(id(ly))
        if ent is not None and ent[0] == key:
            return ent[1]
        with torch.no_grad():
            lins = (ly.q_proj, ly.k_proj, ly.v_proj)
            D = ly.q_proj.in_features
            pad = (-sum(m.out_features for m in lins)) % 16
            W = torch.cat([m.weight.to(device=dev, dtype=dt) for m in lins] +
                          [torch.zeros(pad, D, device=dev, dtype=dt)]).contiguous()
            bias = None
            if any(m.bias is not None for m in lins):
                bias = torch.cat([(m.bias if m.bias is not None else torch.zeros(m.out_features)).to(dev, dt)
                                  for m in lins] + [torch.zeros(pad, device=dev, dtype=dt)]).contiguous()
            norm = ly.q_norm is not None
            side = dict(wo=ly.o_proj.weight.to(device=dev, dtype=dt).contiguous(),
                        inv_freq=ly.rope.inv_freq.to(dev).float().contiguous(),
                        qn=ly.q_norm.weight.detach().to(dev).float().contiguous() if norm else None,
                        kn=ly.k_norm.weight.detach().to(dev).float().contiguous() if norm else None,
                        eps=float(ly.q_norm.eps) if norm else 1e-6,
                        gamma=torch.zeros(ly.HKV, device=dev), res_w=torch.ones(ly.HD, device=dev))
        self._anchor_packs[id(ly)] = (key, (W, bias, side))
        return W, bias, side

    def _scratch(self, dev, name: str, n_floats: int) -> torch.Tensor:
        """Kernel workspaces kept per device and purpose (stable addresses for captured graphs)."""
        t = self._scratch_bufs.get((dev, name))
        if t is None or t.numel() < n_floats:
            t = torch.empty(n_floats, device=dev)
            self._scratch_bufs[(dev, name)] = t
        return t

    def _anchor_fused(self, ly, h: torch.Tensor, pos_start: int, cache: AnchorCache, desc: int | None = None):
        """One token of a softmax-anchor layer as one bolt3_decode_layer call in its anchor mode:
        q | k | v projection, q/k norm and RoPE, the new key and value appended to the cache,
        causal softmax over the cache, o_proj.  ``desc`` as in _bolt3_layer (cache.n is then the
        caller's to advance)."""
        B, _, D = h.shape
        dt, dev = h.dtype, h.device
        W, bias, side = self._anchor_pack(ly, dt, dev)
        if desc is None:
            cache.reserve(cache.n + 1)
        H, HKV, HD = ly.H, ly.HKV, ly.HD
        n_out = side["wo"].shape[0]
        la = A.DecodeLayerArgs()
        a = la.dec
        a.dtype, a.B, a.H, a.HKV, a.HD, a.S = A.dtype_code(dt), B, H, HKV, HD, 128
        a.lin_row_stride = W.shape[0]
        a.qn_w, a.kn_w, a.has_qk_norm = A.ptr(side["qn"]), A.ptr(side["kn"]), int(side["qn"] is not None)
        a.eps, a.inv_freq, a.pos = side["eps"], side["inv_freq"].data_ptr(), int(pos_start)
        a.win_kr, a.win_kp, a.win_v = None, cache.k.data_ptr(), cache.v.data_ptr()
        a.w_sb, a.w_sh = cache.k.stride(0), cache.k.stride(1)
        a.win_beta, a.win_pos = None, None
        a.a_start, a.a_len, a.b_start, a.b_len = 0, cache.n, cache.n, 0
        a.gamma, a.res_w = side["gamma"].data_ptr(), side["res_w"].data_ptr()
        y = self._scratch(dev, f"anchor_y{B}x{H * HD}", B * H * HD // (2 if dt == torch.bfloat16 else 1))
        a.y = y.data_ptr()
        work = self._scratch(dev, "decode_work", A.decode_workspace_bytes(B, H, HKV, HD) // 4)
        a.work, a.work_bytes = work.data_ptr(), work.numel() * 4
        a.step_desc, a.ring_cap = desc, cache.capacity
        pw = self._scratch(dev, "proj_work", A.decode_layer_workspace_bytes(B, D, W.shape[0], H * HD, n_out) // 4)
        la.proj_work, la.proj_work_bytes = pw.data_ptr(), pw.numel() * 4
        la.x, la.x_row_stride, la.d_model = h.data_ptr(), D, D
        la.w_in, la.b_in, la.n_in = W.data_ptr(), A.ptr(bias), W.shape[0]
        la.w_out, la.b_out, la.n_out, la.out_row_stride = side["wo"].data_ptr(), None, n_out, n_out
        out = torch.empty(B, 1, n_out, dtype=dt, device=dev)
        la.out = out.data_ptr()
        A.call("bolt3_decode_layer", la, dev)
        if desc is None:
            cache.n += 1
        return out

    def _anchor_layer(self, ly, h: torch.Tensor, pos_start: int, cache: AnchorCache) -> torch.Tensor:
        """Causal softmax attention of t new tokens over the cached ones and themselves
        (vsa_lm/config/bolt3.py:426-445): query i sees cached keys and new keys up to i.  One bf16
        token: the fused HIP step; otherwise torch's attention on the cache."""
        b, t, _ = h.shape
        if t == 1 and self.fuse_projections and _fused_step_ok(h.dtype, h.shape[-1], ly.H * ly.HD,
                                                               ly.o_proj.out_features) and ly.G <= 8:
            return self._anchor_fused(ly, h, pos_start, cache)
        q, k, v = ly.head_qkv(h)
        q, k = ly.rope(q, pos_start=pos_start), ly.rope(k, pos_start=pos_start)
        n_old = cache.n
        keys, vals = cache.append(k, v)
        if t > 1 and n_old == 0:
            # nothing cached: plain causal attention, which keeps torch on its fused kernel
            y = F.scaled_dot_product_attention(q, keys.to(q.dtype), vals.to(q.dtype), is_causal=True,
                                               enable_gqa=ly.G > 1)
        else:
            visible = None
            if t > 1:
                visible = torch.ones(t, n_old + t, dtype=torch.bool, device=h.device).tril(diagonal=n_old)
            y = F.scaled_dot_product_attention(q, keys.to(q.dtype), vals.to(q.dtype), attn_mask=visible,
                                               enable_gqa=ly.G > 1)
        return ly.o_proj(y.transpose(1, 2).reshape(b, t, ly.H * ly.HD))

    # ------------------------------------------------------------ model-level API

    @torch.no_grad()
    def step(self, tokens: torch.Tensor, pos_start: int, states, kv_caches, record=None):
        """Run the tokens [B, t] through every layer at positions pos_start.. and update the states in
        place, as the reference's step does for any t (vsa_lm/config/bolt3.py:335-425): one
        attention over the window and the new tokens, then, once the current chunk holds C or more
        tokens, one consolidation of the previous chunk.  t is at most 2C minus the tokens already
        in the current chunk (checked for every layer before any state changes).  Returns (normed
        hidden states [B, t, D], states, kv_caches).  ``record``: a list (or a dict per layer index)
        that receives the decision log of every consolidation."""
        m = self.model
        for li, blk in enumerate(m.blocks):
            if hasattr(blk, "vsa"):
                _check_step_len(blk.vsa, kv_caches[li], tokens.shape[1])
        with torch.autocast(tokens.device.type, enabled=False):
            x = m.embed_tokens(tokens)
            for li, blk in enumerate(m.blocks):
                h = blk.norm1(x)
                if hasattr(blk, "vsa"):
                    rec = record.setdefault(li, []) if isinstance(record, dict) else record
                    x = x + self._bolt3_layer(blk.vsa, h, pos_start, states[li], kv_caches[li], rec)
                else:
                    x = x + self._anchor_layer(blk.attn, h, pos_start, kv_caches[li])
                x = x + blk.mlp(blk.norm2(x))
            return m.norm(x), states, kv_caches

    def _feed(self, ids: torch.Tensor, pos: int, states, kv_caches):
        """Step ids through the model in chunks of C tokens; returns (last hidden states, next position)."""
        h = None
        for s in range(0, ids.shape[1], self.C):
            part = ids[:, s:s + self.C]
            h, _, _ = self.step(part, pos, states, kv_caches)
            pos += part.shape[1]
        return h, pos

    @torch.no_grad()
    def prefill(self, ids: torch.Tensor, max_kv_len: int = 4096, record=None):
        """The prompt through every layer (vsa_lm/config/bolt3.py:450-457).  The reference steps it
        chunk by chunk through all layers; here each layer takes the whole prompt at once (a layer's
        output for a chunk depends only on that layer's inputs up to the chunk, so the order of the
        two loops does not change what is computed): the Bolt-3 layers through the forward's
        kernels (_bolt3_prefill), the anchors through causal attention over the prompt.  Returns
        (normed hidden states of the last chunk's tokens, states, kv_caches), as the reference.
        ``record``: as for ``step``."""
        b, t = ids.shape
        states, kv = self.blank_state(self.model, b, ids.device, max_kv_len=max(max_kv_len, t + 1024))
        m = self.model
        with torch.autocast(ids.device.type, enabled=False):
            x = m.embed_tokens(ids)
            for li, blk in enumerate(m.blocks):
                h = blk.norm1(x)
                if hasattr(blk, "vsa"):
                    rec = record.setdefault(li, []) if isinstance(record, dict) else record
                    x = x + self._bolt3_prefill(blk.vsa, h, states[li], kv[li], rec)
                else:
                    x = x + self._anchor_layer(blk.attn, h, 0, kv[li])
                x = x + blk.mlp(blk.norm2(x))
            s_last = ((t - 1) // self.C) * self.C
            return m.norm(x[:, s_last:]), states, kv

    @torch.no_grad()
    def generate_batch(self, ids: torch.Tensor, max_new_tokens: int, temperature: float = 0.6, top_k: int = 40,
                       top_p: float = 0.95, eos_ids: set[int] | None = None,
                       close_think_ids: list[int] | None = None):
        """Prefill ids [B, T], then generate up to max_new_tokens per row.  Returns (tokens
        [B, n], lengths [B]): n is max_new_tokens unless every row has ended by a check point (then
        the tokens up to that point), lengths the tokens up to and including each row's eos."""
        B, T = ids.shape
        h, states, kv = self.prefill(ids, max_kv_len=T + max_new_tokens + 64)
        book = _Bookkeeping(B, max_new_tokens, eos_ids, close_think_ids, ids.device)
        logits = self.model.lm_head(h[:, -1])
        graph = self._graph_runner(B, T + max_new_tokens + 1, ids.device, states, kv, T) if max_new_tokens > 1 \
            else None
        n_out = max_new_tokens
        for i in range(max_new_tokens):
            nxt = book.take(i, sample_tokens(logits, temperature, top_k, top_p))
            stop = book.stop_at(i)
            if stop is not None:
                n_out = stop
                break
            if i + 1 < max_new_tokens:
                if graph is not None:
                    logits = graph.step(nxt)
                else:
                    h, _, _ = self.step(nxt, T + i, states, kv)
                    logits = self.model.lm_head(h[:, -1])
        return book.toks[:, :n_out], book.lengths

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, max_new_tokens: int, temperature: float = 0.0, top_k: int = 40,
                 top_p: float = 0.95, eos_ids: set[int] | None = None, close_think_ids: list[int] | None = None):
        """The prompt followed by the first row's generated tokens (up to its eos), [B, T + n]."""
        toks, lengths = self.generate_batch(prompt, max_new_tokens, temperature, top_k, top_p, eos_ids,
                                            close_think_ids)
        return torch.cat([prompt, toks[:, :int(lengths[0])]], dim=1)

    @torch.no_grad()
    def continue_generate(self, ids: torch.Tensor, states, kv_caches, start_pos: int, max_new_tokens: int,
                          temperature: float = 0.0, top_k: int = 40, top_p: float = 0.95,
                          eos_ids: set[int] | None = None):
        """Feed ids from start_pos on an existing state, then generate until the first row emits an
        eos id (that token is returned but not fed).  Returns (tokens, states, kv_caches, next position).
        The returned state must not include tokens after the stop, so each token's stop test is read
        back before the token is fed."""
        h, pos = self._feed(ids, start_pos, states, kv_caches)
        stop = torch.tensor(sorted(eos_ids or ()), dtype=torch.long, device=ids.device)
        toks = torch.empty(ids.shape[0], max_new_tokens, dtype=torch.long, device=ids.device)
        n = 0
        logits = self.model.lm_head(h[:, -1])
        while n < max_new_tokens:
            nxt = sample_tokens(logits, temperature, top_k, top_p)
            toks[:, n] = nxt[:, 0]
            n += 1
            if stop.numel() and bool(torch.isin(nxt[0, 0], stop)):
                break
            h, _, _ = self.step(nxt, pos, states, kv_caches)
            logits = self.model.lm_head(h[:, -1])
            pos += 1
        return toks[:, :n], states, kv_caches, pos

    @torch.no_grad()
    def memorize(self, ids: torch.Tensor, states, kv_caches, start_pos: int):
        """Feed ids and return, per Bolt-3 layer, what they wrote into M_res: (next position,
        M_after - gamma^(tokens // C) * M_before), None for anchor layers
        (vsa_lm/config/bolt3.py:528-546).  Returns (states, kv_caches, next position, traces)."""
        before = [None if s is None else s.clone() for s in states]
        _, pos = self._feed(ids, start_pos, states, kv_caches)
        traces = []
        for li, blk in enumerate(self.model.blocks):
            if not hasattr(blk, "vsa"):
                traces.append(None)
                continue
            ly = blk.vsa
            decay = ly.gamma_delta().view(1, -1, 1, 1).to(states[li].device) ** (ids.shape[1] // ly.C)
            traces.append((pos, states[li] - decay * before[li]))
        return states, kv_caches, pos, traces

    @torch.no_grad()
    def forget(self, traces, states, next_pos: int, kv_caches=None, pre_kv_lens=None):
        """Take memorized writes back out of M_res, each decayed by gamma once per C positions between
        the end of its tokens and next_pos (vsa_lm/config/bolt3.py:548-557)."""
        for li, tr in enumerate(traces):
            if tr is None or states[li] is None:
                continue
            end_pos, delta = tr
            ly = self.model.blocks[li].vsa
            k = max(0, (next_pos - end_pos) // ly.C)
            states[li] = states[li] - ly.gamma_delta().view(1, -1, 1, 1).to(delta.device) ** k * delta
        return states


class DecodeGraph:
    """The one-token step of a whole stack (embedding to last-position logits) captured once as a
    HIP graph and replayed per token.

    Every fused kernel of the step reads its position and window segments from a device step
    descriptor (one shared by the Bolt-3 layers, whose rings move in lockstep, one by the anchor
    layers), and the graph ends by advancing both descriptors on the device.  The host mirrors
    the ring positions; when the current chunk fills, it runs the layers' consolidations eagerly
    after the replay (a layer's consolidation only changes that layer's later steps, so this is
    the eager order's result) and rewrites the descriptors.  Anchor caches are sized for every
    token before capture, so no buffer moves while the graph lives.
    """

    @staticmethod
    def supported(model) -> bool:
        for blk in model.blocks:
            ly = blk.vsa if hasattr(blk, "vsa") else blk.attn
            dt = ly.q_proj.weight.dtype
            if not _fused_step_ok(dt, ly.q_proj.in_features, ly.H * ly.HD, ly.o_proj.out_features) or ly.G > 8:
                return False
        return True

    def __init__(self, dec: Bolt3Decoder, states, kv, B: int, need_len: int, dev: torch.device, pos: int):
        self.dec, self.states, self.kv, self.dev = dec, states, kv, dev
        m = dec.model
        self.b3 = [(li, blk.vsa, kv[li]) for li, blk in enumerate(m.blocks) if hasattr(blk, "vsa")]
        self.an = [(li, blk.attn, kv[li]) for li, blk in enumerate(m.blocks) if not hasattr(blk, "vsa")]
        rings = {(c.prev, c.cur, c.n_sink, c.has_slots) for _, _, c in self.b3}
        lens = {c.n for _, _, c in self.an}
        if len(rings) > 1 or len(lens) > 1:
            raise ValueError("the layers' states are not in lockstep")
        for _, _, c in self.an:
            c.reserve(need_len)
        self.pos = pos
        self.d_b3 = torch.zeros(8, dtype=torch.int32, device=dev)
        self.d_an = torch.zeros(8, dtype=torch.int32, device=dev)
        self._write_descriptors()
        self.tok = torch.zeros(B, 1, dtype=torch.long, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        # warm-up on the capture stream with scratch descriptors of the same values: it writes the
        # new token's key and value where the first replay writes them again, and initialises
        # the libraries' per-stream state outside the capture
        warm_b3, warm_an = self.d_b3.clone(), self.d_an.clone()
        with torch.cuda.stream(side):
            self._forward(warm_b3.data_ptr(), warm_an.data_ptr())
        side.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            self.logits = self._forward(self.d_b3.data_ptr(), self.d_an.data_ptr())
            s = A.stream_of(dev)
            lib = A.load()
            rc = lib.bolt3_step_advance(self.d_b3.data_ptr(), 1, 0, 0, 0, 1, s)
            rc = rc or lib.bolt3_step_advance(self.d_an.data_ptr(), 1, 0, 1, 1, 0, s)
            if rc:
                raise RuntimeError(f"bolt3_step_advance failed with code {rc}")

    def _forward(self, d_b3: int, d_an: int) -> torch.Tensor:
        m, dec = self.dec.model, self.dec
        x = m.embed_tokens(self.tok)
        for li, blk in enumerate(m.blocks):
            h = blk.norm1(x)
            if hasattr(blk, "vsa"):
                y = dec._bolt3_layer(blk.vsa, h, self.pos, self.states[li], self.kv[li], desc=d_b3)
            else:
                y = dec._anchor_fused(blk.attn, h, self.pos, self.kv[li], desc=d_an)
            x = x + y
            x = x + blk.mlp(blk.norm2(x))
        return m.lm_head(m.norm(x)[:, -1])

    def _write_descriptors(self):
        vals = [0] * 16
        if self.b3:
            c = self.b3[0][2]
            vals[:7] = [self.pos, c.prev[0], c.prev[1], c.cur[0], c.cur[1], c.n_sink, int(c.has_slots)]
        if self.an:
            n = self.an[0][2].n
            vals[8:13] = [self.pos, 0, n, n, 0]
        host = torch.tensor(vals, dtype=torch.int32).pin_memory()
        self.d_b3.copy_(host[:8], non_blocking=True)
        self.d_an.copy_(host[8:], non_blocking=True)

    def step(self, tokens: torch.Tensor) -> torch.Tensor:
        """Feed one token per row ([B, 1]) at the next position; returns the logits [B, V] (a
        buffer the next step overwrites)."""
        self.tok.copy_(tokens)
        self.graph.replay()
        self.pos += 1
        for _, _, c in self.an:
            c.n += 1
        full = False
        for _, ly, c in self.b3:
            cs, cl = c.cur
            c.cur = (cs, cl + 1)
            full = c.cur[1] >= ly.C
        if full:
            for li, ly, c in self.b3:
                _, _, side = ly._packed(c.dtype, self.dev)
                self.dec._consolidate(ly, c, self.states[li], side["gamma"], side)
            self._write_descriptors()
        return self.logits

