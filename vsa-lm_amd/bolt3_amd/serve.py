"""Serving dispatch for Bolt-3 checkpoints.

The reference server builds a ``VSARecurrentDecoder`` for every model
(vsa_lm/server.py:141 and :159), which cannot step ``Bolt3Attn`` layers
(vsa_lm/decode.py:265).  ``make_decoder`` is the dispatch it lacks: a
``Bolt3Decoder`` for any stack that carries a Bolt-3 layer, ``None`` for the
others (the caller keeps its own decoder for them).  ``generate_completion``
is the server's completion call (vsa_lm/server.py:124-152) on that decoder.
"""
from __future__ import annotations

import torch

from .bolt3 import Bolt3Attn
from .decoder import Bolt3Decoder


def is_bolt3_model(model) -> bool:
    """True when some block of the stack has a Bolt-3 attention layer (``blk.vsa``)."""
    blocks = getattr(model, "blocks", None)
    if blocks is None:
        return False
    return any(isinstance(getattr(blk, "vsa", None), Bolt3Attn) for blk in blocks)


def make_decoder(model, device=None, **kwargs) -> Bolt3Decoder | None:
    """The decoder a server should build for ``model``: Bolt3Decoder for Bolt-3 stacks, with the
    reference server's cache bound (65536 positions on a GPU, 8192 on a CPU); None otherwise."""
    if not is_bolt3_model(model):
        return None
    dev = torch.device(device) if device is not None else next(model.parameters()).device
    kwargs.setdefault("max_cache_pos", 65536 if dev.type == "cuda" else 8192)
    kwargs.setdefault("wrap_positions", False)
    return Bolt3Decoder(model, **kwargs)


def _eos_ids(tokenizer) -> set[int]:
    eos = getattr(tokenizer, "eos_token_id", None)
    if eos is None:
        return set()
    return {int(e) for e in eos} if isinstance(eos, (list, tuple)) else {int(eos)}


def generate_completion(model, tokenizer, device, messages: list[dict], max_tokens: int = 1024,
                        temperature: float = 0.0, repetition_penalty: float = 1.0,
                        decoder: Bolt3Decoder | None = None, eos_ids: set[int] | None = None) -> str:
    """One chat completion of a Bolt-3 model: the chat template (or role-prefixed lines when the
    tokenizer has none), generation up to max_tokens or an end-of-sequence id, the reply decoded
    without special tokens and without the final end-of-sequence token.  Pass a long-lived decoder
    to reuse it across requests; eos_ids defaults to the tokenizer's eos id(s) (the reference
    server collects more, vsa_lm/server.py:23-38, and can pass them).  repetition_penalty is
    accepted and unused, as in the reference."""
    try:
        prompt = tokenizer.apply_chat_template(messages, tokenize=False, add_generation_prompt=True)
    except Exception:
        prompt = "\n".join(f"{m.get('role', 'user')}: {m.get('content', '')}" for m in messages) + "\nassistant: "
    ids = tokenizer.encode(prompt, add_special_tokens=False)
    stop = set(eos_ids) if eos_ids is not None else _eos_ids(tokenizer)
    if decoder is None:
        decoder = make_decoder(model, device)
        if decoder is None:
            raise TypeError("generate_completion: the model has no Bolt-3 layer; serve it with its own decoder")
    out = decoder.generate(torch.tensor([ids], dtype=torch.long, device=device), max_new_tokens=max_tokens,
                           temperature=temperature, eos_ids=stop)
    reply = out[0, len(ids):].tolist()
    if reply and reply[-1] in stop:
        reply = reply[:-1]
    return tokenizer.decode(reply, skip_special_tokens=True).strip()
