"""Shared test helpers: golden fixtures, seeded modules, comparison metrics."""
from __future__ import annotations

import json
import os

import torch
from safetensors.torch import load_file, safe_open

import recipes
from make_golden import digest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture(name: str):
    path = os.path.join(GOLDEN, f"{name}.safetensors")
    with safe_open(path, framework="pt") as f:
        meta = json.loads(f.metadata()["header"])
    return load_file(path), meta


def layer_cfg(meta: dict) -> dict:
    return dict(meta["cfg"])


def build_layer(meta: dict, dtype=None):
    """Product Bolt3Attn on CPU with the fixture's seeded parameters, and its fp32 input x.
    Checks the recipe digest against the fixture before returning."""
    from bolt3_amd import Bolt3Attn
    mod = recipes.init_module(Bolt3Attn(layer_cfg(meta), S=meta["S"], C=meta["C"]), meta["seed"], meta["nondefault"])
    D = meta["cfg"]["dim"]
    cl = meta.get("clustered")
    if cl:
        x = recipes.clustered_hidden(meta["seed"], meta["B"], meta["T"], D, **cl)
    else:
        x = recipes.hidden(meta["seed"], meta["B"], meta["T"], D)
    inputs = {f"param.{k}": v for k, v in mod.state_dict().items()}
    inputs["x"] = x
    assert digest(inputs) == meta["inputs_sha256"], "recipe drifted from the golden fixture"
    dt = dtype or getattr(torch, meta["dtype"])
    return mod.to(dt), x.to(dt)


def build_grad_case(meta: dict):
    """Product Bolt3Attn (CPU, fp32) of a gradient fixture, its input x and the upstream gradient;
    checks the recipe digest (parameters, x, upstream) against the fixture."""
    from bolt3_amd import Bolt3Attn
    mod = recipes.init_module(Bolt3Attn(layer_cfg(meta), S=meta["S"], C=meta["C"]), meta["seed"], meta["nondefault"])
    D = meta["cfg"]["dim"]
    cl = meta.get("clustered")
    x = recipes.clustered_hidden(meta["seed"], meta["B"], meta["T"], D, **cl) if cl else \
        recipes.hidden(meta["seed"], meta["B"], meta["T"], D)
    g = recipes.upstream(meta["seed"], meta["B"], meta["T"], D)
    inputs = {f"param.{k}": v for k, v in mod.state_dict().items()}
    inputs["x"] = x
    inputs["upstream"] = g
    assert digest(inputs) == meta["inputs_sha256"], "recipe drifted from the golden fixture"
    return mod, x, g


def build_model(meta: dict, dtype=None):
    """Product HybridLM on CPU matching the decoder fixture."""
    from bolt3_amd import HybridLM
    mc = dict(meta["model_cfg"])
    model = HybridLM(**mc)
    shapes = [(k, tuple(v.shape)) for k, v in model.state_dict().items()]
    model.load_state_dict(recipes.model_params(shapes, meta["seed"]), strict=False)
    recipes.init_module(model.blocks[0].vsa, meta["seed"], nondefault=True)
    ids = recipes.tokens(meta["seed"], meta["B"], meta["n_prompt"] + meta["n_decode"], mc["vocab_size"])
    inputs = {f"param.{k}": v for k, v in model.state_dict().items()}
    inputs["ids"] = ids.float()
    assert digest(inputs) == meta["inputs_sha256"], "recipe drifted from the golden fixture"
    return model.to(dtype or getattr(torch, meta["dtype"])).eval(), ids


def build_fixture_model(meta: dict, n_tokens: int):
    """Product HybridLM on CPU matching a generation or memory fixture (its model config, an
    untied output head drawn by the recipe when the config says so) and its token ids; checks
    the recipe digest against the fixture."""
    from bolt3_amd import HybridLM
    mc = dict(meta["model_cfg"])
    model = HybridLM(**mc)
    shapes = [(k, tuple(v.shape)) for k, v in model.state_dict().items()]
    model.load_state_dict(recipes.model_params(shapes, meta["seed"], head=not mc["tie_word_embeddings"]),
                          strict=False)
    recipes.init_module(model.blocks[0].vsa, meta["seed"], nondefault=True)
    ids = recipes.tokens(meta["seed"], meta["B"], n_tokens, mc["vocab_size"])
    inputs = {f"param.{k}": v for k, v in model.state_dict().items()}
    inputs["ids"] = ids.float()
    assert digest(inputs) == meta["inputs_sha256"], "recipe drifted from the golden fixture"
    return model.to(getattr(torch, meta["dtype"])).eval(), ids


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_abs(a, b) -> float:
    return float((a.double() - b.double()).abs().max())


def cosine(a, b) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return float((a @ b) / (a.norm() * b.norm()).clamp_min(1e-30))


def decisions_from_kernel_log(log: torch.Tensor):
    """The slot decisions a kernel's decision log records, as the oracle's ``consolidate(force=...)``
    takes them: fill picks (the token order row), merge flags and argmax slots, and the
    replacement pairs (token order, slot order, win).  ``log`` is one step [bh, rows, cols] or
    a stack of steps [n, bh, rows, cols] (then a list, one dict per step)."""
    from bolt3_amd import _abi as A
    if log.dim() == 4:
        return [decisions_from_kernel_log(log[i]) for i in range(log.shape[0])]
    log = log.detach().cpu()
    row = lambda name: log[:, A.LOG_FIELDS.index(name)]
    return dict(picked=row("top_tok").long(), slot=row("slot").long(), merge=row("merge") != 0,
                top_toks=row("top_tok").long(), bot_slots=row("bot_slot").long(), win=row("win") != 0)


def decisions_from_oracle_log(lg: dict) -> dict:
    """The decisions an oracle step log holds, in the same form (fill: picked; steady: the rest)."""
    if lg["kind"] == "fill":
        return dict(picked=lg["picked"])
    return {k: lg[k] for k in ("slot", "merge", "top_toks", "bot_slots", "win")}


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """The bf16 spacing at |x|: 2^(floor(log2 |x|) - 7) (8 significant bits)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def bf16_check(y: torch.Tensor, ref: torch.Tensor):
    """The bf16 output bar: every element within max(2e-2, 2 ulp_bf16(ref)) of the reference,
    and cosine >= 0.9995.  2e-2 absolute is the contract's bound; it is kept wherever it exceeds
    two bf16 ulps of the reference value (|ref| < 2.56).  Above that one ulp is 2^-6 or more, and
    two correct implementations whose products sum in another order round the same output up to
    an ulp apart on top of ulp-sized differences in their bf16 inputs, so the bound there is two
    ulps.  Returns (ok, max-abs error, worst error / bound, cosine)."""
    y, ref = y.double(), ref.double()
    err = (y - ref).abs()
    bound = torch.clamp(2.0 * bf16_ulp(ref), min=2e-2)
    ratio = float((err / bound).max()) if err.numel() else 0.0
    cs = cosine(y, ref)
    return ratio <= 1.0 and cs >= 0.9995, float(err.max()) if err.numel() else 0.0, ratio, cs
