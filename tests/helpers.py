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


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_abs(a, b) -> float:
    return float((a.double() - b.double()).abs().max())


def cosine(a, b) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return float((a @ b) / (a.norm() * b.norm()).clamp_min(1e-30))
