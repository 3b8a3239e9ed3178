"""Deterministic synthetic parameters and inputs for Bolt-3 layers.

Shared by tests/golden/make_golden.py (which feeds them to the reference) and
the tests and bench (which feed them to the oracle and to the HIP path), so a
fixture can store only what the reference computed.  All draws use numpy's
PCG64 ``default_rng`` streams keyed by the case seed.
"""
from __future__ import annotations

import numpy as np
import torch

PROJ = ("q_proj", "k_proj", "v_proj", "o_proj")


def _n(rng, shape, std):
    return torch.from_numpy((rng.standard_normal(shape) * std).astype(np.float32))


def _u(rng, shape, lo, hi):
    return torch.from_numpy(rng.uniform(lo, hi, shape).astype(np.float32))


def layer_params(named_shapes, seed: int, nondefault: bool) -> dict:
    """Parameter tensors (fp32) for a module with the reference Bolt3Attn names.

    Projections (and their biases) ~N(0, 0.02); q/k-norm weights ~U(0.6, 1.4).
    With ``nondefault`` the Bolt-3 parameters are drawn too (beta/eta gates
    ~N(0, 0.02) with random biases, kappa ~U(0.5, 1.5), log_gamma ~U(1, 4),
    res_norm ~U(0.5, 1.5)); otherwise they keep the constructor defaults
    (vsa_lm/config/bolt3.py:44-54) and are not returned.
    """
    rng = np.random.default_rng([seed, 0])
    out = {}
    for name, shape in sorted(named_shapes):
        shape = tuple(shape)
        head = name.split(".")[0]
        if head in PROJ:
            out[name] = _n(rng, shape, 0.02)
        elif head in ("q_norm", "k_norm"):
            out[name] = _u(rng, shape, 0.6, 1.4)
        elif nondefault:
            if name in ("beta_proj.weight", "eta_proj.weight"):
                out[name] = _n(rng, shape, 0.02)
            elif name == "beta_proj.bias":
                out[name] = _u(rng, shape, -1.5, 1.0)
            elif name == "eta_proj.bias":
                out[name] = _u(rng, shape, -0.8, 0.8)
            elif name == "kappa":
                out[name] = _u(rng, shape, 0.5, 1.5)
            elif name == "log_gamma":
                out[name] = _u(rng, shape, 1.0, 4.0)
            elif name == "res_norm.weight":
                out[name] = _u(rng, shape, 0.5, 1.5)
    return out


def init_module(mod, seed: int, nondefault: bool):
    """Load layer_params into ``mod`` (any module with the reference parameter names)."""
    shapes = [(k, tuple(v.shape)) for k, v in mod.state_dict().items()]
    mod.load_state_dict(layer_params(shapes, seed, nondefault), strict=False)
    return mod


def hidden(seed: int, B: int, T: int, D: int) -> torch.Tensor:
    """x ~ N(0, 1) of shape [B, T, D] (fp32)."""
    rng = np.random.default_rng([seed, 1])
    return _n(rng, (B, T, D), 1.0)


def clustered_hidden(seed: int, B: int, T: int, D: int, n_centres: int, noise: float,
                     zipf_a: float = 1.1) -> torch.Tensor:
    """Hidden states drawn around ``n_centres`` centres: x_t = c_{z_t} + noise * n_t with
    z_t ~ Zipf(zipf_a) over the centres.  Projected keys/values of one cluster then have
    cosines near 1, so consolidation merges fire."""
    rng = np.random.default_rng([seed, 2])
    centres = _n(rng, (n_centres, D), 1.0)
    prob = np.arange(1, n_centres + 1, dtype=np.float64) ** (-zipf_a)
    prob /= prob.sum()
    z = rng.choice(n_centres, size=(B, T), p=prob)
    return centres[torch.from_numpy(z)] + _n(rng, (B, T, D), noise)


def upstream(seed: int, B: int, T: int, D: int) -> torch.Tensor:
    """Gradient of the loss with respect to the layer output, ~N(0, 1) [B, T, D] (fp32): the
    gradient fixtures back-propagate loss = sum(y * upstream)."""
    rng = np.random.default_rng([seed, 5])
    return _n(rng, (B, T, D), 1.0)


def tokens(seed: int, B: int, T: int, vocab: int) -> torch.Tensor:
    rng = np.random.default_rng([seed, 3])
    return torch.from_numpy(rng.integers(0, vocab, size=(B, T))).long()


def model_params(named_shapes, seed: int, head: bool = False) -> dict:
    """Non-Bolt-3 weights of a small hybrid model: 2-D weights ~N(0, 0.02), the
    embedding ~N(0, 1); norms keep their ones.  ``head``: an untied output head,
    drawn ~N(0, 1) after everything else (with tied embeddings the head is the
    embedding and is not drawn)."""
    rng = np.random.default_rng([seed, 4])
    out = {}
    for name, shape in sorted(named_shapes):
        if name == "embed_tokens.weight":
            out[name] = _n(rng, tuple(shape), 1.0)
        elif len(shape) == 2 and "beta_proj" not in name and "eta_proj" not in name and name != "lm_head.weight":
            out[name] = _n(rng, tuple(shape), 0.02)
    if head:
        shape = dict(named_shapes)["lm_head.weight"]
        out["lm_head.weight"] = _n(np.random.default_rng([seed, 6]), tuple(shape), 1.0)
    return out
