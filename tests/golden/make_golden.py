"""Write the Bolt-3 golden vectors from the reference implementation.

Run in the build container only (the reference tree is not present on GPU
boxes):  python tests/golden/make_golden.py [/root/reference]

It imports vsa_lm.config.bolt3 (Bolt3Attn, Bolt3Decoder) and
vsa_lm.config.standard (UniversalVSALM) from the reference tree on CPU, feeds
them the seeded synthetic inputs of tests/golden/recipes.py and stores what
they compute as safetensors files next to this script.  These pin the parts of
the oracle that no closed form covers: the composite Bolt3Attn.forward
(vsa_lm/config/bolt3.py:194-276), the multi-step _consolidate_functional
trajectories (:68-192), the Bolt3Decoder.step state machine (:335-457), the
generation rules of generate_batch (:459-500), memorize / forget (:528-557) and the
gradients of the forward (CPU autograd, fp32).

Every file carries a JSON header in its metadata (torch version, case
parameters, seed).  Parameters and inputs are regenerated from the recipes by
the tests; each file stores a checksum of them so a drifting recipe fails
loudly instead of comparing different problems.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import recipes  # noqa: E402


def digest(tensors: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(tensors):
        h.update(k.encode())
        h.update(tensors[k].detach().float().contiguous().numpy().tobytes())
    return h.hexdigest()


def layer_cfg(D, H, HKV, HD, theta, eps, qk_norm, qkv_bias=False):
    return dict(dim=D, num_heads=H, num_kv_heads=HKV, head_dim=HD, rope_theta=theta, eps=eps,
                qk_norm=qk_norm, qkv_bias=qkv_bias, rope_scaling=None)


def record_consolidations(mod):
    """Wrap mod._consolidate_functional to keep each call's outputs."""
    calls = []
    orig = mod._consolidate_functional

    def wrapped(*args, **kw):
        out = orig(*args, **kw)
        calls.append(tuple(o.detach().clone() if torch.is_tensor(o) else o for o in out))
        return out

    mod._consolidate_functional = wrapped
    return calls


def fwd_case(name, cfg, B, T, seed, dtype, nondefault, clustered=None, rows_every=1, S=128, C=128):
    from vsa_lm.config.bolt3 import Bolt3Attn
    mod = recipes.init_module(Bolt3Attn(cfg, S=S, C=C), seed, nondefault)
    D = cfg["dim"]
    x = recipes.clustered_hidden(seed, B, T, D, **clustered) if clustered else recipes.hidden(seed, B, T, D)
    inputs = {f"param.{k}": v for k, v in mod.state_dict().items()}
    inputs["x"] = x
    mod = mod.to(dtype)
    calls = record_consolidations(mod)
    with torch.no_grad():
        y = mod(x.to(dtype))
    tensors = {"y": y[:, ::rows_every].contiguous()}
    for i, c in enumerate(calls):
        ak, av, mass, util, pm, act, m_res, n_filled = c
        tensors[f"cons{i}.mass"] = mass.contiguous()
        tensors[f"cons{i}.util"] = util.contiguous()
        tensors[f"cons{i}.pm"] = pm.contiguous()
        tensors[f"cons{i}.act"] = act.to(torch.uint8).contiguous()
        tensors[f"cons{i}.m_res_rownorm"] = m_res.norm(dim=-1).contiguous()
        if i == len(calls) - 1:
            tensors["final.ak"] = ak.contiguous()
            tensors["final.av"] = av.contiguous()
            tensors["final.m_res"] = m_res.contiguous()
    meta = dict(case=name, torch=torch.__version__, cfg=cfg, B=B, T=T, S=S, C=C, seed=seed,
                dtype=str(dtype).replace("torch.", ""), nondefault=nondefault, clustered=clustered,
                rows_every=rows_every, n_consolidations=len(calls), n_filled=[int(c[7]) for c in calls],
                inputs_sha256=digest(inputs))
    save_file(tensors, os.path.join(HERE, f"{name}.safetensors"), metadata={"header": json.dumps(meta)})
    merged = sum(int((c[2] > 1).sum()) for c in calls[-1:])
    print(f"{name}: y {tuple(y.shape)} consolidations={len(calls)} n_filled={meta['n_filled']} "
          f"slots with mass>1 at end={merged}")


def grad_case(name, cfg, B, T, seed, nondefault, clustered=None, S=128, C=128):
    """Gradients of loss = sum(y * upstream) with respect to x and every parameter, fp32 CPU
    autograd through the reference forward (vsa_lm/config/bolt3.py:194-276): the slot
    selection runs under no_grad there, so the gradients follow that forward's decisions."""
    from vsa_lm.config.bolt3 import Bolt3Attn
    mod = recipes.init_module(Bolt3Attn(cfg, S=S, C=C), seed, nondefault)
    D = cfg["dim"]
    x = recipes.clustered_hidden(seed, B, T, D, **clustered) if clustered else recipes.hidden(seed, B, T, D)
    g = recipes.upstream(seed, B, T, D)
    inputs = {f"param.{k}": v for k, v in mod.state_dict().items()}
    inputs["x"] = x
    inputs["upstream"] = g
    calls = record_consolidations(mod)
    xg = x.clone().requires_grad_(True)
    y = mod(xg)
    (y * g).sum().backward()
    tensors = {"y": y.detach().contiguous(), "grad.x": xg.grad.contiguous()}
    for k, prm in mod.named_parameters():
        tensors[f"grad.{k}"] = (prm.grad if prm.grad is not None else torch.zeros_like(prm)).contiguous()
    merged = sum(int((c[2] > 1).sum()) for c in calls[-1:])
    meta = dict(case=name, torch=torch.__version__, cfg=cfg, B=B, T=T, S=S, C=C, seed=seed, dtype="float32",
                nondefault=nondefault, clustered=clustered, n_consolidations=len(calls),
                n_filled=[int(c[7]) for c in calls], inputs_sha256=digest(inputs))
    save_file(tensors, os.path.join(HERE, f"{name}.safetensors"), metadata={"header": json.dumps(meta)})
    print(f"{name}: consolidations={len(calls)} slots with mass>1 at end={merged} "
          f"|grad x|={float(xg.grad.norm()):.4g}")


def decoder_case(name, seed, dtype, n_prompt, n_decode, B=2):
    from vsa_lm.config.bolt3 import Bolt3Decoder
    from vsa_lm.config.standard import UniversalVSALM
    mcfg = dict(vocab_size=96, dim=64, num_layers=2, num_heads=4, num_kv_heads=2, intermediate=128,
                max_T=4096, chunk_size=32, hybrid_every=0, rope_theta=10000.0, eps=1e-5, head_dim=64,
                tie_word_embeddings=True, layer_types=["vsa", "softmax"], is_bolt3=True,
                bolt3_S=128, bolt3_C=128, qk_norm=True)
    model = UniversalVSALM(**mcfg)
    shapes = [(k, tuple(v.shape)) for k, v in model.state_dict().items()]
    model.load_state_dict(recipes.model_params(shapes, seed), strict=False)
    recipes.init_module(model.blocks[0].vsa, seed, nondefault=True)
    inputs = {f"param.{k}": v for k, v in model.state_dict().items()}
    ids = recipes.tokens(seed, B, n_prompt + n_decode, mcfg["vocab_size"])
    inputs["ids"] = ids.float()
    model = model.to(dtype).eval()
    dec = Bolt3Decoder(model)
    with torch.no_grad():
        h, states, kv = dec.prefill(ids[:, :n_prompt])
        hs = [h[:, -1].clone()]
        pos = n_prompt
        for _ in range(n_decode):
            h, states, kv = dec.step(ids[:, pos:pos + 1], pos, states, kv)
            hs.append(h[:, -1].clone())
            pos += 1
    sc = kv[0]
    tensors = {"h_last": torch.stack(hs, dim=1).contiguous(), "final.m_res": states[0].contiguous()}
    for key in ("ak", "av", "mass", "util", "pm", "sink_k", "sink_v", "prev_kp", "cur_kp"):
        if sc.get(key) is not None:
            tensors[f"final.{key}"] = sc[key].contiguous()
    tensors["final.act"] = sc["act"].to(torch.uint8).contiguous()
    meta = dict(case=name, torch=torch.__version__, model_cfg=mcfg, seed=seed, B=B, n_prompt=n_prompt,
                n_decode=n_decode, dtype=str(dtype).replace("torch.", ""), n_filled=int(sc.get("n_filled", 0)),
                inputs_sha256=digest(inputs))
    save_file(tensors, os.path.join(HERE, f"{name}.safetensors"), metadata={"header": json.dumps(meta)})
    print(f"{name}: steps={n_decode} n_filled={meta['n_filled']}")


def _ref_model(seed, tied=True, vocab=96):
    """The reference's UniversalVSALM of the decoder fixtures: two layers (Bolt-3, softmax anchor),
    hidden 64; with ``tied=False`` an output head of its own (drawn by the recipe), so that greedy
    tokens depend on the context instead of repeating the last token.  With a vocabulary of 96
    every token's key repeats within a chunk, so tokens merge into slots and nothing reaches
    M_res; the memory case takes 1024."""
    from vsa_lm.config.standard import UniversalVSALM
    mcfg = dict(vocab_size=vocab, dim=64, num_layers=2, num_heads=4, num_kv_heads=2, intermediate=128,
                max_T=4096, chunk_size=32, hybrid_every=0, rope_theta=10000.0, eps=1e-5, head_dim=64,
                tie_word_embeddings=tied, layer_types=["vsa", "softmax"], is_bolt3=True,
                bolt3_S=128, bolt3_C=128, qk_norm=True)
    model = UniversalVSALM(**mcfg)
    shapes = [(k, tuple(v.shape)) for k, v in model.state_dict().items()]
    model.load_state_dict(recipes.model_params(shapes, seed, head=not tied), strict=False)
    recipes.init_module(model.blocks[0].vsa, seed, nondefault=True)
    inputs = {f"param.{k}": v for k, v in model.state_dict().items()}
    return model.eval(), mcfg, inputs


def generate_case(name, seed, n_prompt, n_new, eos, close, B=3):
    """Bolt3Decoder.generate_batch at temperature 0 (vsa_lm/config/bolt3.py:459-500): per-row end of
    sequence, the forced close-of-thinking sequence at the budget point, the all-rows-done test
    every 16 tokens.  Stores the tokens, the lengths and, per step, the smallest top-2 logit gap
    over the rows (where a greedy pick could go either way)."""
    from vsa_lm.config.bolt3 import Bolt3Decoder
    model, mcfg, inputs = _ref_model(seed, tied=False)
    ids = recipes.tokens(seed, B, n_prompt, mcfg["vocab_size"])
    inputs["ids"] = ids.float()
    gaps = []

    def gap_hook(mod, inp, out):
        top2 = out.float().topk(2, dim=-1).values
        gaps.append(float((top2[..., 0] - top2[..., 1]).min()))

    hook = model.lm_head.register_forward_hook(gap_hook)
    with torch.no_grad():
        toks, lengths = Bolt3Decoder(model).generate_batch(ids, n_new, temperature=0.0, eos_ids=set(eos),
                                                           close_think_ids=list(close))
    hook.remove()
    tensors = {"toks": toks.contiguous(), "lengths": lengths.contiguous(),
               "gaps": torch.tensor(gaps[:toks.shape[1]], dtype=torch.float32)}
    meta = dict(case=name, torch=torch.__version__, model_cfg=mcfg, seed=seed, B=B, n_prompt=n_prompt, n_new=n_new,
                eos_ids=sorted(eos), close_think_ids=list(close), dtype="float32", inputs_sha256=digest(inputs))
    save_file(tensors, os.path.join(HERE, f"{name}.safetensors"), metadata={"header": json.dumps(meta)})
    print(f"{name}: tokens {tuple(toks.shape)} lengths {lengths.tolist()} smallest gap {min(gaps):.4g}")


def memory_case(name, seed, n_prompt, n_doc, n_after, n_probe, B=2):
    """Bolt3Decoder.memorize then forget (vsa_lm/config/bolt3.py:528-557): prefill a prompt,
    memorize a document (its trace: M_after - gamma^(len // C) M_before per Bolt-3 layer), feed
    more tokens, forget the trace (decayed by gamma per C positions since its end), then step a
    few tokens on the result.  Stores the trace, M_res after memorize, before and after forget,
    and the probe steps' hidden states."""
    from vsa_lm.config.bolt3 import Bolt3Decoder
    model, mcfg, inputs = _ref_model(seed, tied=True, vocab=1024)
    n = n_prompt + n_doc + n_after + n_probe
    ids = recipes.tokens(seed, B, n, mcfg["vocab_size"])
    inputs["ids"] = ids.float()
    dec = Bolt3Decoder(model)
    C = dec.C
    with torch.no_grad():
        _, states, kv = dec.prefill(ids[:, :n_prompt])
        states, kv, pos, traces = dec.memorize(ids[:, n_prompt:n_prompt + n_doc], states, kv, n_prompt)
        m_mem = states[0].clone()
        for s0 in range(n_prompt + n_doc, n_prompt + n_doc + n_after, C):
            e0 = min(n_prompt + n_doc + n_after, s0 + C)
            _, states, kv = dec.step(ids[:, s0:e0], s0, states, kv)
        m_before = states[0].clone()
        nxt = n_prompt + n_doc + n_after
        states = dec.forget(traces, states, nxt)
        m_after = states[0].clone()
        hs = []
        for i in range(n_probe):
            h, states, kv = dec.step(ids[:, nxt + i:nxt + i + 1], nxt + i, states, kv)
            hs.append(h[:, -1].clone())
    tensors = {"trace": traces[0][1].contiguous(), "m_memorized": m_mem.contiguous(),
               "m_before_forget": m_before.contiguous(), "m_after_forget": m_after.contiguous(),
               "h_probe": torch.stack(hs, dim=1).contiguous()}
    meta = dict(case=name, torch=torch.__version__, model_cfg=mcfg, seed=seed, B=B, n_prompt=n_prompt, n_doc=n_doc,
                n_after=n_after, n_probe=n_probe, trace_end=int(traces[0][0]), dtype="float32",
                inputs_sha256=digest(inputs))
    save_file(tensors, os.path.join(HERE, f"{name}.safetensors"), metadata={"header": json.dumps(meta)})
    print(f"{name}: trace end {traces[0][0]} |trace| {float(traces[0][1].norm()):.4g} "
          f"|M before forget| {float(m_before.norm()):.4g} |M after| {float(m_after.norm()):.4g}")


CASES = [
    # name, cfg args, B, T, seed, dtype, nondefault, clustered, rows_every
    ("fwd_fp32_default", (64, 4, 2, 64, 10000.0, 1e-5, False, False), 2, 896, 1, "float32", False, None, 1),
    ("fwd_fp32_eta", (64, 4, 2, 64, 10000.0, 1e-5, True, True), 2, 1000, 2, "float32", True, None, 1),
    ("fwd_fp32_g3", (96, 6, 2, 64, 500000.0, 1e-6, True, False), 1, 1152, 7, "float32", True, None, 1),
    ("fwd_bf16_eta", (64, 4, 2, 64, 10000.0, 1e-5, True, True), 1, 1024, 3, "bfloat16", True, None, 1),
    ("fwd_fp32_clustered", (64, 4, 2, 64, 10000.0, 1e-5, True, False), 1, 2048, 4, "float32", True,
     dict(n_centres=24, noise=0.12), 1),
    ("fwd_bf16_clustered", (64, 4, 2, 64, 10000.0, 1e-5, True, False), 1, 2048, 5, "bfloat16", True,
     dict(n_centres=24, noise=0.12), 1),
    ("fwd_cfg1_smollm", (576, 9, 3, 64, 10000.0, 1e-5, False, False), 1, 1024, 0, "float32", False, None, 8),
    # the consolidation-heavy configuration's kernel (bf16, head_dim 128, eight kv heads, theta 1e6): about
    # half the tokens merge, a third replace slots, the rest go to M_res
    ("fwd_bf16_clustered_hd128", (256, 16, 8, 128, 1000000.0, 1e-6, True, False), 1, 2048, 8, "bfloat16", True,
     dict(n_centres=512, noise=0.15), 2),
]
GRAD_CASES = [
    # name, cfg args, B, T, seed, nondefault, clustered
    ("grad_fp32_clustered", (64, 4, 2, 64, 10000.0, 1e-5, True, True), 1, 1280, 21, True,
     dict(n_centres=24, noise=0.12)),
    ("grad_fp32_eta", (64, 4, 2, 64, 10000.0, 1e-5, True, False), 2, 1000, 22, True, None),
    ("grad_fp32_short", (64, 4, 2, 64, 10000.0, 1e-5, False, False), 2, 200, 23, False, None),
    ("grad_fp32_hd128", (256, 8, 2, 128, 1000000.0, 1e-6, True, False), 1, 896, 24, True,
     dict(n_centres=64, noise=0.12)),
]
DECODER_CASES = [
    # name, seed, dtype, prompt tokens, decoded tokens
    ("dec_fp32", 6, "float32", 300, 220),
    ("dec_bf16", 9, "bfloat16", 300, 220),
]
GENERATE_CASES = [
    # name, seed, prompt tokens, new tokens, eos ids, close-of-thinking ids
    # rows 1 and 2 end early (eos 77); row 0 runs on and is forced through 5, 6, 7 at the budget point
    ("gen_eos_close", 42, 260, 150, (77,), (5, 6, 7)),
    # row 0 closes on its own (it emits 21, the sequence's second id); every row has ended by token 8,
    # so the loop stops at the check after token 16
    ("gen_all_done", 42, 260, 150, (77, 87), (5, 21, 7)),
    # row 0 closes on its own and never ends: the full 150 tokens
    ("gen_full_length", 42, 260, 150, (77,), (5, 21, 7)),
]
MEMORY_CASES = [
    # name, seed, prompt, document, tokens between memorize and forget, probe steps
    ("mem_forget", 12, 260, 384, 256, 8),
]


def main(ref_root: str, only=()):
    sys.path.insert(0, ref_root)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    for name, c, B, T, seed, dt, nd, cl, every in CASES:
        if not only or name in only:
            fwd_case(name, layer_cfg(*c), B, T, seed, getattr(torch, dt), nd, cl, every)
    for name, c, B, T, seed, nd, cl in GRAD_CASES:
        if not only or name in only:
            grad_case(name, layer_cfg(*c), B, T, seed, nd, cl)
    for name, seed, dt, n_prompt, n_decode in DECODER_CASES:
        if not only or name in only:
            decoder_case(name, seed=seed, dtype=getattr(torch, dt), n_prompt=n_prompt, n_decode=n_decode)
    for name, seed, n_prompt, n_new, eos, close in GENERATE_CASES:
        if not only or name in only:
            generate_case(name, seed, n_prompt, n_new, eos, close)
    for name, seed, n_prompt, n_doc, n_after, n_probe in MEMORY_CASES:
        if not only or name in only:
            memory_case(name, seed, n_prompt, n_doc, n_after, n_probe)


if __name__ == "__main__":
    # python make_golden.py [reference root] [case ...]: all cases, or only the named ones
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", tuple(sys.argv[2:]))
