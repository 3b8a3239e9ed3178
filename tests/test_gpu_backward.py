"""Backward of Bolt3Attn on the HIP path (bolt3_attn_bwd, bolt3_chain_bwd, bolt3_heads_bwd).

* Against the reference's own gradients (tests/golden/grad_*.safetensors, fp32 CPU autograd
  through vsa_lm/config/bolt3.py): the gradient of x and of every parameter within 1e-4
  relative (1e-5 absolute for gradients that are zero in the reference).
* bf16 storage (the heal trainer's autocast) at head_dim 128 with merges: against the oracle's
  autograd on the same bf16 forward, within bf16 tolerance, decisions equal.
* The backward leaves the forward's output unchanged and runs twice in a row with the same
  result (every buffer it reads is the forward's, every output has one writer).
"""
import pytest
import torch

import recipes
from helpers import build_grad_case, cosine, fixture, rel_err
from oracle import bolt3_oracle as O

pytestmark = pytest.mark.gpu

GRAD = ["grad_fp32_short", "grad_fp32_eta", "grad_fp32_clustered", "grad_fp32_hd128"]


def _grads(mod, x, up, dev):
    """(y, {"x": dx, name: grad}) of sum(mod(x) * up) on dev."""
    mod = mod.to(dev)
    mod.zero_grad(set_to_none=True)
    xg = x.to(dev).clone().requires_grad_(True)
    y = mod(xg)
    (y * up.to(dev).to(y.dtype)).sum().backward()
    out = {"x": xg.grad.detach().cpu()}
    for k, prm in mod.named_parameters():
        out[k] = (prm.grad if prm.grad is not None else torch.zeros_like(prm)).detach().cpu()
    return y.detach().cpu(), out


@pytest.mark.parametrize("name", GRAD)
def test_backward_matches_reference_gradients(name, gpu):
    g, meta = fixture(name)
    mod, x, up = build_grad_case(meta)
    print(f"[case] backward vs reference gradients: {name}", flush=True)
    y, gr = _grads(mod, x, up, gpu)
    assert rel_err(y, g["y"]) <= 1e-5, rel_err(y, g["y"])
    errs = {}
    for k in sorted(gr):
        ref = g["grad." + k]
        errs[k] = rel_err(gr[k], ref) if float(ref.norm()) > 0 else float(gr[k].abs().max())
    print("  " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if v > (1e-4 if float(g["grad." + k].norm()) > 0 else 1e-5)}
    assert not bad, bad


@pytest.mark.parametrize("hd,heads,kv,T", [(128, 8, 2, 1024), (64, 4, 2, 1000), (128, 8, 8, 700), (64, 16, 2, 520)])
def test_backward_bf16_vs_oracle(hd, heads, kv, T, gpu):
    """bf16 storage, clustered input where tokens merge, replace slots and go to M_res: the HIP
    gradients against autograd through the oracle's bf16 forward (the reference's bf16
    arithmetic), relative error <= 3e-2 and cosine >= 0.999 for x and every parameter, the
    readout's parameters included.  Head dims 64 and 128, G = 4, 2, 1 and 8, sequence lengths
    with a partial last chunk and a partial last query tile.

    Where the reference's own bf16 arithmetic is more than 5e-2 from the exact gradient (the
    oracle's fp32 autograd on the same bf16-valued weights and input) -- a sum like kappa's, over
    a few slot columns of the softmax gradient, whose rows sum to zero -- two bf16 computations
    cannot agree to 3e-2; there the HIP gradient has to be as close to the exact one as the
    reference's (within 25 % and 5e-3).  Parameters whose gradient is exactly zero in both
    (no token reached M_res) compare equal."""
    import copy
    cfg = dict(dim=256, num_heads=heads, num_kv_heads=kv, head_dim=hd, rope_theta=1e6, eps=1e-6, qk_norm=True)
    from bolt3_amd import Bolt3Attn
    mod = recipes.init_module(Bolt3Attn(cfg), 31, nondefault=True).to(torch.bfloat16)
    x = recipes.clustered_hidden(31, 1, T, 256, n_centres=512, noise=0.15).to(torch.bfloat16)
    up = recipes.upstream(31, 1, T, 256)
    print(f"[case] backward bf16 vs oracle hd={hd} H={heads} HKV={kv} T={T}", flush=True)
    exact = O.forward_grads(O.Bolt3Params.from_module(copy.deepcopy(mod).float()), x.float(), up)[1]
    y, gr = _grads(mod, x, up, gpu)
    yr, ref = O.forward_grads(O.Bolt3Params.from_module(mod), x, up)
    assert rel_err(y.float(), yr.float()) <= 2e-2
    if T >= 1000:
        for k in ("eta_proj.weight", "res_norm.weight", "log_gamma", "beta_proj.weight"):
            assert float(ref[k].norm()) > 0, k      # the M_res path is exercised
    out, bad = [], []
    for k in sorted(ref):
        a, b, e = gr[k].float(), ref[k].float(), exact[k].float()
        if float(a.norm()) == 0 and float(b.norm()) == 0:
            continue
        err, cos = rel_err(a, b), cosine(a, b)
        e_ref, e_hip = rel_err(b, e), rel_err(a, e)
        out.append(f"{k}={err:.2e}/{cos:.5f} (exact: hip {e_hip:.2e}, ref {e_ref:.2e})")
        if e_ref > 5e-2:
            if e_hip > 1.25 * e_ref + 5e-3:
                bad.append((k, e_hip, e_ref))
        elif err > 3e-2 or cos < 0.999:
            bad.append((k, err, cos))
    print("  " + "\n  ".join(out), flush=True)
    assert not bad, bad


def test_backward_under_autocast_and_repeatable(gpu):
    """fp32 parameters under bf16 autocast (the heal trainer's setting): parameter gradients
    come back in fp32, x's in fp32, two forward + backward passes give identical gradients, and the
    output equals the no-grad forward's."""
    g, meta = fixture("grad_fp32_eta")
    mod, x, up = build_grad_case(meta)
    mod = mod.to(gpu)
    xs = x.to(gpu)
    res = []
    for _ in range(2):
        mod.zero_grad(set_to_none=True)
        xg = xs.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = mod(xg)
        assert y.dtype == torch.bfloat16
        (y.float() * up.to(gpu)).sum().backward()
        assert xg.grad.dtype == torch.float32
        assert all(p.grad.dtype == torch.float32 for p in mod.parameters())
        res.append((y.detach().clone(), xg.grad.clone(), [p.grad.clone() for p in mod.parameters()]))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    assert all(torch.equal(a, b) for a, b in zip(res[0][2], res[1][2]))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y0 = mod(xs)
    assert torch.equal(y0, res[0][0])
    # against the fixture's fp32 gradients: bf16 storage, so a loose bound
    assert cosine(res[0][1].cpu(), g["grad.x"]) >= 0.99


def test_backward_under_activation_checkpointing(gpu):
    """The heal trainer wraps every block in torch.utils.checkpoint(use_reentrant=False)
    (vsa_lm/converter.py:698-700): the layer's trace goes through save_for_backward, so between
    the forward and the backward the checkpointed layer holds none of it (the device memory it
    adds over its output is under a quarter of the plain run's), the backward recomputes it, and
    the gradients equal the plain run's bit for bit (the forward is deterministic).  A second
    backward with retain_graph=True gives the same gradients again."""
    from torch.utils.checkpoint import checkpoint
    from bolt3_amd import Bolt3Attn
    cfg = dict(dim=1024, num_heads=8, num_kv_heads=2, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)
    mod = recipes.init_module(Bolt3Attn(cfg), 43, nondefault=True).to(torch.bfloat16).to(gpu)
    x = recipes.clustered_hidden(43, 2, 2048, 1024, n_centres=512, noise=0.15).to(torch.bfloat16).to(gpu)
    up = recipes.upstream(43, 2, 2048, 1024).to(torch.bfloat16).to(gpu)
    print("[case] backward under activation checkpointing", flush=True)

    def run(ckpt: bool, twice: bool = False):
        mod.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_(True)
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated(gpu)
        y = checkpoint(mod, xg, use_reentrant=False) if ckpt else mod(xg)
        torch.cuda.synchronize()
        held = torch.cuda.memory_allocated(gpu) - base - y.numel() * y.element_size()
        torch.cuda.reset_peak_memory_stats(gpu)
        loss = (y * up).sum()
        loss.backward(retain_graph=twice)
        peak = torch.cuda.max_memory_allocated(gpu) - base
        grads = [xg.grad.clone()] + [p.grad.clone() for p in mod.parameters()]
        if twice:
            xg.grad = None
            mod.zero_grad(set_to_none=True)
            loss.backward()
            again = [xg.grad.clone()] + [p.grad.clone() for p in mod.parameters()]
            assert all(torch.equal(a, b) for a, b in zip(grads, again))
        return grads, held, peak

    g_plain, held_plain, peak_plain = run(False, twice=True)
    g_ckpt, held_ckpt, peak_ckpt = run(True)
    print(f"[case] held between forward and backward: plain {held_plain / 2**20:.1f} MiB, checkpointed "
          f"{held_ckpt / 2**20:.1f} MiB; backward peak: plain {peak_plain / 2**20:.1f} MiB, checkpointed "
          f"{peak_ckpt / 2**20:.1f} MiB", flush=True)
    assert held_plain > 0 and held_ckpt < held_plain / 4
    assert all(torch.equal(a, b) for a, b in zip(g_plain, g_ckpt))
