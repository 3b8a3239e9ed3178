#!/usr/bin/env python3
"""Bolt-3 Dual-Field attention on one MI355X: prefill tokens/s, decode us/step, roofline.

Workload ("cfg2"): one Bolt3Attn layer of Qwen3-4B shape
(hidden 2560, 32 query / 8 kv heads, head_dim 128, RoPE theta 1e6, q/k norm,
C=128, S=128), chunked forward over B=4 x T=4096 tokens; bf16 projections and
activations, fp32 Bolt-3 parameters at their default init and fp32 state;
hidden ~N(0,1), projection weights ~N(0,0.02) (synthetic, seeded).

Decode (configs[2], "cfg3"): 64 sequences whose layer state was built by the
decoder's chunked step over 8192 synthetic tokens, then single-token steps
with fresh hidden ~N(0,1).  Several independent state sets are stepped in
turn so that one round touches more than the 256 MB Infinity Cache; each set
sees consecutive steps (consolidation every 128 of them).

Backward (the heal trainer's step on one layer): forward + backward of the
cfg2 layer with bf16 storage, gradients of x and every parameter.

One JSON line on stdout.  ``value`` is prefill tokens/s of the whole forward
(projections + HIP kernels + o_proj) with inputs resident in HBM.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "vsa-lm_amd"), os.path.join(REPO, "tests", "golden")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "Bolt3Attn prefill tokens/s + decode µs/step (Qwen3-4B layer); % roofline"
PEAK_BF16 = 2.5e15        # dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12         # HBM3E, B/s
CFG = dict(dim=2560, num_heads=32, num_kv_heads=8, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)
B, T = 4, 4096
SEED = 21


def prefill_flops(b, t, D=2560, H=32, HKV=8, HD=128, C=128):
    """Algorithmic FLOPs of one forward, split per part (dense attention rectangle)."""
    n_chunks = (t + C - 1) // C
    proj = 2 * b * t * D * (H * HD + 2 * HKV * HD + HKV + H) + 2 * b * t * H * HD * D
    keys = sum(128 if c == 0 else 256 if c == 1 else 4 + 128 + 256 for c in range(n_chunks))
    attn = 4 * b * H * C * HD * keys
    readout = 2 * b * H * C * HD * HD * max(0, n_chunks - 2)
    # consolidation: per steady step and bh, 5 HD-deep [C x S] / [C x C] products + 2 M_res products
    steady = max(0, n_chunks - 4)
    cons = b * HKV * steady * 2 * (5 * C * 128 * HD + 2 * C * HD * HD)
    return dict(proj=proj, attn=attn, readout=readout, consolidation=cons)


def backward_flops(b, t, H=32, HD=128, C=128):
    """Algorithmic FLOPs of bolt3_attn_bwd per forward: the attention's four gradient products
    (dP = dO.V^T, dV = P^T.dO, dQ = dS.K, dK = dS^T.Q) over the forward's key rectangle, and the
    readout's three HD x HD products per query row (q.M, dqn = du.M^T, dM += qn^T du)."""
    n_chunks = (t + C - 1) // C
    keys = sum(128 if c == 0 else 256 if c == 1 else 4 + 128 + 256 for c in range(n_chunks))
    attn = 8 * b * H * C * HD * keys
    readout = 3 * 2 * b * H * C * HD * HD * max(0, n_chunks - 2)
    return attn + readout


def bench_backward(mod, dev, steps, warmup, tune=False):
    """cfg2 forward + backward (the heal trainer's step on one layer): bf16 storage, gradients of
    x and every parameter for loss = sum(y * g) with a seeded upstream g.  tune: TunableOp times
    the solutions of the backward's GEMM shapes in the warm-up steps (and only there)."""
    import torch
    from bolt3_amd import _abi
    g = torch.Generator(device=dev).manual_seed(SEED + 2)
    x = torch.randn(B, T, CFG["dim"], generator=g, device=dev).to(torch.bfloat16)
    up = torch.randn(B, T, CFG["dim"], generator=g, device=dev).to(torch.bfloat16)

    def step():
        mod.zero_grad(set_to_none=True)
        xg = x.clone().requires_grad_(True)
        (mod(xg) * up).sum().backward()

    if tune:
        torch.cuda.tunable.tuning_enable(True)
    for _ in range(warmup):
        step()
    if tune:
        torch.cuda.tunable.tuning_enable(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _abi.set_timing(True)
    for _ in range(steps):
        step()
    kt = _abi.timings()
    _abi.set_timing(False)
    mod.zero_grad(set_to_none=True)
    ms = (t1 - t0) * 1e3 / steps
    # per backward: the sum over the entry point's calls (the attention backward runs as two
    # calls, the readout's and the attention's; the chain backward as four, one per kernel, the
    # M_res recursion on a side stream)
    bwd = kt.get("bolt3_attn_bwd", [])
    bwd_ms = sum(bwd) / steps
    cb = kt.get("bolt3_chain_bwd", [])
    fl = backward_flops(B, T)
    # bf16 storage: the attention and readout gradients run on bf16 MFMA
    return dict(ms_per_forward_backward=round(ms, 3), tokens_per_s=round(B * T / (ms * 1e-3), 1),
                attn_bwd_ms=round(bwd_ms, 3), attn_bwd_calls=len(bwd) // steps,
                chain_bwd_ms=round(sum(cb) / steps, 3), chain_bwd_calls=len(cb) // steps,
                roofline=dict(bound="mfma", kernel="bolt3_attn_bwd", flops=fl,
                              achieved=round(fl / (bwd_ms * 1e-3) / 1e12, 2), peak=PEAK_BF16 / 1e12, unit="TFLOP/s",
                              frac=round(fl / (bwd_ms * 1e-3) / PEAK_BF16, 4)))


def build_layer(dev):
    import torch
    import recipes
    from bolt3_amd import Bolt3Attn
    mod = recipes.init_module(Bolt3Attn(CFG), SEED, nondefault=False)
    for n, prm in mod.named_parameters():    # checkpoint layout: bf16 projections / norms, fp32 Bolt-3 params
        if n.split(".")[0] in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
            prm.data = prm.data.to(torch.bfloat16)
    return mod, mod.to(dev) if dev is not None else mod


def bench_prefill(mod, dev, steps, warmup):
    import torch
    from bolt3_amd import _abi
    g = torch.Generator(device=dev).manual_seed(SEED)
    x = torch.randn(B, T, CFG["dim"], generator=g, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        for _ in range(warmup):
            mod(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            mod(x)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        # per-entry durations from HIP events, in a second block of forwards (the timed block
        # above carries no event overhead)
        _abi.set_timing(True)
        for _ in range(steps):
            mod(x)
        kt = _abi.timings()
        _abi.set_timing(False)
    ms = (t1 - t0) * 1e3 / steps
    # per entry point: milliseconds per forward (sum over its launches) and launches per forward
    kern = {k: (sum(v) / steps, len(v) / steps) for k, v in kt.items()}
    return ms, kern


def bench_decode(dev, n_sets, n_steps, prefill_tokens=8192, batch=64):
    import torch
    from bolt3_amd import Bolt3Decoder, Bolt3LayerState, HybridLM, _abi
    mod = build_layer(dev)[1]
    model = HybridLM(vocab_size=8, dim=CFG["dim"], num_layers=0, num_heads=32, num_kv_heads=8,
                     intermediate=8, layer_types=[]).to(dev)
    dec = Bolt3Decoder(model)
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(SEED + 1)
    sets = []
    with torch.no_grad():
        for _ in range(n_sets):
            st = Bolt3LayerState(mod, batch, dev, bf)
            m = torch.zeros(batch, 8, 128, 128, device=dev)
            for c in range(prefill_tokens // mod.C):
                h = torch.randn(batch, mod.C, CFG["dim"], generator=g, device=dev).to(bf)
                dec._bolt3_layer(mod, h, c * mod.C, m, st)
            sets.append((st, m))
        torch.cuda.synchronize()
        hs = torch.randn(n_steps, batch, 1, CFG["dim"], generator=g, device=dev).to(bf)
        win_lens = []
        t0 = time.perf_counter()
        for s in range(n_steps):
            for st, m in sets:
                win_lens.append(st.prev[1] + st.cur[1] + 1)
                dec._bolt3_layer(mod, hs[s], prefill_tokens + s, m, st)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        # launch durations: a further full cycle of steps (every window length from 129 to 256
        # once, two consolidations per set) with HIP events around every entry point, outside
        # the timed loop above, whose per-step figure carries no event overhead
        n_time = n_steps
        tw = []
        _abi.set_timing(True)
        for s in range(n_time):
            for st, m in sets:
                tw.append(st.prev[1] + st.cur[1] + 1)
                dec._bolt3_layer(mod, hs[s], prefill_tokens + n_steps + s, m, st)
        kt = _abi.timings()
        _abi.set_timing(False)
    calls = n_steps * n_sets
    step_us = (t1 - t0) * 1e6 / calls
    entry = "bolt3_decode_layer"
    dec_ms = kt.get(entry, [])
    cons_ms = kt.get("bolt3_chain", [])
    avg_win = sum(tw) / len(tw)
    # algorithmic bytes of one launch.  Per sequence and kv head (bf16 keys/values, fp32 M_res):
    # the new token's projection row slice (written, then read), sinks, slot keys + values +
    # bias, window keys + values, M_res, the ring append and the attention output (written,
    # then read).  Per launch: both projection weights once, the input and output rows.
    W, _, side = mod._packed(bf, dev)
    n_in, D, K = W.shape[0], CFG["dim"], side["wo"].shape[1]
    per_bh = (2 * 6 * 128 * 2 + 2 * 4 * 128 * 2 + 2 * 128 * 128 * 2 + 128 * 4 + 2 * avg_win * 128 * 2
              + 128 * 128 * 4 + 3 * 128 * 2 + 2 * 4 * 128 * 2)
    bytes_launch = per_bh * batch * 8 + 2 * (n_in * D + D * K) + 2 * batch * (D + D)
    dec_avg = sum(dec_ms) / max(1, len(dec_ms))
    return dict(
        batch=batch, prefill_tokens=prefill_tokens, state_sets=n_sets, steps_per_set=n_steps,
        layer_step_us=round(step_us, 2),
        decode_layer_us=round(dec_avg * 1e3, 2),
        consolidation_us=round(sum(cons_ms) / max(1, len(cons_ms)) * 1e3, 2) if cons_ms else None,
        consolidations=len(cons_ms),
        amortized_kernel_us=round((sum(dec_ms) + sum(cons_ms)) / max(1, len(dec_ms)) * 1e3, 2),
        avg_window=round(sum(win_lens) / len(win_lens), 1),
        tokens_per_s=round(batch * 1e6 / step_us, 1),
        roofline=dict(bound="hbm", achieved=round(bytes_launch / (dec_avg * 1e-3) / 1e9, 1),
                      peak=PEAK_HBM / 1e9, unit="GB/s",
                      frac=round(bytes_launch / (dec_avg * 1e-3) / PEAK_HBM, 4),
                      traffic=measured_traffic(entry), kernel=entry,
                      algorithmic_bytes=int(bytes_launch), avg_launch_ms=round(dec_avg, 5),
                      avg_window=round(avg_win, 1)),
    )


def bench_long(dev, reps=3, T_long=65536):
    """The consolidation-heavy configuration: B=1, T=65536, Qwen3-4B layer (bf16 projections,
    fp32 Bolt-3 params), hidden states around 512 centres with noise 0.15 and Zipf(1.1)
    cluster choice, so that many tokens merge; 510 consolidation steps per forward."""
    import torch
    import recipes
    from bolt3_amd import _abi
    mod = build_layer(dev)[1]
    x = recipes.clustered_hidden(SEED + 2, 1, T_long, CFG["dim"], n_centres=512, noise=0.15).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        trace = {}
        mod(x, _trace=trace)                                # warm-up, and the decision log
        log = trace["log"]
        steady = log[4:, :, :, :128]
        merged = float(steady[:, :, _abi.LOG_FIELDS.index("merge")].mean())
        to_m = float(steady[:, :, _abi.LOG_FIELDS.index("delta")].mean())
        # rows (step, kv head) where exactly equal values decided a swap or a fill, ordered as the
        # reference's torch.topk orders them; and rows where that order would leave the restatement
        info = log[:, :, _abi.LOG_FIELDS.index("info"), 0].to(torch.int32)
        tie_rows = int(((info & (_abi.TIE_TOP | _abi.TIE_BOT)) != 0).sum())
        limit_rows = int(((info & _abi.TIE_LIMIT) != 0).sum())
        rows = int(info.numel())
        del trace, log
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            mod(x)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        _abi.set_timing(True)
        mod(x)
        kt = _abi.timings()
        _abi.set_timing(False)
    n_steps = T_long // mod.C - 2
    chain_ms = sum(kt.get("bolt3_chain", []))
    return dict(batch=1, seq_len=T_long, consolidation_steps=n_steps, ms_per_forward=round(ms, 3),
                tokens_per_s=round(T_long / (ms * 1e-3), 1), chain_ms_per_forward=round(chain_ms, 3),
                merged_share=round(merged, 3), m_res_share=round(to_m, 3),
                exact_tie_rows=tie_rows, tie_order_limit_rows=limit_rows, decision_rows=rows,
                data="synthetic clustered hidden states (512 centres, noise 0.15, Zipf 1.1)")


def build_e2e(dev, layers=36, vocab=151936, dim=2560, inter=9728):
    """The end-to-end configuration's model with random weights, made on the GPU: Qwen3-4B shape
    (hidden 2560, 32 / 8 heads, head_dim 128, SwiGLU 9728, vocabulary 151936, tied embeddings,
    q/k norm, theta 1e6), every 4th layer softmax (9) and 27 Bolt-3 layers at their default
    init; projections ~N(0, 0.02), embedding ~N(0, 1); bf16."""
    import torch
    from bolt3_amd import Bolt3Attn, HybridLM, RMSNorm
    from bolt3_amd.layers import rope_inv_freq
    types = ["softmax" if (i + 1) % 4 == 0 else "vsa" for i in range(layers)]
    with torch.device("meta"):
        m = HybridLM(vocab_size=vocab, dim=dim, num_layers=layers, num_heads=32, num_kv_heads=8, intermediate=inter,
                     layer_types=types, head_dim=128, qk_norm=True, rope_theta=1e6, eps=1e-6, max_T=65536)
    m = m.to_empty(device=dev)
    m.lm_head.weight = m.embed_tokens.weight
    g = torch.Generator(device=dev).manual_seed(SEED + 3)
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, torch.nn.Linear):
                mod.weight.normal_(0.0, 0.02, generator=g)
                if mod.bias is not None:
                    mod.bias.zero_()
            elif isinstance(mod, RMSNorm):
                mod.weight.fill_(1.0)
            if hasattr(mod, "rope"):
                mod.rope.inv_freq.copy_(rope_inv_freq(128, 1e6).to(dev))
        m.embed_tokens.weight.normal_(0.0, 1.0, generator=g)
        for mod in m.modules():
            if isinstance(mod, Bolt3Attn):      # the reference's constructor defaults
                mod.kappa.fill_(1.0)
                mod.log_gamma.fill_(3.5)
                mod.beta_proj.weight.zero_()
                mod.beta_proj.bias.fill_(-1.0)
                mod.eta_proj.weight.zero_()
                mod.eta_proj.bias.zero_()
                mod.res_norm.weight.fill_(0.05)
    return m.to(torch.bfloat16).eval()


def bench_e2e(dev, batch=32, prompt=2048, new=256, layers=36):
    """End-to-end generation: prefill of `prompt` uniform-random token ids for
    `batch` sequences, then `new` greedy tokens through Bolt3Decoder.generate_batch (graph-replayed
    one-token steps).  Prefill is timed alone; decode = generate_batch - prefill."""
    import torch
    import recipes
    from bolt3_amd import Bolt3Decoder
    m = build_e2e(dev, layers=layers)
    ids = recipes.tokens(SEED + 4, batch, prompt, m.config["vocab_size"]).to(dev)
    dec = Bolt3Decoder(m)
    with torch.no_grad():
        dec.generate_batch(ids[:, :256], 8, temperature=0.0)          # warm-up: kernels, handles, a capture
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill(ids)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        toks, _ = dec.generate_batch(ids, new, temperature=0.0)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
    pre_s, gen_s = t1 - t0, t2 - t1
    dec_s = max(gen_s - pre_s, 1e-9)
    return dict(layers=layers, bolt3_layers=sum(hasattr(b, "vsa") for b in m.blocks),
                softmax_layers=sum(not hasattr(b, "vsa") for b in m.blocks), batch=batch, prompt_tokens=prompt,
                new_tokens=int(toks.shape[1]), prefill_ms=round(pre_s * 1e3, 1), decode_ms=round(dec_s * 1e3, 1),
                prefill_tokens_per_s=round(batch * prompt / pre_s, 1),
                decode_tokens_per_s=round(batch * int(toks.shape[1]) / dec_s, 1),
                ms_per_decode_step=round(dec_s * 1e3 / max(1, int(toks.shape[1])), 3),
                data="random-init bf16 weights, uniform-random prompt ids, greedy decoding")


def measured_traffic(entry: str):
    """HBM bytes of an entry point from the rocprofv3 PMC summary committed under profiles/
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration): per forward for the
    prefill entry points (the unit of their roofline), per launch for the decode entry point;
    None when absent."""
    f = os.path.join(REPO, "profiles", "pmc_traffic.json")
    if not os.path.exists(f):
        return None
    with open(f) as fh:
        rec = json.load(fh).get(entry)
    return None if rec is None else rec.get("bytes_per_forward", rec.get("bytes_per_launch"))


def cpu_baseline(min_s=10.0, max_s=30.0):
    """The CPU oracle (the torch restatement of the reference path, oracle/bolt3_oracle.py) on the
    full cfg2 forward (B=4, T=4096, same module layout and dtype), repeated until at least
    ``min_s`` seconds of CPU work (a repeat is skipped when it would pass ``max_s``)."""
    import torch
    import recipes
    from oracle import bolt3_oracle as O
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    mod = build_layer(None)[0]
    p = O.Bolt3Params.from_module(mod)
    x = recipes.hidden(SEED, B, T, CFG["dim"]).to(torch.bfloat16)
    with torch.no_grad():
        O.forward(p, x[:1, :256])
        runs, total = 0, 0.0
        while total < min_s:
            t0 = time.perf_counter()
            O.forward(p, x)
            dt = time.perf_counter() - t0
            runs += 1
            total += dt
            if total + dt > max_s:
                break
    return dict(value=round(runs * B * T / total, 1), unit="tokens/s", cores=cores, kind="port",
                sample=f"oracle/bolt3_oracle.forward on the full cfg2 workload (B={B}, T={T}, bf16 projections, "
                       f"fp32 Bolt-3 params), {runs} forward(s) in {total:.1f} s, torch CPU with {cores} threads "
                       f"({platform.processor() or platform.machine()})")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--decode-sets", type=int, default=4)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-long", action="store_true", help="skip the consolidation-heavy B=1, T=65536 forward")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the 36-layer end-to-end generation")
    ap.add_argument("--no-backward", action="store_true", help="skip the forward + backward leg")
    ap.add_argument("--no-tunableop", action="store_true",
                    help="keep hipBLASLt's default solutions for the projection GEMMs (no TunableOp search)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain elementwise copy of 256 MiB (fp32 negate) three times, the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}): the Bolt-3 path "
              f"shards over (batch, kv-head) rows with no exchange, so N GPUs = N independent copies of this run.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.ones(64 << 20, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    _, mod = build_layer(dev)
    if not args.no_tunableop:
        # PyTorch's TunableOp times the hipBLASLt / rocBLAS solutions of each projection GEMM shape
        # on its first call (in the warm-up forwards) and keeps the fastest; tuning stops after the
        # prefill leg and runs again only in the backward leg's warm-up steps (its GEMM shapes), so
        # no timed region pays for a search
        import tempfile
        torch.cuda.tunable.enable(True)
        torch.cuda.tunable.tuning_enable(True)
        torch.cuda.tunable.set_filename(os.path.join(tempfile.gettempdir(), "bolt3_bench_tunableop.csv"))
    ms, kern = bench_prefill(mod, dev, args.steps, args.warmup)
    if not args.no_tunableop:
        torch.cuda.tunable.tuning_enable(False)
    fl = prefill_flops(B, T)
    total = sum(fl.values())
    # entry points: algorithmic work per forward (FLOPs, or bytes for the head preparation).  The
    # query heads are prepared inside the attention kernel, so bolt3_heads is the key/value launch:
    # per token the k | v columns and the beta gate read (2048 + 8 bf16), k_raw, k_rope and v written
    # (3 x 8 x 128 bf16) and beta (8 fp32); per position pos (fp32) and the (cos, sin) table row (64 x 4 B)
    work = {"bolt3_chunk_attn": ("mfma", fl["attn"] + fl["readout"]),
            "bolt3_chain": ("mfma", fl["consolidation"]),
            "bolt3_heads": ("hbm", B * T * ((2048 + 8) * 2 + 3 * 8 * 128 * 2 + 8 * 4) + T * (4 + 64 * 4))}
    kernels = {}
    for k, (bound, w) in work.items():
        ms_k, calls = kern.get(k, (0.0, 0.0))
        kernels[k] = dict(ms_per_forward=round(ms_k, 4), launches_per_forward=calls, bound=bound,
                          **({"flops": w} if bound == "mfma" else {"bytes": w}))
        if ms_k > 0:   # each entry point against its own roofline (work per forward / its launch time)
            rate = w / (ms_k * 1e-3)
            if bound == "mfma":
                kernels[k].update(achieved_tflops=round(rate / 1e12, 2), frac=round(rate / PEAK_BF16, 4))
            else:
                kernels[k].update(achieved_gbps=round(rate / 1e9, 1), frac=round(rate / PEAK_HBM, 4))
    dom = max(kernels, key=lambda k: kernels[k]["ms_per_forward"])
    d = kernels[dom]
    bound, w = work[dom]
    # the work and the time of all launches of the entry point in one forward (the chain goes out
    # in groups of steps, two launches per group; the attention and heads in two launches)
    fwd_s = d["ms_per_forward"] * 1e-3
    ach = w / fwd_s
    if bound == "hbm":
        roof = dict(bound="hbm", achieved=round(ach / 1e9, 1), peak=PEAK_HBM / 1e9, unit="GB/s",
                    frac=round(ach / PEAK_HBM, 4))
    else:
        roof = dict(bound="mfma", achieved=round(ach / 1e12, 2), peak=PEAK_BF16 / 1e12, unit="TFLOP/s",
                    frac=round(ach / PEAK_BF16, 4))
    roof["traffic"] = measured_traffic(dom)
    roof["kernel"] = dom
    roof["ms_per_forward"] = d["ms_per_forward"]
    roof["launches_per_forward"] = d["launches_per_forward"]
    out = {
        "metric": METRIC,
        "value": round(B * T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "cfg2: Bolt3Attn chunked forward, Qwen3-4B layer shape (hidden 2560, 32/8 heads, "
                               "head_dim 128, C=128, S=128), bf16 projections, fp32 Bolt-3 params and state",
                   "global_batch": B, "seq_len": T, "parallelism": "none (1 GPU)"},
        "roofline": roof,
        "whole_forward": dict(flops=total, tflops=round(total / (ms * 1e-3) / 1e12, 2),
                              frac_bf16_peak=round(total / (ms * 1e-3) / PEAK_BF16, 4)),
        "kernels": kernels,
        "gemm_selection": "hipBLASLt default" if args.no_tunableop else
                          "PyTorch TunableOp (hipBLASLt/rocBLAS solutions timed in the warm-up forwards and, "
                          "for the backward's products, the warm-up forward + backward steps)",
    }
    if not args.no_backward:
        out["backward"] = bench_backward(mod, dev, max(2, args.steps // 2), 2, tune=not args.no_tunableop)
    if not args.no_decode:
        out["decode"] = bench_decode(dev, args.decode_sets, args.decode_steps)
    if not args.no_long:
        out["long_prefill"] = bench_long(dev)
    if not args.no_e2e:
        out["e2e"] = bench_e2e(dev)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
