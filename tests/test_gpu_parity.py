"""HIP path vs the oracle / the reference's golden vectors, on the GPU.

Tolerances (from the path's contract):
  fp32 modules:  relative error <= 1e-4 on outputs;
  bf16 modules:  max-abs error <= 2e-2 and cosine >= 0.9995 on outputs;
  decisions (merge, argmax slot, replacements, delta mask): bit-exact except
  for tokens whose compared quantity lies within 1e-4 (relative) of its
  threshold or of a competing value; those are counted as near-ties and
  reported, not hidden.
"""
from __future__ import annotations

import copy
import math

import pytest
import torch

from bolt3_amd import _abi as A
from oracle import bolt3_oracle as O
from helpers import bf16_check, build_layer, build_model, cosine, decisions_from_kernel_log, fixture, max_abs, rel_err

pytestmark = pytest.mark.gpu

FWD = ["fwd_fp32_default", "fwd_fp32_eta", "fwd_fp32_g3", "fwd_bf16_eta", "fwd_cfg1_smollm",
       "fwd_fp32_clustered", "fwd_bf16_clustered", "fwd_bf16_clustered_hd128"]
TIE = 1e-4
LOG = {name: i for i, name in enumerate(A.LOG_FIELDS)}


def _check_out(y, ref, dtype, what, normed=False):
    """normed=True: y is a final RMS-normalised hidden state (entries up to ~4, bf16 ulp there is
    1.6e-2), compared by relative error instead of max-abs.  bf16 outputs otherwise: max-abs
    2e-2, or two bf16 ulps where the reference value is large enough for that to exceed 2e-2
    (helpers.bf16_check)."""
    if dtype == torch.float32:
        e = rel_err(y, ref)
        assert e <= 1e-4, f"{what}: rel err {e:.3e}"
    elif normed:
        e, cs = rel_err(y, ref), cosine(y, ref)
        assert e <= 1e-2 and cs >= 0.9995, f"{what}: rel err {e:.3e} cos {cs:.6f}"
    else:
        ok, ma, ratio, cs = bf16_check(y, ref)
        assert ok, f"{what}: max-abs {ma:.3e} (worst error / bound {ratio:.3f}) cos {cs:.6f}"


def _near(a, b):
    """A near-tie: two different values within the tolerance of each other (rounding can order
    them either way).  Exactly equal values are not near-ties: the kernel orders them as the
    reference does."""
    return a != b and abs(a - b) <= TIE * max(abs(a), abs(b), 1e-6)


def _any_near(vals, n):
    return any(_near(vals[k], vals[k + 1]) for k in range(min(n, len(vals) - 1)))


ROUND = 2.0 ** -7   # bf16: two roundings of a score apart (8 significant bits)


def _pair(a_o, b_o, a_k, b_k, bf16=False, same_inputs=True):
    """Class of two items an ordering placed differently: "near" -- their values within 4e-4
    relative of each other in the oracle's arithmetic (a_o, b_o) or in the kernel's (a_k, b_k),
    and not exactly equal in both (4e-4 because items of one near-tied group can trade places
    with any member of it).  Values exactly equal in both arithmetics must be ordered as
    torch.topk orders them when the two orderings sort bit-identical arrays (same_inputs); when
    any value of the array differs between the arithmetics, torch.topk's partition steps differ
    and so may its order among equal values, and such a pair is a tie like any other ("near");
    "round" (bf16 storage only) -- within 2^-7 instead, where the two arithmetics already differ
    by more than 1e-4 on one of the items: the reference rounds the slot scores to bf16 before
    their softmax, and a score that rounds the other way moves the read-out by about one bf16
    ulp; "bad" -- anything else."""
    close = lambda a, b, tol: abs(a - b) <= tol * max(abs(a), abs(b), 1e-6)
    if a_o == b_o and a_k == b_k:
        return "bad" if same_inputs else "near"
    if close(a_o, b_o, 4 * TIE) or close(a_k, b_k, 4 * TIE):
        return "near"
    if bf16 and (close(a_o, b_o, ROUND) or close(a_k, b_k, ROUND)) and \
            not (close(a_o, a_k, TIE) and close(b_o, b_k, TIE)):
        return "round"
    return "bad"


def _row_class(classes):
    return "bad" if "bad" in classes else "round" if "round" in classes else "near"


def _inversions(order_o, order_k, n_items, cap):
    """Pairs of items that the two orderings put in opposite order.  order_o / order_k: item ids
    in rank order; only the first ``cap`` ranks count, an item ranked at or after ``cap`` (or
    absent) ranks last, and items that both lists rank last are unordered."""
    ro = torch.full((n_items,), cap, dtype=torch.long)
    rk = torch.full((n_items,), cap, dtype=torch.long)
    oo = torch.as_tensor(order_o[:cap], dtype=torch.long)
    ok_ = torch.as_tensor(order_k[:cap], dtype=torch.long)
    ok_ = ok_[(ok_ >= 0) & (ok_ < n_items)]
    ro[oo] = torch.arange(len(oo))
    rk[ok_] = torch.arange(len(ok_))
    moved = torch.nonzero(ro != rk).flatten().tolist()
    pairs = set()
    for x in moved:
        inv = ((ro[x] < ro) & (rk[x] > rk)) | ((ro[x] > ro) & (rk[x] < rk))
        for y in torch.nonzero(inv).flatten().tolist():
            pairs.add((min(x, y), max(x, y)))
    return sorted(pairs)


def _replacements(toks, slots, win, bh, l):
    """[bh, l]: the slot each token replaces, -1 where it replaces none."""
    out = torch.full((bh, l), -1, dtype=torch.long)
    rows = torch.arange(bh).unsqueeze(1).expand_as(toks)
    out[rows[win], toks[win]] = slots[win]
    return out


def _compare_step(lg, log, bh, l, where, bf16=False):
    """Decisions of one consolidation step: the oracle's log (torch.topk order, the reference's)
    against the kernel's.  Returns (mismatches, near_ties, tie_rows, rounding), counted per
    differing token (merges) or row (fill picks, replacements).  A differing merge or argmax slot is a near-tie
    when the cosine lies within 1e-4 of its threshold or of the runner-up slot's.  Differing fill
    picks or replacements are a near-tie when every pair of tokens (or slots) that the two
    orderings rank oppositely holds values within 4e-4 of each other in either arithmetic and
    not exactly equal in both (exactly equal values must follow torch.topk's order), and where
    one side replaces and the other does not, the token's score and the slot's keep value are
    within that tolerance (``_pair``).  With bf16 storage a row whose only differences are
    "round" pairs counts as a rounding divergence (reported apart from near-ties).  tie_rows
    counts rows where the kernel ordered exactly equal values itself.  Equal decisions are found with tensor comparisons; only differing rows and tokens
    are examined one by one."""
    mism = near = rnd = 0
    log = log.detach().cpu()
    info = log[:bh, LOG["info"], 0].to(torch.int64)
    tie_rows = int(((info & (A.TIE_TOP | A.TIE_BOT)) != 0).sum())
    for r in torch.nonzero(info & A.TIE_LIMIT).flatten().tolist():
        mism += 1
        print(f"  {where} row {r}: tie order left the restatement (depth limit)", flush=True)
    if lg["kind"] == "fill":
        m = lg["picked"].shape[1]
        got_all = log[:bh, LOG["top_tok"], :m].long()
        for r in torch.nonzero((got_all != lg["picked"]).any(dim=1)).flatten().tolist():
            picked, got = lg["picked"][r].tolist(), got_all[r].tolist()
            so, sk = lg["score"][r].tolist(), log[r, LOG["score"], :l].tolist()
            # every pair of tokens the two fills order differently must be a near-tie
            same = so == sk
            cls = {(x, y): _pair(so[x], so[y], sk[x], sk[y], bf16, same) for x, y in _inversions(picked, got, l, m)}
            bad = [xy for xy, c in cls.items() if c == "bad"]
            row = _row_class(cls.values())
            if row != "bad" and all(0 <= t < l for t in got):
                near, rnd = near + (row == "near"), rnd + (row == "round")
            else:
                mism += 1
                x, y = bad[0] if bad else (got[0], got[0])
                print(f"  {where} row {r}: fill order {picked[:8]} vs {got[:8]}; tokens {x} / {y} scores oracle "
                      f"{so[x]!r} / {so[y]!r} kernel {sk[x]!r} / {sk[y]!r}", flush=True)
        return mism, near, tie_rows, rnd
    mg = log[:bh, LOG["merge"], :l] != 0
    sg = log[:bh, LOG["slot"], :l].long()
    mr, sr = lg["merge"].bool(), lg["slot"].long()
    differ = (mr != mg) | (mr & (sr != sg))
    for r, j in torch.nonzero(differ).tolist():
        b, v, b2 = float(lg["best"][r, j]), float(lg["sim_v"][r, j]), float(lg["best2"][r, j])
        if _near(b, O.SIM_K) or _near(v, O.SIM_V) or _near(b, b2):
            near += 1
        else:
            mism += 1
            print(f"  {where} row {r} tok {j}: merge {bool(mr[r, j])}/{bool(mg[r, j])} slot {int(sr[r, j])}/"
                  f"{int(sg[r, j])} best {b:.6f} simv {v:.6f}", flush=True)
    kc = lg["top_vals"].shape[1]
    rep_ref = _replacements(lg["top_toks"].long(), lg["bot_slots"].long(), lg["win"].bool(), bh, l)
    tt_g, bs_g = log[:bh, LOG["top_tok"], :kc].long(), log[:bh, LOG["bot_slot"], :kc].long()
    w_g = log[:bh, LOG["win"], :kc] != 0
    rep_got = _replacements(tt_g, bs_g, w_g, bh, l)
    bad = (rep_ref != rep_got).any(dim=1) | (lg["delta"].bool() != (log[:bh, LOG["delta"], :l] != 0)).any(dim=1)
    merge_rows = set(torch.nonzero(differ.any(dim=1)).flatten().tolist())
    for r in torch.nonzero(bad).flatten().tolist():
        if r in merge_rows:
            continue        # follows from the merge decision above, already counted there
        tv, bv = lg["top_vals"][r].tolist(), lg["bot_vals"][r].tolist()
        gtv, gbv = log[r, LOG["top_val"], :kc].tolist(), log[r, LOG["bot_val"], :kc].tolist()
        so, sk = lg["score"][r].tolist(), log[r, LOG["score"], :l].tolist()
        ko, kk = lg["keep"][r].tolist(), log[r, LOG["keep"], :lg["keep"].shape[1]].tolist()
        # within the replacing prefix of either side: every pair of tokens, and every pair of slots,
        # that the two orderings rank oppositely must be a near-tie; where one side replaces and
        # the other does not, the token's score against the slot's keep value must be one
        nw_o, nw_k = int(lg["win"][r].sum()), int(w_g[r].sum())
        W = max(nw_o, nw_k)
        same_t, same_s = so == sk, ko == kk
        ct = {(x, y): _pair(so[x], so[y], sk[x], sk[y], bf16, same_t)
              for x, y in _inversions(lg["top_toks"][r].tolist(), tt_g[r].tolist(), l, W)}
        cs = {(x, y): _pair(ko[x], ko[y], kk[x], kk[y], bf16, same_s)
              for x, y in _inversions(lg["bot_slots"][r].tolist(), bs_g[r].tolist(), len(ko), W)}
        cw = {k: _pair(tv[k], bv[k], gtv[k], gbv[k], bf16) for k in range(min(nw_o, nw_k), W)}
        bad_t = [xy for xy, c in ct.items() if c == "bad"]
        bad_s = [xy for xy, c in cs.items() if c == "bad"]
        bad_w = [k for k, c in cw.items() if c == "bad"]
        row = _row_class(list(ct.values()) + list(cs.values()) + list(cw.values()))
        if row != "bad":
            near, rnd = near + (row == "near"), rnd + (row == "round")
            if row == "round":
                print(f"  {where} row {r}: replacements differ by a bf16 rounding divergence (token pairs "
                      f"{[(x, y, so[x], so[y], sk[x], sk[y]) for (x, y), c in ct.items() if c == 'round'][:2]} "
                      f"slot pairs {[(x, y) for (x, y), c in cs.items() if c == 'round'][:2]})", flush=True)
        else:
            mism += 1
            print(f"  {where} row {r}: replacements differ (wins {nw_o} / {nw_k}); unexplained token pairs "
                  f"{[(x, y, so[x], so[y], sk[x], sk[y]) for x, y in bad_t[:2]]} slot pairs "
                  f"{[(x, y, ko[x], ko[y], kk[x], kk[y]) for x, y in bad_s[:2]]} win ranks {bad_w[:2]}", flush=True)
    return mism, near, tie_rows, rnd


def _step_has_near_tie(lg) -> bool:
    """Whether an oracle decision log holds a near-tie anywhere a decision depends on it."""
    if lg["kind"] == "fill":
        m = lg["picked"].shape[1]
        return any(_any_near(sorted(r.tolist(), reverse=True), m + 1) for r in lg["score"])
    for r in range(lg["best"].shape[0]):
        best, simv, best2 = lg["best"][r].tolist(), lg["sim_v"][r].tolist(), lg["best2"][r].tolist()
        if any(_near(b, O.SIM_K) or _near(v, O.SIM_V) or _near(b, c) for b, v, c in zip(best, simv, best2)):
            return True
        tv, bv = lg["top_vals"][r].tolist(), lg["bot_vals"][r].tolist()
        if any(_near(a, b) for a, b in zip(tv, bv)) or _any_near(tv, len(tv)) or _any_near(bv, len(bv)):
            return True
    return False


def _oracle_departure(tr, g) -> int | None:
    """First consolidation where this host's CPU oracle leaves the reference's trajectory (the
    fixture's per-step activity, masses and mean positions), or None.  The fixture was written
    on another CPU, whose BLAS sums in another order; a departure must sit on a near-tie."""
    for i, st in enumerate(tr.states):
        same = torch.equal(st.act.to(torch.uint8), g[f"cons{i}.act"]) and torch.equal(st.mass, g[f"cons{i}.mass"]) \
            and rel_err(st.pm, g[f"cons{i}.pm"]) <= 1e-6
        if not same:
            assert _step_has_near_tie(tr.logs[i]), f"oracle left the reference at step {i} without a near-tie"
            return i
    return None


def _forced_compare(tr_f, log, where, bf16=False):
    """Every step of a kernel decision log against the decisions the forced oracle would have made
    itself from the same state (tr_f.logs: its own decisions, each stage given the kernel's
    earlier stages).  Returns (mismatches, near-ties, tie rows, rounding divergences, first step
    with a near-tie or a rounding divergence)."""
    mism = near = tie_rows = rnd = 0
    first = None
    for i, (lg, chunk) in enumerate(zip(tr_f.logs, tr_f.chunks)):
        a, b, c, d = _compare_step(lg, log[i], log.shape[1], chunk[0].shape[1], f"{where} step {i}", bf16)
        mism, near, tie_rows, rnd = mism + a, near + b, tie_rows + c, rnd + d
        if (b or d) and first is None:
            first = i
    return mism, near, tie_rows, rnd, first


def _max_rounding(log) -> int:
    """Rounding divergences accepted in a run: one per 1000 (step, row) decision records of a
    bf16 chain, none below that."""
    return (log.shape[0] * log.shape[1]) // 1000


def _check_state(st, m_res, ref: O.SlotState, dtype, what, m_tol=None):
    """The kernel's slot state and M_res against the oracle's at the same point of one trajectory
    (M_res: 1e-4 relative in fp32, 1e-3 in bf16 unless ``m_tol`` says otherwise)."""
    bf = dtype == torch.bfloat16
    assert torch.equal(st["act"].cpu().bool().view_as(ref.act), ref.act), what
    assert torch.equal(st["mass"].cpu().view_as(ref.mass), ref.mass), what
    assert rel_err(st["pm"].cpu().view_as(ref.pm), ref.pm) <= 1e-6, what
    assert rel_err(st["util"].cpu().view_as(ref.util), ref.util) <= 1e-4, what
    assert rel_err(st["ak"].cpu().float().view_as(ref.ak), ref.ak.float()) <= (1e-2 if bf else 1e-5), what
    assert rel_err(st["av"].cpu().float().view_as(ref.av), ref.av.float()) <= (1e-2 if bf else 1e-5), what
    if ref.m_res.abs().max() > 0:
        e = rel_err(m_res.cpu().view_as(ref.m_res), ref.m_res)
        print(f"  {what}: M_res rel err {e:.2e}", flush=True)
        assert e <= (m_tol or (1e-3 if bf else 1e-4)), (what, e)


@pytest.mark.parametrize("name", FWD)
def test_forward_matches_golden(name, gpu):
    """The HIP forward, whole sequence, against the oracle forced onto the kernel's own decisions
    (every consolidation's fill picks, merges, replacements and delta mask imposed; every value
    computed by the oracle): whole output and end state within the contract's tolerance, and at
    every step the kernel's decisions equal the ones the oracle makes from the same state, exact
    ties in torch.topk's order, only near-ties within 1e-4 allowed to differ (counted).  Against
    the reference's own vectors: the whole output and end state when neither the kernel nor this
    host's CPU oracle took a near-tie the other way; otherwise every chunk before the first
    consolidation such a step touches."""
    g, meta = fixture(name)
    mod, x = build_layer(meta)
    p = O.Bolt3Params.from_module(mod)
    tr = O.ForwardTrace()
    with torch.no_grad():
        O.forward(p, x, trace=tr)
    d_oracle = _oracle_departure(tr, g)
    mod = mod.to(gpu)
    trace = {}
    with torch.no_grad():
        y = mod(x.to(gpu), _trace=trace).cpu()
    log = trace["log"].cpu()
    tr_f = O.ForwardTrace()
    with torch.no_grad():
        y_f = O.forward(p, x, trace=tr_f, decisions=decisions_from_kernel_log(log))
    mism, near, tie_rows, rnd, d_gpu = _forced_compare(tr_f, log, name, x.dtype == torch.bfloat16)
    e_f = rel_err(y, y_f)
    print(f"[decisions] {name}: steps={len(tr_f.logs)} mismatches={mism} near-ties={near} rounding divergences={rnd} "
          f"rows ordered on exact ties={tie_rows} oracle departs at={d_oracle} gpu near-tie at={d_gpu}; "
          f"whole output vs forced oracle rel err {e_f:.3e} max-abs {max_abs(y, y_f):.3e}", flush=True)
    assert mism == 0 and rnd <= _max_rounding(log)
    _check_out(y, y_f, x.dtype, f"{name} whole output vs forced oracle")
    _check_state(trace["state"], trace["m_res"], tr_f.states[-1], x.dtype, f"{name} end state vs forced oracle")
    every = meta["rows_every"]
    if d_oracle is None and d_gpu is None:
        # the kernel's trajectory is the reference's: compare with the reference's own vectors
        st = trace["state"]
        last = len(tr.logs) - 1
        assert torch.equal(st["act"].cpu().view_as(g[f"cons{last}.act"]), g[f"cons{last}.act"])
        assert torch.equal(st["mass"].cpu().view_as(g[f"cons{last}.mass"]), g[f"cons{last}.mass"])
        assert rel_err(st["pm"].cpu(), g[f"cons{last}.pm"].view_as(st["pm"])) <= 1e-6
        tol_s = 1e-4 if x.dtype == torch.float32 else 1e-2
        assert rel_err(st["ak"].cpu().float(), g["final.ak"].float().view_as(st["ak"])) <= tol_s
        assert rel_err(st["av"].cpu().float(), g["final.av"].float().view_as(st["av"])) <= tol_s
        assert rel_err(trace["m_res"].cpu(), g["final.m_res"].view_as(trace["m_res"])) <= \
            (1e-4 if x.dtype == torch.float32 else 1e-3)
        _check_out(y[:, ::every], g["y"], x.dtype, name)
    else:
        d = min(v for v in (d_oracle, d_gpu) if v is not None)
        n_rows = (d + 2) * p.C          # chunks before the first one that reads step d's slots
        ys, ref = y[:, :n_rows:every], g["y"][:, :(n_rows + every - 1) // every]
        _check_out(ys, ref, x.dtype, f"{name} first {n_rows} tokens")
        print(f"[case] {name}: near-tie at step {d}; tokens before {n_rows} match the reference; the whole "
              f"output matches the oracle along the kernel's decisions", flush=True)


def _gpu_step(mod, st_in, chunk, gam, b, dev):
    """One consolidation on the GPU from an oracle state; returns (state dict, m_res, decision log)."""
    kr, kp, v, pos, beta = chunk
    bh, l, hd = kr.shape
    dt = kr.dtype
    if st_in is None:
        st = mod._empty_slots(bh, dt, dev)
        m = torch.zeros(bh, hd, hd, device=dev)
        nf = 0
    else:
        st = dict(ak=st_in.ak.to(dev).contiguous(), av=st_in.av.to(dev).contiguous(),
                  mass=st_in.mass.to(dev).contiguous(), util=st_in.util.to(dev).contiguous(),
                  pm=st_in.pm.to(dev).contiguous(), act=st_in.act.to(torch.uint8).to(dev).contiguous())
        m = st_in.m_res.to(dev).contiguous().clone()
        nf = st_in.n_filled
    kr_d, kp_d, v_d = kr.to(dev).contiguous(), kp.to(dev).contiguous(), v.to(dev).contiguous()
    pos_d, b_d = pos.float().to(dev).contiguous(), beta.float().to(dev).contiguous()
    W, bias, side = mod._packed(dt, dev)
    log = torch.zeros(1, bh, A.LOG_ROWS, A.LOG_COLS, device=dev)
    mod._chain(dt, dev, b, kr_d.data_ptr(), kp_d.data_ptr(), v_d.data_ptr(), l * hd, pos_d.data_ptr(),
               b_d.data_ptr(), l, 1, 0, l, l, l, nf, st, m, gam.to(dev), side, log=log)
    torch.cuda.synchronize()
    return {k: t.cpu() for k, t in st.items()}, m.cpu(), log[0].cpu()


@pytest.mark.parametrize("name", FWD)
def test_chain_decisions_teacher_forced(name, gpu):
    """Every consolidation step run on the GPU from the reference's state before it (the oracle's
    trajectory, equal to the reference's): decisions bit-exact, exact ties included, near-ties
    counted; the state after the step equal to the reference's where no near-tie was involved."""
    g, meta = fixture(name)
    mod, x = build_layer(meta)
    p = O.Bolt3Params.from_module(mod)
    tr = O.ForwardTrace()
    with torch.no_grad():
        O.forward(p, x, trace=tr)
    mod = mod.to(gpu)
    gam = O.gamma_delta(p.log_gamma)
    b = meta["B"]
    mism = near = tie_rows = rnd = 0
    for i, (chunk, lg) in enumerate(zip(tr.chunks, tr.logs)):
        print(f"[case] {name} step {i} kind={lg['kind']}", flush=True)
        st_prev = tr.states[i - 1] if i > 0 else None
        st, m, log = _gpu_step(mod, st_prev, chunk, gam, b, gpu)
        ref = tr.states[i]
        bh, l = chunk[0].shape[:2]
        a, c, t, d = _compare_step(lg, log, bh, l, f"{name} step {i}", x.dtype == torch.bfloat16)
        mism, near, tie_rows, rnd = mism + a, near + c, tie_rows + t, rnd + d
        if c == 0 and d == 0:
            assert torch.equal(st["act"].bool(), ref.act), (name, i)
            assert torch.equal(st["mass"], ref.mass), (name, i)
            assert rel_err(st["pm"], ref.pm) <= 1e-6, (name, i)
            assert rel_err(st["util"], ref.util) <= 1e-4, (name, i)
            assert rel_err(st["ak"].float(), ref.ak.float()) <= (1e-5 if ref.ak.dtype == torch.float32 else 1e-2)
            tol_m = 1e-4 if ref.ak.dtype == torch.float32 else 1e-3
            if ref.m_res.abs().max() > 0:
                assert rel_err(m, ref.m_res) <= tol_m, (name, i, rel_err(m, ref.m_res))
    print(f"[decisions] {name}: steps={len(tr.logs)} mismatches={mism} near-ties={near} rounding divergences={rnd} "
          f"rows ordered on exact ties={tie_rows}", flush=True)
    assert mism == 0 and rnd == 0


def _to_oracle_state(st: dict, m: torch.Tensor, nf: int) -> O.SlotState:
    return O.SlotState(ak=st["ak"].cpu(), av=st["av"].cpu(), mass=st["mass"].cpu(), util=st["util"].cpu(),
                       pm=st["pm"].cpu(), act=st["act"].cpu().bool(), m_res=m.cpu(), n_filled=nf)


@pytest.mark.parametrize("name", ["fwd_fp32_clustered", "fwd_bf16_clustered", "fwd_fp32_eta", "fwd_bf16_eta",
                                  "fwd_bf16_clustered_hd128"])
def test_chain_kernel_trajectory_checked(name, gpu):
    """The kernel's own trajectory: every step the oracle, started from the kernel's state, must
    make the same decisions (near-ties excepted) and reach the same state; and the one-launch
    chain of the forward ends in the state of this step-by-step run."""
    g, meta = fixture(name)
    mod, x = build_layer(meta)
    p = O.Bolt3Params.from_module(mod)
    tr_o = O.ForwardTrace()
    with torch.no_grad():
        O.forward(p, x, trace=tr_o)
    mod = mod.to(gpu)
    gam = O.gamma_delta(p.log_gamma)
    b = meta["B"]
    st_k = None
    mism = near = tie_rows = rnd = 0
    for i, chunk in enumerate(tr_o.chunks):
        print(f"[case] {name} kernel-trajectory step {i}", flush=True)
        st_g, m_g, log = _gpu_step(mod, st_k, chunk, gam, b, gpu)
        lg = {}
        ref = O.consolidate(p, st_k, *chunk, gam, b, log=lg)
        bh, l = chunk[0].shape[:2]
        a, c, t, d = _compare_step(lg, log, bh, l, f"{name} step {i}", x.dtype == torch.bfloat16)
        mism, near, tie_rows, rnd = mism + a, near + c, tie_rows + t, rnd + d
        if c == 0 and d == 0:
            assert torch.equal(st_g["act"].bool(), ref.act) and torch.equal(st_g["mass"], ref.mass), (name, i)
            assert rel_err(st_g["util"], ref.util) <= 1e-4, (name, i)
            bf = ref.ak.dtype == torch.bfloat16
            assert rel_err(st_g["ak"].float(), ref.ak.float()) <= (1e-2 if bf else 1e-5), (name, i)
            if ref.m_res.abs().max() > 0:
                assert rel_err(m_g, ref.m_res) <= (1e-3 if bf else 1e-4), (name, i)
        st_k = _to_oracle_state(st_g, m_g, ref.n_filled)
    print(f"[decisions] {name} kernel trajectory: mismatches={mism} near-ties={near} rounding divergences={rnd} "
          f"rows ordered on exact ties={tie_rows}", flush=True)
    assert mism == 0 and rnd == 0
    # one launch over all steps (as the forward runs it) == the step-by-step run above
    dt = x.dtype
    bh = b * p.HKV
    n = len(tr_o.chunks)
    C = p.C
    toks = {k: torch.zeros(bh, n * C, p.HD, dtype=dt) for k in ("kr", "kp", "v")}
    posa = torch.zeros(n * C)
    beta_a = torch.zeros(bh, n * C)
    for i, (ckr, ckp, cv, cpos, cb) in enumerate(tr_o.chunks):
        off = i * C + (C - ckr.shape[1])
        toks["kr"][:, off:(i + 1) * C], toks["kp"][:, off:(i + 1) * C], toks["v"][:, off:(i + 1) * C] = ckr, ckp, cv
        posa[off:(i + 1) * C], beta_a[:, off:(i + 1) * C] = cpos, cb.float()
    d = {k: t.to(gpu).contiguous() for k, t in toks.items()}
    posd, betad = posa.to(gpu), beta_a.to(gpu)
    st1 = mod._empty_slots(bh, dt, gpu)
    m1 = torch.zeros(bh, p.HD, p.HD, device=gpu)
    W, bias, side = mod._packed(dt, gpu)
    ns = C - tr_o.chunks[0][0].shape[1]
    mod._chain(dt, gpu, b, d["kr"].data_ptr(), d["kp"].data_ptr(), d["v"].data_ptr(), n * C * p.HD, posd.data_ptr(),
               betad.data_ptr(), n * C, n, ns, C - ns, C, C, 0, st1, m1, gam.to(gpu), side)
    torch.cuda.synchronize()
    assert torch.equal(st1["ak"].cpu(), st_g["ak"]) and torch.equal(st1["mass"].cpu(), st_g["mass"])
    assert torch.equal(m1.cpu(), m_g)


def _split_mt(m: torch.Tensor) -> torch.Tensor:
    """fp32 M [..., HD, HD] -> the bf16 forward's snapshot form: per matrix M^T rounded to bf16
    (hi), then the bf16 rounding of what hi leaves (lo), HD*HD elements each, in a buffer of
    the fp32 matrix's size."""
    mt = m.transpose(-1, -2).contiguous()
    hi = mt.to(torch.bfloat16)
    lo = (mt - hi.float()).to(torch.bfloat16)
    hd = m.shape[-1]
    both = torch.cat([hi.reshape(*m.shape[:-2], hd * hd), lo.reshape(*m.shape[:-2], hd * hd)], dim=-1)
    return both.view(torch.float32).view(m.shape)


@pytest.mark.parametrize("name", ["fwd_fp32_clustered", "fwd_bf16_clustered", "fwd_fp32_eta", "fwd_bf16_eta",
                                  "fwd_bf16_clustered_hd128"])
def test_attention_from_oracle_states(name, gpu):
    """The chunk-attention kernel fed with the oracle's heads and per-chunk slot states reproduces the
    oracle's pre-o_proj output (isolates attention + readout from trajectory divergence).  bf16
    takes the forward's kernel and snapshot form (M^T as bf16 hi + lo); at head_dim 128 with four
    query heads per kv head that is the kernel the full-size configurations run."""
    g, meta = fixture(name)
    mod, x = build_layer(meta)
    p = O.Bolt3Params.from_module(mod)
    tr = O.ForwardTrace()
    with torch.no_grad():
        O.forward(p, x, trace=tr, ties="torch")
    q_raw, q_rope, k_raw, k_rope, v, beta, eta = tr.heads
    b, T = meta["B"], meta["T"]
    dt = x.dtype
    split = dt == torch.bfloat16
    snap_k = torch.stack([O.slot_keys(p, s, b) for s in tr.states])
    snap_v = torch.stack([s.av for s in tr.states])
    snap_b = torch.stack([O.slot_bias(p, s, b) for s in tr.states])
    snap_m = torch.stack([s.m_res for s in tr.states])       # fp32 M[c][d] blocks
    if split:
        snap_m = _split_mt(snap_m)
    dv = lambda t: t.to(gpu).contiguous()
    from bolt3_amd import _abi as A
    mod = mod.to(gpu)
    W, bias, side = mod._packed(dt, gpu)
    qr, qp, kp, vv = dv(q_raw), dv(q_rope), dv(k_rope), dv(v)
    et = dv(eta.squeeze(-1).float())
    sk, sv, sb, sm = dv(snap_k), dv(snap_v), dv(snap_b), dv(snap_m)
    gam = dv(O.gamma_delta(p.log_gamma))
    y = torch.empty(b, T, p.H * p.HD, dtype=dt, device=gpu)
    a = A.AttnArgs()
    a.dtype, a.B, a.H, a.HKV, a.HD, a.S, a.C, a.n_sinks = A.dtype_code(dt), b, p.H, p.HKV, p.HD, p.S, p.C, 4
    a.mode, a.n_q, a.score_round = 0, T, 1
    a.q_rope, a.q_raw, a.q_sb, a.q_sh = qp.data_ptr(), qr.data_ptr(), qp.stride(0), qp.stride(1)
    a.eta, a.e_sb, a.e_sh = et.data_ptr(), et.stride(0), et.stride(1)
    a.win_k, a.win_v, a.w_sb, a.w_sh = kp.data_ptr(), vv.data_ptr(), kp.stride(0), kp.stride(1)
    a.slot_k, a.slot_v, a.slot_bias = sk.data_ptr(), sv.data_ptr(), sb.data_ptr()
    a.slot_step, a.m_res, a.m_step = b * p.HKV * p.S * p.HD, sm.data_ptr(), b * p.HKV * p.HD * p.HD
    a.m_split = int(split)
    a.gamma, a.res_w, a.eps = gam.data_ptr(), side["res_w"].data_ptr(), p.eps
    a.y, a.y_sb, a.y_st = y.data_ptr(), y.stride(0), y.stride(1)
    A.call("bolt3_chunk_attn", a, gpu)
    ref = tr.y_pre.transpose(1, 2).reshape(b, T, -1)
    _check_out(y.cpu(), ref, dt, name)


def test_consolidate_functional_api(gpu):
    """The reference's internal entry point (15 positional args + n_filled, 8-tuple result)."""
    g, meta = fixture("fwd_fp32_eta")
    mod, x = build_layer(meta)
    p = O.Bolt3Params.from_module(mod)
    tr = O.ForwardTrace()
    O.forward(p, x, trace=tr, ties="torch")
    mod = mod.to(gpu)
    i = 3
    st0, (kr, kp, v, pos, beta) = tr.states[i - 1], tr.chunks[i]
    b, hkv, S, hd = meta["B"], p.HKV, p.S, p.HD
    l = kr.shape[1]
    d = lambda t: t.to(gpu)
    out = mod._consolidate_functional(
        d(st0.ak), d(st0.av), d(st0.mass), d(st0.util), d(st0.pm), d(st0.act), d(st0.m_res),
        d(kr.view(b, hkv, l, hd)), d(kp.view(b, hkv, l, hd)), d(v.view(b, hkv, l, hd)), d(pos.view(1, 1, l)),
        d(beta.view(b, hkv, l)), d(p.inv_freq), None, d(O.gamma_delta(p.log_gamma)), n_filled=st0.n_filled)
    ref = tr.states[i]
    assert out[7] == ref.n_filled
    assert torch.equal(out[5].cpu(), ref.act)
    assert torch.equal(out[2].cpu(), ref.mass)
    assert rel_err(out[6].cpu(), ref.m_res) <= 1e-4


@pytest.mark.parametrize("name", ["dec_fp32", "dec_bf16"])
def test_decoder_matches_golden(name, gpu):
    """The decoder (chunked prefill, 220 single-token steps, in-decode consolidations).  Against the
    oracle forced onto the kernel's decisions: every step's final hidden state, every
    consolidation's decisions (equal to the oracle's own from the same state, near-ties within
    1e-4 counted), and the end state.  Against the reference's own vectors: every step and the
    end state when neither the kernel nor this host's CPU oracle took a near-tie the other way,
    otherwise the steps before the first one it affects.  The fixture's 96-token vocabulary
    repeats keys exactly, so equal redundancy and utility values decide evictions: the kernel
    orders them as torch.topk does."""
    g, meta = fixture(name)
    model, ids = build_model(meta)
    model_cpu = copy.deepcopy(model)
    from bolt3_amd import Bolt3Decoder
    n_prompt, n_dec = meta["n_prompt"], meta["n_decode"]

    def oracle_run(ref):
        with torch.no_grad():
            h, st = ref.prefill(ids[:, :n_prompt])
            hr, ev = [h[:, -1]], [len(ref.logs.get(0, []))]     # consolidations before each compared step
            for i in range(n_dec):
                pos = n_prompt + i
                hr.append(ref.step(ids[:, pos:pos + 1], pos, st)[:, -1])
                ev.append(len(ref.logs.get(0, [])))
        return torch.stack(hr, dim=1), st, ev

    ref_logs = {}
    h_oracle, _, ev_ref = oracle_run(O.HybridRef(model_cpu, logs=ref_logs))
    model = model.to(gpu)
    dec = Bolt3Decoder(model)
    ids_d = ids.to(gpu)
    rec = {}
    print(f"[case] {name} prefill {n_prompt} + {n_dec} steps", flush=True)
    with torch.no_grad():
        states, kv = dec.blank_state(model, ids.shape[0], gpu, max_kv_len=n_prompt + n_dec + 64)
        for s0 in range(0, n_prompt, dec.C):
            h, states, kv = dec.step(ids_d[:, s0:min(n_prompt, s0 + dec.C)], s0, states, kv, record=rec)
        hs = [h[:, -1]]
        for i in range(n_dec):
            pos = n_prompt + i
            h, states, kv = dec.step(ids_d[:, pos:pos + 1], pos, states, kv, record=rec)
            hs.append(h[:, -1])
    hs = torch.stack(hs, dim=1).cpu()
    # the oracle along the kernel's decisions
    forced = {li: [decisions_from_kernel_log(e["log"]) for e in evs] for li, evs in rec.items()}
    f_logs = {}
    h_f, st_f, _ = oracle_run(O.HybridRef(model_cpu, logs=f_logs, decisions=forced))
    mism = near = tie_rows = rnd = 0
    d_gpu = None
    for li, evs in rec.items():
        assert len(evs) == len(f_logs[li]) == len(ref_logs[li])
        for e, (gl, lg) in enumerate(zip(evs, f_logs[li])):
            a, b, c, d = _compare_step(lg, gl["log"].cpu(), gl["log"].shape[0], gl["tokens"],
                                       f"{name} layer {li} event {e}", meta["dtype"] == "bfloat16")
            mism, near, tie_rows, rnd = mism + a, near + b, tie_rows + c, rnd + d
            if (b or d) and (d_gpu is None or e < d_gpu):
                d_gpu = e
    fp32 = meta["dtype"] == "float32"
    for k in range(hs.shape[1]):
        _check_out(hs[:, k], h_f[:, k], hs.dtype, f"{name} step {k} vs forced oracle", normed=True)
    for li in rec:
        _check_state(kv[li], states[li].view(-1, *states[li].shape[2:]), st_f[li][1].st,
                     hs.dtype, f"{name} layer {li} end state vs forced oracle")
        e = rel_err(states[li].cpu(), st_f[li][0])
        assert e <= (1e-4 if fp32 else 1e-3), (li, e)
    close = lambda a, b: rel_err(a, b) <= (1e-5 if fp32 else 1e-2)
    d_oracle = next((k for k in range(h_oracle.shape[1]) if not close(h_oracle[:, k], g["h_last"][:, k])), None)
    lgs = ref_logs.get(0, [])
    if d_oracle is not None:            # a consolidation done before that step sat on a near-tie
        assert any(_step_has_near_tie(lg) for lg in lgs[:ev_ref[d_oracle]]), \
            f"oracle left the reference at step {d_oracle} without a near-tie"
    print(f"[decisions] {name}: events={len(lgs)} mismatches={mism} near-ties={near} rounding divergences={rnd} "
          f"rows ordered on exact ties={tie_rows} oracle departs at step={d_oracle} gpu near-tie at event={d_gpu}; "
          f"every step and the end state match the forced oracle", flush=True)
    assert mism == 0 and rnd == 0
    n_cmp = hs.shape[1]
    if d_gpu is not None:
        n_cmp = min(n_cmp, next(k for k in range(len(ev_ref)) if ev_ref[k] > d_gpu))
    if d_oracle is not None:
        n_cmp = min(n_cmp, d_oracle)
    for k in range(n_cmp):
        _check_out(hs[:, k], g["h_last"][:, k], hs.dtype, f"{name} step {k}", normed=True)
    if d_oracle is None and d_gpu is None:
        st = kv[0]
        assert st.n_filled == meta["n_filled"]
        assert torch.equal(st["act"].cpu().to(torch.uint8).view_as(g["final.act"]), g["final.act"])
        assert torch.equal(st["mass"].cpu().view_as(g["final.mass"]), g["final.mass"])
        assert rel_err(st["ak"].cpu().float(), g["final.ak"].float().view_as(st["ak"])) <= (1e-5 if fp32 else 1e-2)
        assert rel_err(states[0].cpu(), g["final.m_res"]) <= (1e-4 if fp32 else 1e-3)
    else:
        print(f"[case] {name}: compared with the reference on steps 0..{n_cmp - 1}", flush=True)


@pytest.mark.parametrize("dtype,head_dim,heads,qkv_bias", [
    (torch.float32, 128, (8, 2), False), (torch.bfloat16, 128, (8, 2), False),
    (torch.float32, 64, (8, 2), False), (torch.bfloat16, 64, (8, 2), False),
    (torch.bfloat16, 128, (8, 8), False), (torch.bfloat16, 128, (8, 1), False),
    (torch.bfloat16, 64, (8, 2), True), (torch.float32, 64, (8, 2), True)])
def test_decode_kernel_vs_oracle_layer_step(dtype, head_dim, heads, qkv_bias, gpu):
    """Prefill by chunks then single-token steps of one Bolt-3 layer, compared every step (both head
    dims the kernels are built for; bf16 runs the fused decode layer, fp32 the split kernels; the
    fused layer also at one and at eight query heads per kv head, the most it takes; and with
    biased q/k/v projections)."""
    from bolt3_amd import HybridLM, Bolt3Decoder
    import recipes
    torch.manual_seed(0)
    H, HKV = heads
    print(f"[case] decode layer step {dtype} head_dim={head_dim} heads={H}/{HKV} qkv_bias={qkv_bias}", flush=True)
    model = HybridLM(vocab_size=64, dim=128, num_layers=1, num_heads=H, num_kv_heads=HKV, intermediate=64,
                     layer_types=["vsa"], head_dim=head_dim, qk_norm=True, rope_theta=1e6, eps=1e-6,
                     qkv_bias=qkv_bias)
    recipes.init_module(model.blocks[0].vsa, 11, nondefault=True)
    model.load_state_dict(recipes.model_params([(k, tuple(v.shape)) for k, v in model.state_dict().items()], 11),
                          strict=False)
    model = model.to(dtype).eval()
    ref = O.HybridRef(model, ties="torch")
    import copy
    dev_model = copy.deepcopy(model).to(gpu)
    dec = Bolt3Decoder(dev_model)
    ids = recipes.tokens(11, 2, 300 + 140, 64)
    with torch.no_grad():
        h_ref, st_ref = ref.prefill(ids[:, :300])
        h, states, kv = dec.prefill(ids[:, :300].to(gpu))
        _check_out(h.cpu(), h_ref, dtype, "prefill", normed=True)
        for i in range(140):
            pos = 300 + i
            h_ref = ref.step(ids[:, pos:pos + 1], pos, st_ref)
            h, states, kv = dec.step(ids[:, pos:pos + 1].to(gpu), pos, states, kv)
            _check_out(h.cpu(), h_ref, dtype, f"decode step {i}", normed=True)
    assert kv[0].n_filled == st_ref[0][1].st.n_filled == 128


def _qwen3_layer(seed):
    """A Qwen3-4B-shape Bolt-3 layer as real checkpoints hold it: bf16 projections and q/k norms,
    fp32 Bolt-3 parameters (vsa_lm/benchmark.py:92-99)."""
    from bolt3_amd import Bolt3Attn
    import recipes
    cfg = dict(dim=2560, num_heads=32, num_kv_heads=8, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)
    mod = recipes.init_module(Bolt3Attn(cfg), seed, nondefault=False)
    for n, prm in mod.named_parameters():
        if "proj" in n and not n.startswith(("beta", "eta")) or "norm" in n and not n.startswith("res"):
            prm.data = prm.data.to(torch.bfloat16)
    return mod


def _whole_vs_forced(mod, x, y, trace, what):
    """The kernel's whole output and end state against the oracle run along the kernel's decisions;
    every step's decisions against the oracle's own from the same state.  Returns the forced
    oracle's trace."""
    log = trace["log"].cpu()
    tr_f = O.ForwardTrace()
    with torch.no_grad():
        y_f = O.forward(O.Bolt3Params.from_module(mod), x, trace=tr_f, decisions=decisions_from_kernel_log(log))
    mism, near, tie_rows, rnd, first = _forced_compare(tr_f, log, what, bf16=True)
    print(f"[decisions] {what}: steps={len(tr_f.logs)} rows={log.shape[1]} mismatches={mism} near-ties={near} "
          f"rounding divergences={rnd} rows ordered on exact ties={tie_rows} first near-tie at step={first}; "
          f"whole output vs forced oracle max-abs {max_abs(y, y_f):.3e} cos {cosine(y, y_f):.6f}", flush=True)
    assert mism == 0 and rnd <= _max_rounding(log)
    _check_out(y, y_f, torch.bfloat16, f"{what}: whole output vs forced oracle")
    _check_state(trace["state"], trace["m_res"], tr_f.states[-1], torch.bfloat16, f"{what}: end state")
    return tr_f


def test_full_size_cfg2_whole_output(gpu):
    """cfg2 at full size (B=4, T=4096, Qwen3-4B layer, bf16 projections, fp32 Bolt-3 params): the
    whole output (all 4 x 4096 tokens) and the end state against the oracle along the kernel's
    decisions, all 30 steps x 32 rows of decisions against the oracle's own; the output on the
    first 1024 tokens does not depend on what follows."""
    import recipes
    mod = _qwen3_layer(21)
    x = recipes.hidden(21, 4, 4096, 2560).to(torch.bfloat16)
    mod_d = copy.deepcopy(mod).to(gpu)
    print("[case] cfg2 full size B=4 T=4096 bf16", flush=True)
    trace = {}
    with torch.no_grad():
        y_full = mod_d(x.to(gpu), _trace=trace)
        y_pre = mod_d(x[:1, :1024].to(gpu))
    assert torch.isfinite(y_full).all()
    ma, cs = max_abs(y_full[:1, :1024].cpu(), y_pre.cpu()), cosine(y_full[:1, :1024].cpu(), y_pre.cpu())
    assert ma <= 2e-2 and cs >= 0.9995, (ma, cs)
    _whole_vs_forced(mod, x, y_full.cpu(), trace, "cfg2 B=4 T=4096")


def test_consolidation_heavy_long_prefill(gpu):
    """The consolidation-heavy configuration at full size (B=1, T=65536, Qwen3-4B layer, bf16
    projections, fp32 Bolt-3 parameters; hidden states around 512 centres with noise 0.15 and
    Zipf(1.1) cluster choice): 510 consolidation steps.  The whole output (65536 tokens) and the
    end state against the oracle along the kernel's decisions, every step's decisions against
    the oracle's own from the same state (clustered keys put many tokens within rounding of the
    merge thresholds and make fill and keep scores tie exactly: near-ties are counted, exact
    ties follow torch.topk's order); a steady share of merges; the first 2048 tokens do not
    depend on what follows."""
    import recipes
    mod = _qwen3_layer(31)
    print("[case] consolidation-heavy prefill B=1 T=65536 bf16", flush=True)
    x = recipes.clustered_hidden(31, 1, 65536, 2560, n_centres=512, noise=0.15).to(torch.bfloat16)
    mod_d = copy.deepcopy(mod).to(gpu)
    trace = {}
    with torch.no_grad():
        y = mod_d(x.to(gpu), _trace=trace)
        y_pre = mod_d(x[:, :2048].to(gpu))
    assert torch.isfinite(y).all()
    log = trace["log"]                       # [steps, bh, rows, cols]
    steady = log[4:, :, :, :128]             # the slots are full after the first steps
    merged = float(steady[:, :, LOG["merge"]].mean())
    to_m = float(steady[:, :, LOG["delta"]].mean())
    print(f"[case] merged share {merged:.3f}, M_res share {to_m:.3f} over {steady.shape[0]} steady steps", flush=True)
    assert 0.05 <= merged <= 0.95 and to_m > 0.0
    ma, cs = max_abs(y[:, :2048].cpu(), y_pre.cpu()), cosine(y[:, :2048].cpu(), y_pre.cpu())
    assert ma <= 2e-2 and cs >= 0.9995, (ma, cs)
    _whole_vs_forced(mod, x, y.cpu(), trace, "cfg4 B=1 T=65536")


def test_forward_under_autocast_matches_bf16_oracle(gpu):
    """An fp32 module called under bf16 autocast (the reference's eval, benchmark and heal paths
    run it so) stores its activations in bf16, as the reference's autocast linears produce them.
    With every parameter and input exactly representable in bf16, autocast's weight casts are
    exact, so the bf16 oracle (the reference's CPU semantics on the bf16-cast module) is the
    expected result: compared over the first chunks (before any consolidation, where no
    near-tie can move a decision) and, with bf16 tolerance, over the whole sequence."""
    import copy
    import recipes
    from bolt3_amd import Bolt3Attn
    cfg = dict(dim=256, num_heads=8, num_kv_heads=2, head_dim=128, rope_theta=1e6, eps=1e-6, qk_norm=True)
    mod = recipes.init_module(Bolt3Attn(cfg), 41, nondefault=True)
    with torch.no_grad():
        for prm in mod.parameters():
            prm.copy_(prm.to(torch.bfloat16).float())
    x = recipes.hidden(41, 2, 640, 256).to(torch.bfloat16).float()
    mod_bf = copy.deepcopy(mod).to(torch.bfloat16)
    with torch.no_grad():
        ref = O.forward(O.Bolt3Params.from_module(mod_bf), x.to(torch.bfloat16))
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = copy.deepcopy(mod).to(gpu)(x.to(gpu))
    assert y.dtype == torch.bfloat16
    _check_out(y[:, :256].float().cpu(), ref[:, :256].float(), torch.bfloat16, "autocast, first chunks")
    _check_out(y.float().cpu(), ref.float(), torch.bfloat16, "autocast, whole sequence")
