"""The decision comparison the GPU parity tests use (test_gpu_parity._compare_step), checked on
the CPU: an oracle run's decisions written in the kernel's log format agree with themselves, and
planted mistakes -- a flipped merge flag, a replacement sent to another slot, two fill picks
exchanged across the ranking -- are counted as mismatches, not excused as near-ties."""
import pytest
import torch

from bolt3_amd import _abi as A
from helpers import build_layer, decisions_from_kernel_log, fixture
from oracle import bolt3_oracle as O
import test_gpu_parity as P

LOG = {n: i for i, n in enumerate(A.LOG_FIELDS)}


def _kernel_log(lg, bh, l):
    """An oracle step log in the chain kernel's log layout (the rows the comparison reads)."""
    log = torch.zeros(bh, A.LOG_ROWS, A.LOG_COLS)
    if lg["kind"] == "fill":
        m = lg["picked"].shape[1]
        log[:, LOG["top_tok"], :m] = lg["picked"].float()
        log[:, LOG["score"], :l] = lg["score"]
        return log
    kc = lg["top_vals"].shape[1]
    log[:, LOG["merge"], :l] = lg["merge"].float()
    log[:, LOG["slot"], :l] = lg["slot"].float()
    log[:, LOG["delta"], :l] = lg["delta"].float()
    log[:, LOG["score"], :l] = lg["score"]
    log[:, LOG["keep"], :lg["keep"].shape[1]] = lg["keep"]
    log[:, LOG["top_tok"], :kc] = lg["top_toks"].float()
    log[:, LOG["bot_slot"], :kc] = lg["bot_slots"].float()
    log[:, LOG["win"], :kc] = lg["win"].float()
    log[:, LOG["top_val"], :kc] = lg["top_vals"]
    log[:, LOG["bot_val"], :kc] = lg["bot_vals"]
    return log


def _run(name):
    g, meta = fixture(name)
    mod, x = build_layer(meta)
    p = O.Bolt3Params.from_module(mod)
    tr = O.ForwardTrace()
    with torch.no_grad():
        O.forward(p, x, trace=tr)
    logs = torch.stack([_kernel_log(lg, c[0].shape[0], c[0].shape[1]) for lg, c in zip(tr.logs, tr.chunks)])
    return p, x, tr, logs


@pytest.mark.parametrize("name", ["fwd_fp32_eta", "fwd_bf16_clustered"])
def test_compare_rule_accepts_equal_and_catches_planted(name):
    p, x, tr, logs = _run(name)
    bf16 = x.dtype == torch.bfloat16
    assert P._forced_compare(tr, logs, name, bf16)[:4] == (0, 0, 0, 0)
    # the kernel-log round trip gives back the oracle's decisions
    tr2 = O.ForwardTrace()
    with torch.no_grad():
        assert torch.equal(O.forward(p, x, trace=tr2, decisions=decisions_from_kernel_log(logs)), O.forward(p, x))
    last = len(tr.logs) - 1
    # a merge flag flipped on a token whose cosine is far from the thresholds
    lg = tr.logs[last]
    far = ((lg["best"] - O.SIM_K).abs() > 0.05) & ((lg["sim_v"] - O.SIM_V).abs() > 0.05)
    r, j = [int(v) for v in torch.nonzero(far)[0]]
    bad = logs.clone()
    bad[last, r, LOG["merge"], j] = 1.0 - bad[last, r, LOG["merge"], j]
    assert P._forced_compare(tr, bad, name, bf16)[0] == 1
    # a winning token sent to another slot
    i = max(k for k, lg in enumerate(tr.logs) if lg["kind"] == "steady" and bool(lg["win"][:, 0].any()))
    r = int(torch.nonzero(tr.logs[i]["win"][:, 0])[0])
    bad = logs.clone()
    bad[i, r, LOG["bot_slot"], 0] = float((int(bad[i, r, LOG["bot_slot"], 0]) + 1) % p.S)
    assert P._forced_compare(tr, bad, name, bf16)[0] == 1
    # the first fill's 1st and 101st picks exchanged (scores far apart)
    bad = logs.clone()
    a, b = bad[0, 0, LOG["top_tok"], 0].clone(), bad[0, 0, LOG["top_tok"], 100].clone()
    sc = tr.logs[0]["score"][0]
    assert abs(float(sc[int(a)] - sc[int(b)])) > 1e-3 * abs(float(sc[int(a)]))
    bad[0, 0, LOG["top_tok"], 0], bad[0, 0, LOG["top_tok"], 100] = b, a
    assert P._forced_compare(tr, bad, name, bf16)[0] == 1
