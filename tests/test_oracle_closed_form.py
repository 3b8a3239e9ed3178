"""Pin the oracle with closed forms, invariants and brute force on small inputs.

Each check uses a formulation independent of the oracle's code path (numpy,
complex rotation, torch SDPA, Python sorting) so that a dropped term, a wrong
sign or index, or a transposed operand fails at least one of them.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import bolt3_oracle as O


def _params(D=32, H=4, HKV=2, HD=16, S=8, C=8, seed=0, theta=10000.0, eta=False):
    g = torch.Generator().manual_seed(seed)
    n = lambda *s, std=0.02: torch.randn(*s, generator=g) * std
    return O.Bolt3Params(
        D=D, H=H, HKV=HKV, HD=HD, eps=1e-5, S=S, C=C,
        wq=n(H * HD, D, std=0.2), wk=n(HKV * HD, D, std=0.2), wv=n(HKV * HD, D, std=0.2), wo=n(D, H * HD, std=0.2),
        wb=n(HKV, D) if eta else torch.zeros(HKV, D), bb=torch.full((HKV,), -1.0),
        we=n(H, D, std=0.3) if eta else torch.zeros(H, D), be=torch.zeros(H),
        kappa=torch.ones(HKV), log_gamma=torch.full((HKV,), 3.5), res_w=torch.full((HD,), 0.05),
        inv_freq=O.rope_inv_freq(HD, theta))


# ------------------------------------------------------------------ RoPE and gamma

def test_rope_is_complex_rotation():
    HD = 16
    inv = O.rope_inv_freq(HD, 10000.0)
    x = torch.randn(3, 5, HD, dtype=torch.float64).float()
    pos = torch.tensor([0.0, 1.0, 7.5, 1000.0, 65535.0])
    y = O.rope_at(x, pos.view(1, 5).expand(3, 5), inv)
    z = (x[..., :HD // 2].double() + 1j * x[..., HD // 2:].double())
    ang = (pos[:, None] * inv[None, :]).double()       # the angle is defined as an fp32 product
    zr = z * torch.exp(1j * ang)
    ref = torch.cat([zr.real, zr.imag], dim=-1)
    assert float((y.double() - ref).abs().max()) < 2e-5
    assert torch.equal(O.rope_at(x, torch.zeros(3, 5), inv), x)  # position 0 is the identity


def test_inv_freq_closed_form():
    inv = O.rope_inv_freq(128, 1e6)
    ref = np.array([1e6 ** (-2 * i / 128) for i in range(64)])
    assert np.allclose(inv.double().numpy(), ref, rtol=1e-6)


def test_gamma_default():
    g = O.gamma_delta(torch.full((3,), 3.5))
    assert abs(float(g[0]) - 0.999 / (1 + math.exp(-3.5))) < 1e-6
    assert float(O.gamma_delta(torch.tensor([100.0]))) == pytest.approx(0.999, abs=1e-6)
    assert float(O.gamma_delta(torch.tensor([-100.0]))) == pytest.approx(1e-3, abs=1e-9)


# ------------------------------------------------------------------ attention

def test_first_two_chunks_are_causal_sdpa():
    """Before any consolidation the layer is causal attention over the previous and current chunk."""
    p = _params(C=8)
    x = torch.randn(2, 16, p.D)
    y = O.forward(p, x)
    q, k, v, _, _ = O.project(p, x)
    pos = torch.arange(16, dtype=torch.float32)
    q, k = O.rope_at(q, pos, p.inv_freq), O.rope_at(k, pos, p.inv_freq)
    a = F.scaled_dot_product_attention(q.double(), k.double().repeat_interleave(p.G, 1),
                                       v.double().repeat_interleave(p.G, 1), is_causal=True)
    ref = F.linear(a.transpose(1, 2).reshape(2, 16, -1), p.wo.double())
    assert float((y.double() - ref).abs().max()) < 1e-5


def test_chunk_attention_brute_force():
    """Chunk >= 2 against an explicit loop over the key list [sinks | slots | window]."""
    p = _params(C=8, S=8, eta=True)
    b, T = 1, 24
    x = torch.randn(b, T, p.D)
    tr = O.ForwardTrace()
    y = O.forward(p, x, trace=tr)
    q_raw, k_raw, v, _, eta = O.project(p, x)
    pos = torch.arange(T, dtype=torch.float32)
    qp, kp = O.rope_at(q_raw, pos, p.inv_freq), O.rope_at(k_raw, pos, p.inv_freq)
    st = tr.states[0]                      # consolidation of chunk 0 feeds chunk 2
    gam = O.gamma_delta(p.log_gamma)
    outs = []
    for t in range(16, 24):
        row = []
        for h in range(p.H):
            kv = h // p.G
            keys, vals, bias = [], [], []
            for j in range(4):
                keys.append(kp[0, kv, j]); vals.append(v[0, kv, j]); bias.append(0.0)
            for s in range(p.S):
                ang = st.pm[kv, s] * p.inv_freq
                c, si = torch.cos(torch.cat([ang, ang])), torch.sin(torch.cat([ang, ang]))
                a = st.ak[kv, s]
                rot = torch.cat([-a[p.HD // 2:], a[:p.HD // 2]])
                keys.append(a * c + rot * si); vals.append(st.av[kv, s])
                bias.append(float(p.kappa[kv]) * math.log(max(float(st.mass[kv, s]), 1.0)) if st.act[kv, s]
                            else -math.inf)
            for j in range(8, t + 1):
                keys.append(kp[0, kv, j]); vals.append(v[0, kv, j]); bias.append(0.0)
            sc = torch.stack([(qp[0, h, t].double() @ kk.double()) / math.sqrt(p.HD) + bb
                              for kk, bb in zip(keys, bias)])
            pr = torch.softmax(sc, 0)
            att = sum(pr[i] * vals[i].double() for i in range(len(vals)))
            qn = q_raw[0, h, t].double() / q_raw[0, h, t].double().norm()
            ym = qn @ st.m_res[kv].double() * (1 - float(gam[kv])) / math.sqrt(p.HD)
            ym = ym / torch.sqrt((ym ** 2).mean() + p.eps) * p.res_w.double()
            row.append(att + float(eta[0, h, t, 0]) * ym)
        outs.append(torch.cat(row))
    ref = torch.stack(outs) @ p.wo.double().T
    assert float((y[0, 16:24].double() - ref).abs().max()) < 1e-5


# ------------------------------------------------------------------ consolidation

def _steady_state(bh=1, S=8, HD=16, seed=1, util=0.5):
    g = torch.Generator().manual_seed(seed)
    ak = torch.randn(bh, S, HD, generator=g)
    st = O.SlotState(ak=ak, av=torch.randn(bh, S, HD, generator=g), mass=torch.ones(bh, S),
                     util=torch.full((bh, S), util), pm=torch.arange(S, dtype=torch.float32).repeat(bh, 1),
                     act=torch.ones(bh, S, dtype=torch.bool), m_res=torch.randn(bh, HD, HD, generator=g) * 0.1,
                     n_filled=S)
    return st


def test_first_fill_picks_highest_variance_values():
    p = _params(H=2, HKV=1, S=8, C=8, HD=16)
    g = torch.Generator().manual_seed(3)
    l = 6
    kr, v = torch.randn(1, l, 16, generator=g), torch.randn(1, l, 16, generator=g)
    st = O.consolidate(p, None, kr, kr, v, torch.arange(10, 10 + l, dtype=torch.float32), torch.ones(1, l),
                       torch.full((1,), 0.9), 1)
    vn = v[0].numpy() / np.linalg.norm(v[0].numpy(), axis=1, keepdims=True)
    order = np.argsort(-vn.var(axis=1, ddof=1), kind="stable")
    assert st.n_filled == 6
    assert torch.equal(st.ak[0, :6], kr[0, torch.from_numpy(order.copy())])
    assert torch.equal(st.pm[0, :6], torch.from_numpy(10.0 + order).float())
    assert torch.all(st.util[0, :6] == 0.15) and torch.all(st.util[0, 6:] == 0) and int(st.act.sum()) == 6
    assert torch.count_nonzero(st.m_res) == 0


def test_delta_rule_single_key_closed_form():
    """One token that neither merges nor wins: M <- g*M + k^T (v - k M) * beta (classic delta rule)."""
    p = _params(H=2, HKV=1, S=8, C=8, HD=16)
    st = _steady_state(util=1e6)                       # huge utility: no slot can be evicted
    g = torch.Generator().manual_seed(5)
    kr = torch.randn(1, 1, 16, generator=g)
    v = torch.randn(1, 1, 16, generator=g)
    gam = torch.tensor([0.97])
    new = O.consolidate(p, st, kr, kr, v, torch.tensor([100.0]), torch.tensor([[0.3]]), gam, 1)
    k = (kr[0, 0] / kr[0, 0].norm()).double()
    M = st.m_res[0].double()
    ref = 0.97 * M + torch.outer(k, (v[0, 0].double() - k @ M) * 0.3)
    assert float((new.m_res[0].double() - ref).abs().max()) < 1e-6
    assert torch.equal(new.ak, st.ak) and torch.equal(new.mass, st.mass)


def test_delta_rule_zero_beta_is_pure_decay():
    p = _params(H=2, HKV=1, S=8, C=8, HD=16)
    st = _steady_state(util=1e6)
    kr = torch.randn(1, 5, 16)
    new = O.consolidate(p, st, kr, kr, torch.randn(1, 5, 16), torch.arange(5.0), torch.zeros(1, 5),
                        torch.tensor([0.9]), 1)
    assert torch.allclose(new.m_res, 0.9 * st.m_res, rtol=0, atol=1e-7)


def test_gershgorin_scaling_bounds_the_step():
    """Parallel keys: the row sums of |K K^T| diag(w) are capped so that the joint step stays <= 1."""
    p = _params(H=2, HKV=1, S=8, C=8, HD=16)
    st = _steady_state(util=1e6)
    st.m_res.zero_()
    k = torch.randn(16)
    kr = torch.stack([k, 2 * k, -k, 0.5 * k]).unsqueeze(0)          # all parallel: |cos| = 1
    v = torch.randn(1, 4, 16)
    beta = torch.full((1, 4), 0.8)
    new = O.consolidate(p, st, kr, kr, v, torch.arange(4.0), beta, torch.tensor([1.0]), 1)
    kh = (k / k.norm()).double()
    signs = torch.tensor([1.0, 1.0, -1.0, 1.0], dtype=torch.float64)
    w = 0.8 / max(4 * 0.8, 1.0)                                      # every row sums to 3.2
    ref = sum(torch.outer(signs[j] * kh, v[0, j].double() * w) for j in range(4))
    assert float((new.m_res[0].double() - ref).abs().max()) < 1e-5


def test_merge_is_mass_weighted_mean():
    p = _params(H=2, HKV=1, S=8, C=8, HD=16)
    st = _steady_state(util=1e6)
    st.mass[0, 3] = 3.0
    kr = (2.5 * st.ak[0, 3]).view(1, 1, 16)            # cos_k = 1 with slot 3
    v = (0.7 * st.av[0, 3]).view(1, 1, 16)             # cos_v = 1
    new = O.consolidate(p, st, kr, kr, v, torch.tensor([40.0]), torch.ones(1, 1), torch.tensor([0.9]), 1)
    assert float(new.mass[0, 3]) == 4.0
    assert torch.allclose(new.ak[0, 3], (3 * st.ak[0, 3] + kr[0, 0]) / 4, atol=1e-6)
    assert torch.allclose(new.av[0, 3], (3 * st.av[0, 3] + v[0, 0]) / 4, atol=1e-6)
    assert float(new.pm[0, 3]) == pytest.approx((3 * 3.0 + 40.0) / 4)
    others = [s for s in range(8) if s != 3]
    assert torch.equal(new.ak[0, others], st.ak[0, others])
    assert torch.allclose(new.m_res, 0.9 * st.m_res)   # the merged token is not written to M_res
    assert float(new.mass.sum() - st.mass.sum()) == 1.0


def test_eviction_brute_force():
    """Replacement set against a direct sort: i-th best free token vs i-th least useful slot."""
    p = _params(H=2, HKV=1, S=8, C=8, HD=16)
    for seed in range(6):
        st = _steady_state(seed=seed, util=0.0)
        g = torch.Generator().manual_seed(100 + seed)
        st.util = torch.rand(1, 8, generator=g) * 0.5
        kr = torch.randn(1, 8, 16, generator=g)
        v = torch.randn(1, 8, 16, generator=g)
        log = {}
        new = O.consolidate(p, st, kr, kr, v, torch.arange(50.0, 58.0), torch.ones(1, 8), torch.tensor([0.9]),
                            1, log=log)
        score = log["score"][0].tolist()
        merged = log["merge"][0].tolist()
        akn = F.normalize(new.ak[0].float(), dim=-1)
        cand = [(-1e9 if merged[j] else score[j], j) for j in range(8)]
        tops = sorted(cand, key=lambda t: -t[0])
        keep = log["keep"][0].tolist()
        bots = sorted([(keep[s], s) for s in range(8)], key=lambda t: t[0])
        wins = [(tj, bs) for (tv, tj), (bv, bs) in zip(tops, bots) if tv > bv and tv > -1e8]
        assert log["win"][0].tolist() == sorted(log["win"][0].tolist(), reverse=True)   # a prefix
        for tj, bs in wins:
            assert torch.equal(new.ak[0, bs], kr[0, tj]) and float(new.mass[0, bs]) == 1.0
            assert float(new.pm[0, bs]) == 50.0 + tj
        win_toks = {tj for tj, _ in wins}
        expect_delta = [not merged[j] and j not in win_toks for j in range(8)]
        assert log["delta"][0].tolist() == expect_delta
        del akn


def test_keep_score_uses_redundancy():
    """Duplicate slots are the least useful ones."""
    p = _params(H=2, HKV=1, S=8, C=8, HD=16)
    st = _steady_state(util=0.5)
    st.ak[0, 5] = st.ak[0, 2] * 1.01
    log = {}
    O.consolidate(p, st, torch.randn(1, 8, 16), torch.randn(1, 8, 16), torch.randn(1, 8, 16), torch.arange(8.0),
                  torch.ones(1, 8), torch.tensor([0.9]), 1, log=log)
    keep = log["keep"][0]
    assert set(log["bot_slots"][0, :2].tolist()) == {2, 5}
    assert float(keep[2]) == pytest.approx(0.5 * 0.995 * 0.02, rel=1e-3)


def test_llama3_inv_freq_against_transformers():
    """The llama3 band rescaling (vsa_lm/surgery.py:56-72), oracle and product, against the
    independent implementation in transformers (Llama 3.2 settings), and its band structure:
    the high-frequency band unchanged, the low-frequency band divided by `factor`."""
    tr = pytest.importorskip("transformers")
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    from bolt3_amd.layers import rope_inv_freq
    rs = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
    for hd, theta in ((64, 500000.0), (128, 500000.0)):
        cfg = tr.LlamaConfig(hidden_size=32 * hd, num_attention_heads=32, head_dim=hd, rope_theta=theta,
                             rope_scaling=rs, max_position_embeddings=131072)
        ref, _ = ROPE_INIT_FUNCTIONS["llama3"](cfg, "cpu")
        assert torch.equal(O.rope_inv_freq(hd, theta, rs), ref.float())
        assert torch.equal(rope_inv_freq(hd, theta, rs), ref.float())
        plain = O.rope_inv_freq(hd, theta)
        wl = 2 * math.pi / plain
        hi_band, lo_band = wl < 8192 / 4.0, wl > 8192 / 1.0
        assert hi_band.any() and lo_band.any()
        assert torch.equal(ref.float()[hi_band], plain[hi_band])
        assert torch.allclose(ref.float()[lo_band], plain[lo_band] / 32.0, rtol=1e-6)
