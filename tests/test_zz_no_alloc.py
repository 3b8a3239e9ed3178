"""bolt3_chain_noalloc (the allocation-free variant of bolt3_chain) against bolt3_chain through
the C ABI: the same inputs give bit-identical slot states, M_res, snapshots and decision logs,
on two calls in a row, the second smaller than the first; a request beyond the library's scratch
is rejected before anything runs."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _problem(seed, B, HKV, HD, n_steps, dt, dev):
    """Keys and values around 12 centres per row (per-coordinate noise 0.2: cosines near 0.98, so
    tokens merge into the slots of their cluster), every second token drawn fresh (it competes
    for eviction or goes to M_res)."""
    g = torch.Generator().manual_seed(seed)
    C, bh = 128, B * HKV
    n_tok = n_steps * C
    ck, cv = torch.randn(bh, 12, HD, generator=g), torch.randn(bh, 12, HD, generator=g)
    z = torch.randint(0, 12, (bh, n_tok), generator=g)
    fresh = (torch.arange(n_tok) % 2 == 1).view(1, -1, 1)
    rows = torch.arange(bh).view(-1, 1)
    kr = torch.where(fresh, torch.randn(bh, n_tok, HD, generator=g), ck[rows, z] + 0.2 * torch.randn(bh, n_tok, HD, generator=g))
    v = torch.where(fresh, torch.randn(bh, n_tok, HD, generator=g), cv[rows, z] + 0.2 * torch.randn(bh, n_tok, HD, generator=g))
    pos = torch.arange(n_tok, dtype=torch.float32)
    ang = pos[:, None] * (1.0 / (1e4 ** (torch.arange(0, HD, 2).float() / HD)))[None, :]
    ang = torch.cat((ang, ang), dim=-1)
    rot = torch.cat((-kr[..., HD // 2:], kr[..., :HD // 2]), dim=-1)
    kp = kr * ang.cos() + rot * ang.sin()
    beta = torch.rand(bh, n_tok, generator=g)
    d = lambda t, t_dt=None: t.to(dtype=t_dt or t.dtype).to(dev).contiguous()
    return dict(kr=d(kr, dt), kp=d(kp, dt), v=d(v, dt), pos=d(pos), beta=d(beta),
                kappa=d(torch.rand(HKV, generator=g) + 0.5), gamma=d(torch.rand(HKV, generator=g) * 0.5 + 0.45),
                inv_freq=d((1.0 / (1e4 ** (torch.arange(0, HD, 2).float() / HD)))))


def _run(name, prob, B, HKV, HD, n_steps, dt, dev, lib):
    from bolt3_amd import _abi as A
    bh, S, C = B * HKV, 128, 128
    st = dict(ak=torch.empty(bh, S, HD, dtype=dt, device=dev), av=torch.empty(bh, S, HD, dtype=dt, device=dev),
              mass=torch.empty(bh, S, device=dev), util=torch.empty(bh, S, device=dev),
              pm=torch.empty(bh, S, device=dev), act=torch.empty(bh, S, dtype=torch.uint8, device=dev),
              m=torch.empty(bh, HD, HD, device=dev),
              snap_k=torch.empty(n_steps, bh, S, HD, dtype=dt, device=dev),
              snap_v=torch.empty(n_steps, bh, S, HD, dtype=dt, device=dev),
              snap_b=torch.empty(n_steps, bh, S, device=dev), snap_m=torch.empty(n_steps, bh, HD, HD, device=dev),
              log=torch.zeros(n_steps, bh, A.LOG_ROWS, A.LOG_COLS, device=dev))
    a = A.ChainArgs()
    a.dtype, a.B, a.HKV, a.HD, a.S = A.dtype_code(dt), B, HKV, HD, S
    a.kr, a.kp, a.v, a.tok_bh_stride = prob["kr"].data_ptr(), prob["kp"].data_ptr(), prob["v"].data_ptr(), n_steps * C * HD
    a.pos, a.beta, a.beta_bh_stride = prob["pos"].data_ptr(), prob["beta"].data_ptr(), n_steps * C
    a.n_steps, a.off0, a.len0, a.step_stride, a.step_len = n_steps, 0, C, C, C
    a.n_filled, a.kp_exact = 0, 1
    a.ak, a.av, a.mass, a.util, a.pm, a.act = (st[k].data_ptr() for k in ("ak", "av", "mass", "util", "pm", "act"))
    a.m_res = st["m"].data_ptr()
    a.kappa, a.gamma, a.inv_freq = prob["kappa"].data_ptr(), prob["gamma"].data_ptr(), prob["inv_freq"].data_ptr()
    a.snap_k, a.snap_v, a.snap_bias, a.snap_m = (st[k].data_ptr() for k in ("snap_k", "snap_v", "snap_b", "snap_m"))
    a.log = st["log"].data_ptr()
    work = None
    if name == "bolt3_chain":
        work = torch.empty(A.chain_workspace_bytes(dt, B, HKV, HD, S, n_steps), dtype=torch.uint8, device=dev)
        a.work, a.work_bytes = work.data_ptr(), work.numel()
    stream = torch.cuda.current_stream(dev)
    rc = getattr(lib, name)(ctypes.byref(a), ctypes.c_void_p(stream.cuda_stream))
    assert rc == 0, (name, rc)
    torch.cuda.synchronize()
    return {k: t.cpu() for k, t in st.items()}


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_noalloc_matches_chain_twice(dt, gpu):
    from bolt3_amd import _abi as A
    lib = A.load()
    C = 128
    for B, HKV, HD, n_steps in ((4, 8, 128, 6), (1, 2, 64, 5)):    # the second call is smaller
        print(f"[case] noalloc vs chain {dt} B={B} HKV={HKV} HD={HD} steps={n_steps}", flush=True)
        prob = _problem(B * 100 + n_steps, B, HKV, HD, n_steps, dt, gpu)
        ref = _run("bolt3_chain", prob, B, HKV, HD, n_steps, dt, gpu, lib)
        got = _run("bolt3_chain_noalloc", prob, B, HKV, HD, n_steps, dt, gpu, lib)
        for k in ref:
            assert torch.equal(ref[k], got[k]), (dt, B, k)
        # the merge, eviction and M_res branches all ran through the scratch (steady steps: 2..)
        steady = ref["log"][2:, :, :, :C]
        n_merge = int(steady[:, :, A.LOG_FIELDS.index("merge")].sum())
        n_win = int(ref["log"][2:, :, A.LOG_FIELDS.index("win"), :C].sum())
        n_delta = int(steady[:, :, A.LOG_FIELDS.index("delta")].sum())
        print(f"[case] merged {n_merge}, replaced {n_win}, to M_res {n_delta}", flush=True)
        assert n_merge > 0 and n_win > 0 and n_delta > 0
        assert float(ref["m"].abs().max()) > 0


def test_noalloc_rejects_oversize(gpu):
    from bolt3_amd import _abi as A
    lib = A.load()
    a = A.ChainArgs()
    a.dtype, a.B, a.HKV, a.HD, a.S, a.n_steps = 1, 64, 8, 128, 128, 100
    need = A.chain_workspace_bytes(torch.bfloat16, 64, 8, 128, 128, 100)
    assert need > A.CHAIN_NOALLOC_SCRATCH_BYTES
    assert lib.bolt3_chain_noalloc(ctypes.byref(a), None) == 1003
