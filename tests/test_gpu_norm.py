"""bolt3_rms_norm (the RMSNorm of the layers around the Bolt-3 path) against the torch ops of
vsa_lm/surgery.py:48-52 on the same device: fp32 within 2 ulp-level relative error, bf16 within
one bf16 rounding of every element; row counts that leave partial workgroups, strided rows, fp32
and bf16 weights; and the CPU path still the torch ops."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _torch_rms(x, w, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * w.float()).to(x.dtype)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 2560), (7, 3, 128), (33, 2560), (2, 5, 64)])
def test_rms_norm_matches_torch(dt, wdt, shape, gpu):
    from bolt3_amd import RMSNorm
    g = torch.Generator(device=gpu).manual_seed(3)
    x = (torch.randn(*shape, generator=g, device=gpu) * 3.0).to(dt)
    norm = RMSNorm(shape[-1], 1e-6).to(gpu)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(shape[-1], generator=g, device=gpu) + 0.5)
    norm = norm.to(wdt)
    with torch.no_grad():
        y = norm(x)
        ref = _torch_rms(x, norm.weight, 1e-6)
    assert y.dtype == dt and y.shape == x.shape
    d = (y.float() - ref.float()).abs()
    tol = ref.float().abs() * (2 ** -7 if dt == torch.bfloat16 else 4e-7) + 1e-30
    assert bool((d <= tol).all()), float((d / tol).max())


def test_rms_norm_strided_rows_and_cpu(gpu):
    from bolt3_amd import RMSNorm
    norm = RMSNorm(128, 1e-5).to(gpu)
    big = torch.randn(10, 256, device=gpu)
    x = big[:, 64:192]                          # rows 256 floats apart
    with torch.no_grad():
        y = norm(x)
        assert torch.allclose(y, _torch_rms(x, norm.weight, 1e-5), rtol=1e-6, atol=1e-7)
        xc = x.cpu()
        assert torch.equal(norm.cpu()(xc), _torch_rms(xc, norm.weight.cpu(), 1e-5))
