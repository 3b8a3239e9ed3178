"""The kernels' RoPE sine / cosine (vsa-lm_amd/csrc/bolt3_math.h, sincos_rope) over every angle
the configurations produce: position * inverse frequency for positions 0..65535 and fractional
slot positions, against double precision and against torch's fp32 sin / cos (what the
reference's RoPE calls, vsa_lm/surgery.py:86-93, vsa_lm/config/bolt3.py:17-20).  The function
is compiled for the host from the same header; its operations (fmaf, rintf, products) round
alike on host and device."""
import os
import subprocess
import tempfile

import numpy as np
import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def probe():
    d = tempfile.mkdtemp()
    exe = os.path.join(d, "rope_probe")
    r = subprocess.run([HIPCC, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950",
                        f"-I{os.path.join(REPO, 'vsa-lm_amd', 'csrc')}",
                        os.path.join(REPO, "tests", "rope_math_probe.cpp"), "-o", exe],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip(f"hipcc unavailable for the host probe: {r.stderr[-500:]}")
    return exe


def _run(exe, x: np.ndarray):
    out = subprocess.run([exe], input=x.astype(np.float32).tobytes(), capture_output=True, check=True).stdout
    y = np.frombuffer(out, dtype=np.float32)
    return y[:x.size], y[x.size:]


def _angles():
    """pos * inv_freq as the kernels form it (one fp32 product) for every position up to 65535 and
    the frequencies of head_dim 64 / theta 1e4 and head_dim 128 / theta 1e6, plus fractional
    positions (slot means) up to 65535."""
    pos = np.arange(65536, dtype=np.float32)
    rng = np.random.default_rng(0)
    frac = (rng.random(200000) * 65535).astype(np.float32)
    out = []
    for hd, theta in ((64, 1e4), (128, 1e6)):
        inv = (1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.int64).float() / hd))).numpy().astype(np.float32)
        for f in inv[::3]:
            out.append(pos * f)
            out.append(frac * f)
    return np.concatenate(out)


def test_sincos_against_double_and_torch(probe):
    x = _angles()
    s, c = _run(probe, x)
    xd = x.astype(np.float64)
    ulp = lambda v: np.spacing(np.abs(v).astype(np.float32)).astype(np.float64)
    es = np.abs(s - np.sin(xd)) / np.maximum(ulp(np.sin(xd)), np.spacing(np.float32(1e-30)))
    ec = np.abs(c - np.cos(xd)) / np.maximum(ulp(np.cos(xd)), np.spacing(np.float32(1e-30)))
    # in ulps of the result, except near zeros of sin / cos where the absolute error counts
    big_s, big_c = np.abs(np.sin(xd)) > 1e-3, np.abs(np.cos(xd)) > 1e-3
    assert es[big_s].max() <= 2.5 and ec[big_c].max() <= 2.5, (es[big_s].max(), ec[big_c].max())
    assert np.abs(s - np.sin(xd)).max() <= 3e-7 and np.abs(c - np.cos(xd)).max() <= 3e-7
    ts, tc = torch.from_numpy(x).sin().numpy(), torch.from_numpy(x).cos().numpy()
    assert np.abs(s - ts).max() <= 4.8e-7 and np.abs(c - tc).max() <= 4.8e-7


def test_rope_identity_and_quadrants(probe):
    x = np.array([0.0, np.pi / 2, np.pi, 3 * np.pi / 2, 2 * np.pi, -np.pi / 2, 1e-20], dtype=np.float32)
    s, c = _run(probe, x)
    assert s[0] == 0.0 and c[0] == 1.0 and s[6] == np.float32(1e-20) and c[6] == 1.0
    assert np.allclose(s[1:6], [1, 0, -1, 0, -1], atol=3e-7) and np.allclose(c[1:6], [0, -1, 0, 1, 0], atol=3e-7)
