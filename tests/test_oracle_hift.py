"""Pins of the HiFT oracle (CPU): ISTFT against torch.istft, STFT/ISTFT round trip, closed forms of Snake, the
cross-fade, the noise seeds and the NSF phase of a constant f0, and the reference's own outputs (golden vectors)."""

import os

import numpy as np
import pytest
import torch

from oracle import hift as oh

import t2w_amd  # noqa: F401
from t2w_amd.config import HiFTConfig
from t2w_amd.weights import init_hift

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "hift_reference_vectors.npz")


@pytest.fixture(scope="module")
def h():
    return oh.HiFT(init_hift(HiFTConfig(), seed=3))


def test_istft_overlap_add_equals_torch_istft():
    g = torch.Generator().manual_seed(0)
    spec = torch.complex(torch.randn(2, 9, 41, generator=g), torch.randn(2, 9, 41, generator=g))
    spec[:, 0].imag = 0
    spec[:, 8].imag = 0
    win = torch.hann_window(16, periodic=True)
    ref = torch.istft(spec, 16, 4, 16, win, center=True)
    torch.testing.assert_close(oh.istft_overlap_add(spec, 16, 4, win), ref, rtol=1e-5, atol=1e-6)


def test_stft_then_istft_is_identity(h):
    x = torch.randn(3, 480 * 5, generator=torch.Generator().manual_seed(1))
    re, im = h._stft(x)
    y = oh.istft_overlap_add(torch.complex(re, im), 16, 4, h.stft_window)
    torch.testing.assert_close(y, x, rtol=1e-5, atol=1e-5)


def test_snake_closed_form():
    x = torch.linspace(-5, 5, 101)[None, None].expand(1, 3, 101)
    a = torch.tensor([0.5, 1.0, 1.7])
    ref = x.double() + (1 / (a.double()[None, :, None] + 1e-9)) * torch.sin(x.double() * a.double()[None, :, None]) ** 2
    np.testing.assert_allclose(oh.snake(x, a).double().numpy(), ref.numpy(), rtol=1e-6, atol=1e-6)


def test_fade_in_out_closed_form():
    win = oh.hamming_window()
    n = len(win) // 2
    a, b = torch.randn(1, 5000), torch.randn(1, 4000)
    out = oh.fade_in_out(a, b, win)
    w = np.hamming(2 * n)
    np.testing.assert_allclose(out[0, :n].numpy(), (a[0, :n].double().numpy() * w[:n] + b[0, -n:].double().numpy() * w[n:]).astype(np.float32),
                               rtol=1e-6, atol=1e-7)
    assert torch.equal(out[:, n:], a[:, n:])


def test_chunk_noise_seed_closed_form():
    assert oh.chunk_noise_seed(0, 5) == 5
    assert oh.chunk_noise_seed(3, 2) == 3 * 1_000_003 + 2
    assert oh.chunk_noise_seed(2 ** 62, 1) == (2 ** 62 * 1_000_003 + 1) % 2 ** 63


def test_nsf_phase_of_a_constant_f0(h):
    """Constant voiced f0 F: the integrated phase of harmonic k is 2 pi k F / sr (n + 240.5) wherever the linear
    interpolation stays inside the frame range (a dropped x480, a cumsum offset or a wrong interpolation centre fails);
    noise zero, so the source is tanh(w . 0.1 sin(phase) + b)."""
    T, F = 20, 137.0
    f0 = torch.full((1, T), F)
    noise = torch.zeros(1, T * 480, 9)
    s = oh.source(h, torch.zeros(1, 80, T), torch.zeros(1, 1, 0), torch.zeros(1, 9), noise, f0=f0)[0, 0].double()
    n = torch.arange(240, (T - 1) * 480 + 240, dtype=torch.float64)
    k = torch.arange(1, 10, dtype=torch.float64)
    rad = torch.remainder(F * k / 24000, 1)
    ph = 2 * np.pi * rad[None] * (n[:, None] + 240.5)
    w, b = h.m_source.w.double()[0], h.m_source.b.double()[0]
    ref = torch.tanh((0.1 * torch.sin(ph)) @ w + b)
    err = (s[240:(T - 1) * 480 + 240] - ref).abs().max()
    assert err < 2e-3, float(err)  # fp32 phase of ~1e5 rad carries ~1e-2 rad of rounding; sin is bounded by it


def test_rand_ini_never_reaches_the_source(h):
    """The frame-rate phase interpolates samples 480 f + 239 / 240, so the initial phases added to sample 0 drop out."""
    g = torch.Generator().manual_seed(2)
    mel = torch.randn(1, 80, 6, generator=g) * 2 - 5
    nz = torch.randn(1, 6 * 480, 9, generator=g)
    a = oh.source(h, mel, torch.zeros(1, 1, 0), torch.zeros(1, 9), nz)
    b = oh.source(h, mel, torch.zeros(1, 1, 0), torch.rand(1, 9, generator=g), nz)
    assert torch.equal(a, b)


@pytest.mark.skipif(not os.path.exists(GOLDEN), reason="golden vectors not generated")
def test_matches_reference_hift_forward_noise_golden(h):
    """Vectors written by tests/golden/make_hift_golden.py from the reference's own ``hift_forward_noise`` /
    ``fade_in_out`` / ``chunk_noise_seed`` run on this oracle's module objects."""
    z = np.load(GOLDEN)
    mel, cs, ri, nz = (torch.from_numpy(z[k]) for k in ("mel", "cache_source", "rand_ini", "noise"))
    sp, src = oh.forward_noise(h, mel, cs, ri, nz)
    np.testing.assert_allclose(sp.numpy(), z["speech"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(src.numpy(), z["source"], rtol=1e-5, atol=1e-6)
    fo = oh.fade_in_out(torch.from_numpy(z["fade_a"]), torch.from_numpy(z["fade_b"]), oh.hamming_window())
    np.testing.assert_array_equal(fo.numpy(), z["fade_out"])
    assert [oh.chunk_noise_seed(int(a), int(b)) for a, b in z["seed_args"]] == list(z["seeds"])
