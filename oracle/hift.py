"""Oracle of the HiFT vocoder with injected source noise, and of its streaming glue (fp32, CPU).

Follows, in the reference repository:

* ``engine/models/token2wav.py:214-236`` (``hift_forward_noise``: f0 predictor, nearest upsampling by 480, harmonic
  frequencies, ``rad = (fn / sr) % 1``, ``rand_ini[:, 0] = 0`` added to the first frame, phase integrated at frame rate
  by linear down-interpolation, cumsum, times 2 pi, linear up-interpolation of ``phase * 480``; ``sin * sine_amp``;
  voiced/unvoiced mix with the given noise; ``tanh(Linear(9 -> 1))``; the first ``cache_source`` samples replaced by the
  cache), ``:160-192`` (``_hift_decode``: STFT of the source, conv_pre, three upsampling stages with leaky ReLU,
  transposed conv, reflection pad before the last stage's fusion, source branch, mean of three ResBlocks; leaky ReLU
  (slope 0.01), conv_post, ``exp`` clipped at 1e2, ``sin`` phase, ISTFT, clamp), ``:128-138`` (``istft_overlap_add``),
  ``:112-121`` (``hift_noise``), ``:108-109`` (``chunk_noise_seed``), ``:81-85`` (``fade_in_out``), ``:319-332``
  (streaming decode glue: 8 cached mel frames, 3840 cached source samples, Hamming cross-fade, hold-back);
* ``engine/runtime/hift_lean.py:27-30, 115-124`` (Snake ``x + 1 / (alpha + 1e-9) * sin(x * alpha)^2``; weight norm
  folded once, so weights here are plain tensors).

Defined here (inside ``stepaudio2`` / CosyVoice2's ``HiFTGenerator``, not visible in the reference): 24 kHz, base 512
channels halving per stage, upsample rates 8/5/3 with kernels 16/11/7, ResBlock kernels 3/7/11 with dilations 1/3/5,
source ResBlock kernels 7/7/11, source downsampling convs (kernel 2u, stride u, pad u//2; 1x1 for u = 1), 8 harmonics,
sine amp 0.1, noise std 0.003, voiced threshold 10, lrelu slope 0.1, audio limit 0.99, Hann window (periodic) of 16,
f0 predictor = five kernel-3 convs with ELU then Linear(512 -> 1) and abs.  Parity unpinned against stepaudio2; the glue
order is pinned by golden vectors from the reference's own ``hift_forward_noise`` / ``_hift_decode`` (see
``tests/golden``).

The class below exposes the attribute names ``hift_forward_noise`` reads, so the same object can drive the reference
functions when the golden vectors are regenerated.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

SAMPLE_RATE = 24000
MEL_CACHE = 8
SOURCE_CACHE = MEL_CACHE * 480


@dataclass(frozen=True)
class HiFTDims:
    mel: int = 80
    base: int = 512
    up_rates: tuple = (8, 5, 3)
    up_kernels: tuple = (16, 11, 7)
    res_kernels: tuple = (3, 7, 11)
    res_dilations: tuple = (1, 3, 5)
    src_res_kernels: tuple = (7, 7, 11)
    n_fft: int = 16
    hop: int = 4
    harmonics: int = 8
    sr: int = SAMPLE_RATE
    sine_amp: float = 0.1
    noise_std: float = 0.003
    voiced_threshold: float = 10.0
    lrelu_slope: float = 0.1
    audio_limit: float = 0.99
    f0_channels: int = 512
    f0_layers: int = 5

    @property
    def upsample_scale(self) -> int:
        return int(np.prod(self.up_rates)) * self.hop

    @property
    def stage_channels(self) -> list[int]:
        return [self.base // (2 ** (i + 1)) for i in range(len(self.up_rates))]

    @property
    def down_rates(self) -> list[int]:
        """Cumulative source downsampling per stage (``[15, 3, 1]`` for rates 8/5/3)."""
        r = [1] + list(self.up_rates[::-1][:-1])
        return list(np.cumprod(r)[::-1].astype(int))


def snake(x, alpha):
    """``x + 1 / (alpha + 1e-9) * sin(x * alpha) ** 2`` over [B, C, T] with alpha [C] (``hift_lean.py:27-30``)."""
    a = alpha[None, :, None]
    return x + (1.0 / (a + 1e-9)) * torch.sin(x * a) ** 2


def get_padding(k, d):
    return (k * d - d) // 2


class _Conv:
    def __init__(self, w, b, stride=1, padding=0, dilation=1):
        self.w, self.b, self.stride, self.padding, self.dilation = w, b, stride, padding, dilation

    def __call__(self, x):
        return F.conv1d(x, self.w, self.b, self.stride, self.padding, self.dilation)


class _ConvT:
    def __init__(self, w, b, stride, padding):
        self.w, self.b, self.stride, self.padding = w, b, stride, padding

    def __call__(self, x):
        return F.conv_transpose1d(x, self.w, self.b, self.stride, self.padding)


class _ResBlock:
    """CosyVoice2 HiFT ResBlock: per dilation ``x = conv2(snake2(conv1(snake1(x)))) + x``."""

    def __init__(self, W, p, ch, k, dils):
        self.c1 = [_Conv(W[f"{p}.convs1.{j}.weight"], W[f"{p}.convs1.{j}.bias"], 1, get_padding(k, d), d) for j, d in enumerate(dils)]
        self.c2 = [_Conv(W[f"{p}.convs2.{j}.weight"], W[f"{p}.convs2.{j}.bias"], 1, get_padding(k, 1), 1) for j, _ in enumerate(dils)]
        self.a1 = [W[f"{p}.activations1.{j}.alpha"] for j in range(len(dils))]
        self.a2 = [W[f"{p}.activations2.{j}.alpha"] for j in range(len(dils))]

    def __call__(self, x):
        for c1, c2, a1, a2 in zip(self.c1, self.c2, self.a1, self.a2):
            x = c2(snake(c1(snake(x, a1)), a2)) + x
        return x


class _F0Predictor:
    def __init__(self, W, layers):
        self.convs = [_Conv(W[f"f0_predictor.condnet.{2 * i}.weight"], W[f"f0_predictor.condnet.{2 * i}.bias"], 1, 1) for i in range(layers)]
        self.w, self.b = W["f0_predictor.classifier.weight"], W["f0_predictor.classifier.bias"]

    def __call__(self, mel):
        x = mel
        for c in self.convs:
            x = F.elu(c(x))
        return torch.abs(F.linear(x.transpose(1, 2), self.w, self.b).squeeze(-1))


class _Upsample:
    def __init__(self, scale):
        self.scale_factor = float(scale)

    def __call__(self, x):
        return F.interpolate(x, scale_factor=self.scale_factor, mode="nearest")


class _SineGen:
    def __init__(self, d: HiFTDims):
        self.harmonic_num, self.sampling_rate, self.upsample_scale = d.harmonics, d.sr, d.upsample_scale
        self.sine_amp, self.noise_std, self.voiced_threshold = d.sine_amp, d.noise_std, d.voiced_threshold
        self.dim = d.harmonics + 1
        self.flag_for_pulse = False

    def _f02uv(self, f0):
        return (f0 > self.voiced_threshold).type(torch.float32)


class _Source:
    def __init__(self, W, d):
        self.l_sin_gen = _SineGen(d)
        self.w, self.b = W["m_source.l_linear.weight"], W["m_source.l_linear.bias"]
        self.l_tanh = torch.tanh

    def l_linear(self, x):
        return F.linear(x, self.w, self.b)


class HiFT:
    """The vocoder as plain fp32 ops over a weight dict (attribute names as ``HiFTGenerator``'s)."""

    def __init__(self, W: dict, d: HiFTDims = HiFTDims()):
        self.d = d
        self.f0_predictor = _F0Predictor(W, d.f0_layers)
        self.f0_upsamp = _Upsample(d.upsample_scale)
        self.m_source = _Source(W, d)
        self.conv_pre = _Conv(W["conv_pre.weight"], W["conv_pre.bias"], 1, 3)
        self.ups = [_ConvT(W[f"ups.{i}.weight"], W[f"ups.{i}.bias"], u, (k - u) // 2) for i, (u, k) in enumerate(zip(d.up_rates, d.up_kernels))]
        self.source_downs, self.source_resblocks = [], []
        for i, (u, k) in enumerate(zip(d.down_rates, d.src_res_kernels)):
            ch = d.stage_channels[i]
            if u == 1:
                self.source_downs.append(_Conv(W[f"source_downs.{i}.weight"], W[f"source_downs.{i}.bias"]))
            else:
                self.source_downs.append(_Conv(W[f"source_downs.{i}.weight"], W[f"source_downs.{i}.bias"], u, u // 2))
            self.source_resblocks.append(_ResBlock(W, f"source_resblocks.{i}", ch, k, d.res_dilations))
        self.resblocks = []
        for i, ch in enumerate(d.stage_channels):
            for j, k in enumerate(d.res_kernels):
                self.resblocks.append(_ResBlock(W, f"resblocks.{i * len(d.res_kernels) + j}", ch, k, d.res_dilations))
        self.conv_post = _Conv(W["conv_post.weight"], W["conv_post.bias"], 1, 3)
        self.num_upsamples, self.num_kernels = len(d.up_rates), len(d.res_kernels)
        self.lrelu_slope, self.audio_limit = d.lrelu_slope, d.audio_limit
        self.istft_params = {"n_fft": d.n_fft, "hop_len": d.hop}
        self.stft_window = torch.hann_window(d.n_fft, periodic=True, dtype=torch.float32)

    def reflection_pad(self, x):
        return F.pad(x, (1, 0), mode="reflect")

    def _stft(self, x):
        spec = torch.stft(x, self.d.n_fft, self.d.hop, self.d.n_fft, window=self.stft_window, return_complex=True)
        spec = torch.view_as_real(spec)
        return spec[..., 0], spec[..., 1]


def istft_overlap_add(spec: torch.Tensor, n_fft: int, hop: int, window: torch.Tensor) -> torch.Tensor:
    """``token2wav.py:128-138``: per-frame inverse real FFT times the window, overlap-add, division by the summed squared
    window, ``n_fft // 2`` trimmed at both ends (``torch.istft(center=True)``)."""
    frames = torch.fft.irfft(spec, n=n_fft, dim=1) * window[None, :, None]
    T = frames.shape[2]
    total = (T - 1) * hop + n_fft
    y = F.fold(frames, output_size=(1, total), kernel_size=(1, n_fft), stride=(1, hop))[:, 0, 0]
    env = F.fold((window ** 2)[None, :, None].expand(1, n_fft, T), output_size=(1, total), kernel_size=(1, n_fft), stride=(1, hop))[0, 0, 0]
    half = n_fft // 2
    return (y / env)[:, half:total - half]


def source(h: HiFT, mel: torch.Tensor, cache_source: torch.Tensor, rand_ini: torch.Tensor, noise: torch.Tensor, f0=None) -> torch.Tensor:
    """The NSF source ``s`` [B, 1, 480 T] (``token2wav.py:218-235``); ``f0`` [B, T] replaces the f0 predictor's."""
    gen = h.m_source.l_sin_gen
    f0 = h.f0_predictor(mel) if f0 is None else f0
    s = h.f0_upsamp(f0[:, None]).transpose(1, 2)  # [B, n, 1]
    fn = s * torch.arange(1, gen.harmonic_num + 2, dtype=torch.float32)[None, None, :]
    rad = (fn / gen.sampling_rate) % 1
    ri = rand_ini.clone()
    ri[:, 0] = 0
    rad[:, 0, :] = rad[:, 0, :] + ri
    rad = F.interpolate(rad.transpose(1, 2), scale_factor=1 / gen.upsample_scale, mode="linear").transpose(1, 2)
    phase = torch.cumsum(rad, dim=1) * 2 * np.pi
    phase = F.interpolate(phase.transpose(1, 2) * gen.upsample_scale, scale_factor=gen.upsample_scale, mode="linear").transpose(1, 2)
    sine = torch.sin(phase) * gen.sine_amp
    uv = gen._f02uv(fn[..., :1])
    sine = sine * uv + (uv * gen.noise_std + (1 - uv) * gen.sine_amp / 3) * noise
    out = h.m_source.l_tanh(h.m_source.l_linear(sine)).transpose(1, 2)
    if cache_source.shape[2] != 0:
        out[:, :, :cache_source.shape[2]] = cache_source
    return out


def decode(h: HiFT, x: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``_hift_decode`` (``token2wav.py:160-192``) in strict fp32."""
    sr, si = h._stft(s.squeeze(1))
    s_stft = torch.cat([sr, si], dim=1)
    x = h.conv_pre(x)
    for i in range(h.num_upsamples):
        x = F.leaky_relu(x, h.lrelu_slope)
        x = h.ups[i](x)
        if i == h.num_upsamples - 1:
            x = h.reflection_pad(x)
        x = x + h.source_resblocks[i](h.source_downs[i](s_stft))
        xs = None
        for j in range(h.num_kernels):
            r = h.resblocks[i * h.num_kernels + j](x)
            xs = r if xs is None else xs + r
        x = xs / h.num_kernels
    x = F.leaky_relu(x)
    x = h.conv_post(x)
    nf = h.istft_params["n_fft"]
    mag = torch.clip(torch.exp(x[:, :nf // 2 + 1, :]), max=1e2)
    ph = torch.sin(x[:, nf // 2 + 1:, :])
    y = istft_overlap_add(torch.complex(mag * torch.cos(ph), mag * torch.sin(ph)), nf, h.istft_params["hop_len"], h.stft_window)
    return torch.clamp(y, -h.audio_limit, h.audio_limit)


def forward_noise(h: HiFT, mel, cache_source, rand_ini, noise):
    """``hift_forward_noise``: (speech [B, 480 T], source [B, 1, 480 T])."""
    s = source(h, mel, cache_source, rand_ini, noise)
    return decode(h, mel, s), s


# --- noise and streaming glue ---------------------------------------------------------------------------------------

def chunk_noise_seed(noise_seed: int, chunk: int) -> int:
    """``token2wav.py:108-109``."""
    return (noise_seed * 1_000_003 + chunk) & ((1 << 63) - 1)


def hift_noise(dim: int, seeds: list[int], n_samples: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``token2wav.py:112-121``: row i draws ``rand(1, dim)`` then ``randn(1, dim, n)`` (transposed) from a generator
    seeded ``seeds[i]``."""
    gens = [torch.Generator().manual_seed(int(x)) for x in seeds]
    rand_ini = torch.cat([torch.rand(1, dim, generator=g) for g in gens])
    noise = torch.cat([torch.randn(1, dim, n_samples, generator=g) for g in gens]).transpose(1, 2)
    return rand_ini, noise


def fade_in_out(fade_in: torch.Tensor, fade_out: torch.Tensor, window: torch.Tensor) -> torch.Tensor:
    """``token2wav.py:81-85``."""
    n = int(window.shape[0] / 2)
    out = fade_in.clone()
    out[..., :n] = fade_in[..., :n] * window[:n] + fade_out[..., -n:] * window[n:]
    return out


def hamming_window() -> torch.Tensor:
    return torch.from_numpy(np.hamming(2 * SOURCE_CACHE))


@dataclass
class HiftState:
    """A stream's HiFT cache (``token2wav.py:319-332``): the last 8 mel frames, 3840 source and 3840 speech samples."""
    mel: torch.Tensor
    source: torch.Tensor
    speech: torch.Tensor
    chunks: int = 0
    noise_seed: int = 0


def new_hift_state(mel_dim: int = 80, noise_seed: int = 0) -> HiftState:
    return HiftState(torch.zeros(1, mel_dim, 0), torch.zeros(1, 1, 0), torch.zeros(1, 0), 0, noise_seed)


def vocode_chunk(h: HiFT, st: HiftState, mel: torch.Tensor, last: bool) -> np.ndarray:
    """One stream's window mel [1, 80, T] -> float32 samples, as ``Token2Wav._decode`` after the flow
    (``token2wav.py:319-332``); updates ``st``."""
    full = torch.cat([st.mel, mel], dim=2)
    rand_ini, noise = hift_noise(h.m_source.l_sin_gen.dim, [chunk_noise_seed(st.noise_seed, st.chunks)], full.shape[2] * h.d.upsample_scale)
    speech, src = forward_noise(h, full, st.source, rand_ini, noise)
    first = st.speech.shape[-1] == 0
    if not first:
        speech = fade_in_out(speech, st.speech, hamming_window())  # float64 window, as the reference's
    st.mel, st.source, st.speech = full[..., -MEL_CACHE:].clone(), src[:, :, -SOURCE_CACHE:].clone(), speech[:, -SOURCE_CACHE:].clone()
    if not last:
        speech = torch.cat([torch.zeros(1, SOURCE_CACHE), speech[:, :-SOURCE_CACHE]], dim=1) if first else speech[:, :-SOURCE_CACHE]
    st.chunks += 1
    return speech.float().numpy()[0]
