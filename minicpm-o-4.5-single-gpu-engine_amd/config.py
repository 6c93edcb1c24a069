"""Model dimensions of the Token2Wav hot path (flow encoder, DiT estimator, HiFT vocoder).

The reference reads every shape from ``stepaudio2`` modules at runtime (``engine/runtime/dit_fast.py:107-145``,
``engine/models/token2wav.py:250-261``); those modules are not part of the reference repository, so the shapes of the
synthetic workloads are fixed here: DiT 22 blocks, hidden 1024, 16 heads of 64, FFN 2x, mel 80, ``in_proj`` 4 x 80 ->
hidden; HiFT CosyVoice2-style at 24 kHz (base 512 channels, upsampling 8 x 5 x 3, ISTFT 16 / 4); the flow encoder
CosyVoice2's ``UpsampleConformerEncoder`` (width 512, 8 heads, FFN 2048, 6 + 4 layers, 2x upsampling, vocabulary 6561).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class DiTConfig:
    mel: int = 80
    hidden: int = 1024
    depth: int = 22
    heads: int = 16
    head_dim: int = 64
    ffn: int = 2048
    freq: int = 256          # sinusoid size of the timestep embedder
    eps_block: float = 1e-6  # norm1/2/3 (no affine)
    eps_qk: float = 1e-6     # per-head q/k LayerNorm (affine)
    eps_conv: float = 1e-5   # the conv block's LayerNorm (affine)
    eps_final: float = 1e-6
    cfg_rate: float = 0.7    # CausalConditionalCFM.inference_cfg_rate
    steps: int = 10
    noise_frames: int = 50 * 300  # the flow's fixed noise buffer ``rand_noise`` [1, mel, frames]
    rope_theta: float = 0.0  # > 0: rotary embedding of q and k at stream positions (not in the reference; 0 = off)

    @property
    def in_dim(self) -> int:
        return 4 * self.mel


@dataclass(frozen=True)
class HiFTConfig:
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
    sr: int = 24000
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
        r = [1] + list(self.up_rates[::-1][:-1])
        return [int(v) for v in np.cumprod(r)[::-1]]


@dataclass(frozen=True)
class FlowConfig:
    vocab: int = 6561
    dim: int = 512
    heads: int = 8
    ffn: int = 2048
    depth1: int = 6          # conformer layers before the upsampling
    depth2: int = 4          # after it
    look: int = 3            # pre-lookahead tokens
    stride: int = 2          # token frames -> mel frames
    mel: int = 80
    spk: int = 192           # speaker embedding size (before the affine layer)
    eps_layer: float = 1e-12  # norm_mha / norm_ff
    eps_embed: float = 1e-5   # the input layers' LayerNorm
    eps_after: float = 1e-5   # after_norm
    rmax: int = 4096         # relative positions +-(rmax - 1) are tabulated: keys per stream and stack at most rmax

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads

    @property
    def cnn_frames(self) -> int:
        return 2 + 2 * self.stride


SILENCE_TOKEN = 4218
SAMPLE_RATE = 24000
MEL_CACHE = 8
SOURCE_CACHE = MEL_CACHE * 480
TRIM_SUFFIX = 100
