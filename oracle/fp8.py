"""MX fp8 restatement (test infrastructure: only tests and the bench's CPU leg use it).

No function of the reference covers this path's fp8 mode: the reference's fp8 convention (``engine/runtime/fp8.py:15-37``)
scales e4m3 weights per output channel by max|w| / 448, which ``quantize_weight`` follows.  Activations are quantized
in blocks of 32 consecutive values along K with one power-of-two (E8M0) scale per block: the smallest power of two
2^e with max|x| * 2^-e <= 448, so no value clips; values are rounded to nearest even e4m3 (torch's float8_e4m3fn cast,
a library routine).  Pinned by properties in tests/test_oracle_fp8.py (scale minimality, round-trip error within half
an e4m3 step, exactness on representable inputs) and, on the GPU, bit for bit against the device quantizer.
"""

from __future__ import annotations

import numpy as np
import torch

E4M3_MAX = 448.0


def block_exponent(amax: np.ndarray) -> np.ndarray:
    """Smallest e (int) with amax * 2^-e <= 448, clamped to [-126, 126]; -126 for zero blocks."""
    amax = np.asarray(amax, dtype=np.float32)
    bits = amax.view(np.uint32) & 0x7FFFFFFF
    E = (bits >> 23).astype(np.int64) - 127
    mant = bits & 0x7FFFFF
    e = E - 8 + (mant > 0x600000).astype(np.int64)
    e = np.where(bits < 0x00800000, -126, e)
    return np.clip(e, -126, 126)


def quantize_mx(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [M, K] (K % 32 == 0; bf16 or fp32 values) -> (q [M, K] uint8 e4m3 codes, s [M, K / 32] uint8 E8M0 = e + 127)."""
    xf = x.float().cpu()
    M, K = xf.shape
    blocks = xf.reshape(M, K // 32, 32)
    e = torch.from_numpy(block_exponent(blocks.abs().amax(dim=2).numpy()))
    scaled = blocks * torch.pow(2.0, -e.double()).float()[:, :, None]
    q = scaled.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8).reshape(M, K)
    return q, (e + 127).to(torch.uint8)


def dequantize_mx(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    M, K = q.shape
    v = q.cpu().view(torch.float8_e4m3fn).float().reshape(M, K // 32, 32)
    return (v * torch.pow(2.0, s.cpu().double() - 127).float()[:, :, None]).reshape(M, K)


def quantize_weight(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """w [N, K] -> (e4m3 codes [N, K] uint8, per-output-channel fp32 scale [N] = max|w_n| / 448)."""
    wf = w.float().cpu()
    sc = (wf.abs().amax(dim=1) / E4M3_MAX).clamp_min(1e-30)
    q = (wf / sc[:, None]).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
    return q, sc


def dequantize_weight(q: torch.Tensor, sc: torch.Tensor) -> torch.Tensor:
    return q.cpu().view(torch.float8_e4m3fn).float() * sc.cpu()[:, None]
