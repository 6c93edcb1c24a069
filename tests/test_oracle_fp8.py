"""The MX fp8 restatement (oracle/fp8.py) pinned by what the format fixes: known block exponents, scale minimality, the
half-step round-trip bound of e4m3, exactness on representable values, and the e4m3 code table itself."""

import numpy as np
import torch

from oracle import fp8 as of


def test_block_exponent_known_values():
    amax = np.array([448.0, 449.0, 1.0, 1.75, np.nextafter(np.float32(1.75), np.float32(2)), 0.0, 3.0e-3, 896.0, 897.0], dtype=np.float32)
    e = of.block_exponent(amax)
    # 448 fits at 2^0; 449 needs 2^1; 1.0 * 2^8 = 256 fits, 2^9 would be 512; 1.75 * 2^8 = 448 fits exactly
    assert list(e[:5]) == [0, 1, -8, -8, -7]
    assert e[5] == -126
    assert list(e[7:]) == [1, 2]


def test_block_exponent_is_minimal():
    rng = np.random.default_rng(0)
    amax = (10.0 ** rng.uniform(-20, 20, 20000)).astype(np.float32)
    e = of.block_exponent(amax).astype(np.float64)
    a = amax.astype(np.float64)
    assert np.all(a * 2.0 ** -e <= 448.0)
    assert np.all(a * 2.0 ** -(e - 1) > 448.0)


def test_roundtrip_within_half_step():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 256, generator=g) * torch.exp(torch.randn(64, 8, generator=g) * 3).repeat_interleave(32, dim=1)
    q, s = of.quantize_mx(x)
    y = of.dequantize_mx(q, s)
    scale = torch.pow(2.0, s.double() - 127).float().repeat_interleave(32, dim=1)
    # e4m3 keeps 3 mantissa bits: half a step is |x| 2^-4 for normals, 2^-10 scale in the subnormal range
    bound = torch.maximum(x.abs() * 2.0 ** -4, 2.0 ** -10 * scale) * (1 + 1e-6)
    assert torch.all((y - x).abs() <= bound)
    # the largest magnitude of every block lands in the top binade of e4m3
    amax = x.abs().reshape(64, 8, 32).amax(2) / torch.pow(2.0, s.double() - 127).float()
    assert torch.all((amax > 224) & (amax <= 448))


def test_exact_on_representable_values():
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]  # no NaN codes
    vals = codes.view(torch.float8_e4m3fn).float()
    x = vals[torch.randperm(len(vals), generator=torch.Generator().manual_seed(2))][:224].reshape(7, 32)
    x[:, 0] = 448.0  # every block's maximum at 448: scale exponent 0
    q, s = of.quantize_mx(x)
    assert torch.all(s == 127)
    assert torch.equal(of.dequantize_mx(q, s), x)


def test_e4m3_code_table():
    # OCP e4m3fn: bias 7, 3 mantissa bits, max 448 (0x7e), subnormal step 2^-9, 0x7f NaN
    v = torch.tensor([0x7E, 0x08, 0x01, 0x38, 0xB8, 0x40], dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    assert v.tolist() == [448.0, 2.0 ** -6, 2.0 ** -9, 1.0, -1.0, 2.0]


def test_weight_quantization_per_channel():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(16, 96, generator=g) * torch.rand(16, 1, generator=g)
    q, sc = of.quantize_weight(w)
    assert torch.allclose(sc, w.abs().amax(1) / 448.0)
    back = of.dequantize_weight(q, sc)
    assert torch.all((back - w).abs() <= w.abs().amax(1, keepdim=True) * 2.0 ** -4 + 1e-12)
