"""Pins of the DiT oracle's composition (CPU): the timestep embedder, the adaLN chunk positions, the block's branch order,
the final layer and the input packing.

Each expected value is computed here in float64 numpy from a special case that collapses the block to plain linear
algebra, with the chunk names in the order the reference unpacks them (``engine/runtime/token2wav_batch.py:104``:
shift/scale/gate of msa, then mlp, then conv) and the branch order of ``_block_chunk`` (``:105-110``: attention on
norm1, conv block on norm3, MLP on norm2).  With one frame and empty caches, attention's softmax has a single key, so
the branch is ``proj(to_v(a))``; the causal convs see two zero cache frames, so each is its last tap.  The adaLN weights
are zeroed and their biases set, so the nine chunks are known vectors.  Permuting chunks, swapping branches or feeding a
branch the wrong residual changes the result by O(1).
"""

import math

import numpy as np
import pytest
import torch

from oracle import dit as od

import t2w_amd  # noqa: F401
from t2w_amd.config import DiTConfig
from t2w_amd.weights import init_dit

CFG = DiTConfig(hidden=128, depth=1, heads=2, ffn=256, steps=4)
CHUNKS = ("shift_msa", "scale_msa", "gate_msa", "shift_mlp", "scale_mlp", "gate_mlp", "shift_conv", "scale_conv", "gate_conv")


def _np(t):
    return t.detach().double().numpy()


def _ln(x, eps, w=None, b=None):
    y = (x - x.mean(-1, keepdims=True)) / np.sqrt(x.var(-1, keepdims=True) + eps)
    return y * w + b if w is not None else y


def _gelu_tanh(x):
    return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def _mish(x):
    return x * np.tanh(np.log1p(np.exp(x)))


def _lin(W, name, x):
    return x @ _np(W[name + ".weight"]).T + _np(W[name + ".bias"])


@pytest.fixture()
def W():
    return init_dit(CFG, seed=21)


def _set_mods(W, b, chunks: dict) -> None:
    H = CFG.hidden
    W[f"blocks.{b}.adaLN_modulation.1.weight"] = torch.zeros(9 * H, H)
    W[f"blocks.{b}.adaLN_modulation.1.bias"] = torch.cat([chunks[n] for n in CHUNKS]).float()


def _closed_form_block(W, h, c):
    """One frame, empty caches: the block as the reference composes it, in float64."""
    p = "blocks.0."
    a = _ln(h, 1e-6) * (1 + c["scale_msa"]) + c["shift_msa"]
    att = _lin(W, p + "attn.proj", _lin(W, p + "attn.to_v", a))
    h1 = h + c["gate_msa"] * att
    x = _ln(h1, 1e-6) * (1 + c["scale_conv"]) + c["shift_conv"]
    y = x @ _np(W[p + "conv.block.1.weight"])[:, :, 2].T + _np(W[p + "conv.block.1.bias"])
    y = _mish(_ln(y, 1e-5, _np(W[p + "conv.block.3.weight"]), _np(W[p + "conv.block.3.bias"])))
    y = y @ _np(W[p + "conv.block.6.weight"])[:, :, 2].T + _np(W[p + "conv.block.6.bias"])
    h2 = h1 + c["gate_conv"] * y
    m = _ln(h2, 1e-6) * (1 + c["scale_mlp"]) + c["shift_mlp"]
    return h2 + c["gate_mlp"] * _lin(W, p + "mlp.fc2", _gelu_tanh(_lin(W, p + "mlp.fc1", m)))


def _oracle_block(W, h):
    d = od.dims_of(W, steps=CFG.steps)
    H = d.hidden
    temb = torch.randn(1, H)  # irrelevant: the adaLN weights are zero
    out, _, _ = od.block_chunk(W, d, 0, torch.from_numpy(h).float()[None, None], temb, torch.zeros(1, 2 * H, 2),
                               torch.zeros(1, d.heads, 0, 2 * d.head_dim), torch.ones(1, 1, 1, dtype=torch.bool), torch.tensor([1]))
    return _np(out[0, 0])


def _random_chunks(seed, open_gates=("gate_msa", "gate_mlp", "gate_conv")):
    g = torch.Generator().manual_seed(seed)
    c = {n: torch.randn(CFG.hidden, generator=g) * 0.5 for n in CHUNKS}
    for n in ("gate_msa", "gate_mlp", "gate_conv"):
        c[n] = c[n] + 1.0 if n in open_gates else torch.zeros(CFG.hidden)
    return c


def test_adaln_chunks_and_branch_order_closed_form(W):
    """All nine chunks distinct and all gates open: the oracle's block equals the closed form to fp32 precision, and a
    swap of any two chunk positions of the same kind (a plausible mistake) moves the result far outside it."""
    c = _random_chunks(1)
    _set_mods(W, 0, c)
    h = np.random.default_rng(2).standard_normal(CFG.hidden) * 2
    ref = _closed_form_block(W, h, {k: _np(v) for k, v in c.items()})
    got = _oracle_block(W, h)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)
    for a, b in (("shift_msa", "shift_mlp"), ("scale_mlp", "scale_conv"), ("gate_msa", "gate_conv"), ("shift_conv", "shift_mlp")):
        sw = dict(c)
        sw[a], sw[b] = c[b], c[a]
        wrong = _closed_form_block(W, h, {k: _np(v) for k, v in sw.items()})
        assert np.abs(wrong - got).max() > 1e-2, (a, b)


@pytest.mark.parametrize("gates", [("gate_msa",), ("gate_conv",), ("gate_mlp",), ("gate_msa", "gate_conv"), ("gate_conv", "gate_mlp"),
                                   ("gate_msa", "gate_mlp")])
def test_one_branch_at_a_time(W, gates):
    """Closed gates remove their branch: each branch alone reads the block input, and with two open the later branch
    reads the earlier one's residual (attention -> conv -> MLP)."""
    c = _random_chunks(3, gates)
    _set_mods(W, 0, c)
    h = np.random.default_rng(4).standard_normal(CFG.hidden)
    np.testing.assert_allclose(_oracle_block(W, h), _closed_form_block(W, h, {k: _np(v) for k, v in c.items()}), rtol=2e-5, atol=2e-5)


def test_final_layer_shift_then_scale(W):
    """Final layer: adaLN chunks (shift, scale), no-affine LayerNorm, then Linear H -> mel (the one block's gates are
    closed, so it passes the in_proj output through)."""
    H = CFG.hidden
    g = torch.Generator().manual_seed(5)
    _set_mods(W, 0, _random_chunks(6, open_gates=()))
    sh, sc = torch.randn(H, generator=g), torch.randn(H, generator=g)
    W["final_layer.adaLN_modulation.1.weight"] = torch.zeros(2 * H, H)
    W["final_layer.adaLN_modulation.1.bias"] = torch.cat([sh, sc])
    d = od.dims_of(W, steps=CFG.steps)
    x, mu, cond = (torch.randn(1, 80, 1, generator=g) for _ in range(3))
    spk = torch.randn(1, 80, generator=g)
    got, _, _ = od.estimator_chunk(W, d, x, mu, torch.zeros(1, H), spk, cond, torch.zeros(1, 1, 2 * H, 2), torch.zeros(1, 1, d.heads, 0, 2 * d.head_dim),
                                   torch.ones(1, 1, 1, dtype=torch.bool), torch.tensor([1]))
    inp = np.concatenate([_np(x[0, :, 0]), _np(mu[0, :, 0]), _np(spk[0]), _np(cond[0, :, 0])])
    h = _lin(W, "in_proj", inp)
    ref = _lin(W, "final_layer.linear", _ln(h, 1e-6) * (1 + _np(sc)) + _np(sh))
    np.testing.assert_allclose(_np(got[0, :, 0]), ref, rtol=2e-5, atol=2e-5)


def test_input_packing_order():
    """``[x | mu | spk | cond]`` per frame, the speaker embedding repeated over frames."""
    B, T = 2, 3
    x, mu, cond = (torch.full((B, 80, T), float(v)) for v in (1, 2, 4))
    spk = torch.arange(B, dtype=torch.float32)[:, None].expand(B, 80) + 10
    p = od.pack_inputs(x, mu, spk, cond)
    assert p.shape == (B, T, 320)
    for b in range(B):
        for t in range(T):
            row = p[b, t]
            assert torch.all(row[:80] == 1) and torch.all(row[80:160] == 2) and torch.all(row[240:] == 4)
            assert torch.all(row[160:240] == 10 + b)


def test_timestep_sinusoid_closed_forms():
    """``[cos(1000 t f_k) | sin(1000 t f_k)]``, f_k = 10000^(-k/128): t = 0 gives ones then zeros; t = pi / 2000 puts the
    first frequency at a quarter turn; the last frequency is 10000^(-127/128), half a turn at t = pi / (1000 f_127)."""
    e0 = od.timestep_sinusoid(torch.zeros(1), 256)[0]
    assert torch.all(e0[:128] == 1) and torch.all(e0[128:] == 0)
    f = od.freq_table(256)
    assert float(f[0]) == 1.0
    assert abs(float(f[127]) - 10000 ** (-127 / 128)) < 1e-9
    e = od.timestep_sinusoid(torch.tensor([math.pi / 2000]), 256)[0]
    assert abs(float(e[0])) < 1e-6 and abs(float(e[128]) - 1) < 1e-6
    assert abs(float(e[1]) - math.cos(math.pi / 2 * 10000 ** (-1 / 128))) < 1e-6
    t_half = math.pi / (1000 * 10000 ** (-127 / 128))
    e = od.timestep_sinusoid(torch.tensor([t_half]), 256)[0]
    assert abs(float(e[127]) + 1) < 1e-4 and abs(float(e[255])) < 1e-3


def test_t_embedder_silu_between_linears():
    """Linear -> SiLU -> Linear: identity linears turn t = 0 into SiLU([1 .. 1 | 0 .. 0]); adaLN = SiLU then Linear."""
    H = 256
    W = init_dit(DiTConfig(hidden=H, depth=1, heads=4, ffn=512, steps=4), seed=0)
    W["t_embedder.mlp.0.weight"], W["t_embedder.mlp.0.bias"] = torch.eye(H), torch.zeros(H)
    W["t_embedder.mlp.2.weight"], W["t_embedder.mlp.2.bias"] = torch.eye(H) * 2, torch.ones(H)
    te = od.t_embed(W, torch.zeros(1))[0]
    s1 = 1 / (1 + math.exp(-1))
    np.testing.assert_allclose(_np(te[:128]), 2 * s1 + 1, rtol=1e-6)
    np.testing.assert_allclose(_np(te[128:]), 1.0, rtol=1e-6)
    W["blocks.0.adaLN_modulation.1.weight"] = torch.zeros(9 * H, H)
    W["blocks.0.adaLN_modulation.1.weight"][:H] = torch.eye(H)
    W["blocks.0.adaLN_modulation.1.bias"] = torch.zeros(9 * H)
    temb = torch.linspace(-3, 3, H)[None]
    m = od.block_mods(W, 0, temb)
    np.testing.assert_allclose(_np(m[0][0]), _np(temb[0]) / (1 + np.exp(-_np(temb[0]))), rtol=1e-6, atol=1e-7)
    assert all(float(x.abs().max()) == 0 for x in m[1:])
