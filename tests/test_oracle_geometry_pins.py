"""Closed-form pins of the oracle functions whose definitions live inside ``stepaudio2`` (CosyVoice2's HiFT and
``UpsampleConformerEncoder``), which the reference repository only calls: the HiFT ResBlock, the f0 predictor, the
up/down-sampling geometry of the decoder and the flow encoder's conformer layer, linear input layer and layer order.

Each test builds weights that make the function reduce to a closed form (delta kernels, identity maps, zeroed branches),
evaluates that closed form in float64 numpy with explicit index arithmetic (no torch conv), and compares.  The special
cases are chosen so that a plausible mistake fails one of them: a dilation on the wrong conv, a padding off by a
sample, Snake and conv in the other order, a post-norm layer, ReLU for ELU / SiLU, the FFN before the attention, the
sqrt(dim) scale before the LayerNorm, a layer on the wrong side of the upsampling.
"""

import math

import numpy as np
import pytest
import torch

from oracle import flow as of
from oracle import hift as oh

import t2w_amd  # noqa: F401
from t2w_amd.config import FlowConfig, HiFTConfig
from t2w_amd.weights import init_flow, init_hift

RNG = np.random.default_rng(11)


# --- numpy closed-form helpers ------------------------------------------------------------------------------------

def np_snake(x, a):
    """x [C, T], a [C]."""
    a = a[:, None]
    return x + (1.0 / (a + 1e-9)) * np.sin(x * a) ** 2


def np_shift(x, s):
    """y[:, t] = x[:, t + s], zero outside [0, T)."""
    T = x.shape[1]
    y = np.zeros_like(x)
    for t in range(T):
        if 0 <= t + s < T:
            y[:, t] = x[:, t + s]
    return y


def np_elu(x):
    return np.where(x > 0, x, np.expm1(np.minimum(x, 0)))


def np_silu(x):
    return x / (1.0 + np.exp(-x))


def np_ln(x, g, b, eps):
    """Row LayerNorm over the last axis."""
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def delta(co, ci, k, tap, gain=1.0):
    """Conv weight [co, ci, k]: channel c -> c (c < min(co, ci)) through tap ``tap`` only."""
    w = torch.zeros(co, ci, k, dtype=torch.float32)
    for c in range(min(co, ci)):
        w[c, c, tap] = gain
    return w


def t64(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))


# --- HiFT ---------------------------------------------------------------------------------------------------------

SMALL = HiFTConfig(base=16, f0_channels=8, mel=6)
SMALL_DIMS = oh.HiFTDims(base=16, f0_channels=8, mel=6)


def _resblock_weights(ch, k, dils, c1, c2, b1=None, b2=None):
    W, p = {}, "rb"
    for j, _ in enumerate(dils):
        W[f"{p}.convs1.{j}.weight"] = c1(j)
        W[f"{p}.convs1.{j}.bias"] = torch.zeros(ch) if b1 is None else t64(b1[j])
        W[f"{p}.convs2.{j}.weight"] = c2(j)
        W[f"{p}.convs2.{j}.bias"] = torch.zeros(ch) if b2 is None else t64(b2[j])
        W[f"{p}.activations1.{j}.alpha"] = t64(RNG.uniform(0.5, 1.5, ch))
        W[f"{p}.activations2.{j}.alpha"] = t64(RNG.uniform(0.5, 1.5, ch))
    return W, p


def _alphas(W, p, dils):
    a1 = [W[f"{p}.activations1.{j}.alpha"].double().numpy() for j in range(len(dils))]
    a2 = [W[f"{p}.activations2.{j}.alpha"].double().numpy() for j in range(len(dils))]
    return a1, a2


def test_resblock_order_gains_and_biases():
    """Centre-tap convs with gains g1, g2 and biases: per dilation x <- g2 snake(g1 snake(x, a1) + b1, a2) + b2 + x.
    Conv before Snake, a missing residual or the Snakes swapped all change this."""
    ch, k, dils, T = 4, 7, (1, 3, 5), 40
    g1, g2 = 0.7, -1.3
    b1, b2 = RNG.normal(0, 0.3, (3, ch)), RNG.normal(0, 0.3, (3, ch))
    W, p = _resblock_weights(ch, k, dils, lambda j: delta(ch, ch, k, k // 2, g1), lambda j: delta(ch, ch, k, k // 2, g2), b1, b2)
    x = RNG.normal(0, 1, (ch, T))
    got = oh._ResBlock(W, p, ch, k, dils)(t64(x)[None])[0].double().numpy()
    a1, a2 = _alphas(W, p, dils)
    ref = x.copy()
    for j in range(len(dils)):
        ref = g2 * np_snake(g1 * np_snake(ref, a1[j]) + b1[j][:, None], a2[j]) + b2[j][:, None] + ref
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("tap", [0, 2, 6])
def test_resblock_conv1_is_dilated(tap):
    """conv1 of dilation step j is dilated by d_j with 'same' padding: a delta at tap i reads x[t + (i - 3) d_j]."""
    ch, k, dils, T = 3, 7, (1, 3, 5), 50
    W, p = _resblock_weights(ch, k, dils, lambda j: delta(ch, ch, k, tap), lambda j: delta(ch, ch, k, k // 2))
    x = RNG.normal(0, 1, (ch, T))
    got = oh._ResBlock(W, p, ch, k, dils)(t64(x)[None])[0].double().numpy()
    a1, a2 = _alphas(W, p, dils)
    ref = x.copy()
    for j, d in enumerate(dils):
        ref = np_snake(np_shift(np_snake(ref, a1[j]), (tap - k // 2) * d), a2[j]) + ref  # snake(0) = 0 keeps the zero padding
    assert got.shape == (ch, T)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("tap", [0, 5])
def test_resblock_conv2_is_not_dilated(tap):
    """conv2 has dilation 1 in every step (padding (k - 1) / 2): a delta at tap i reads x[t + i - (k - 1) / 2]."""
    ch, k, dils, T = 3, 7, (1, 3, 5), 50
    W, p = _resblock_weights(ch, k, dils, lambda j: delta(ch, ch, k, k // 2), lambda j: delta(ch, ch, k, tap))
    x = RNG.normal(0, 1, (ch, T))
    got = oh._ResBlock(W, p, ch, k, dils)(t64(x)[None])[0].double().numpy()
    a1, a2 = _alphas(W, p, dils)
    ref = x.copy()
    for j in range(len(dils)):
        ref = np_shift(np_snake(np_snake(ref, a1[j]), a2[j]), tap - k // 2) + ref
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_f0_predictor_elu_linear_abs():
    """Five kernel-3 convs, each followed by ELU, then Linear(C -> 1) over channels and abs.  The first conv carries a
    delta at tap 0 (reads frame t - 1: padding 1), the others centre deltas; the classifier mixes two channels with a
    bias so that its output takes both signs."""
    W = init_hift(SMALL, seed=1)
    C, M, T = SMALL.f0_channels, SMALL.mel, 30
    for i in range(SMALL.f0_layers):
        W[f"f0_predictor.condnet.{2 * i}.weight"] = delta(C, M if i == 0 else C, 3, 0 if i == 0 else 1)
        W[f"f0_predictor.condnet.{2 * i}.bias"] = torch.zeros(C)
    w = np.zeros((1, C))
    w[0, 0], w[0, 1] = -2.0, 0.5
    W["f0_predictor.classifier.weight"] = t64(w)
    W["f0_predictor.classifier.bias"] = torch.tensor([0.3])
    mel = RNG.normal(0, 1.5, (M, T))
    got = oh.HiFT(W, SMALL_DIMS).f0_predictor(t64(mel)[None])[0].double().numpy()
    h = np.zeros((C, T))
    h[:M] = np_shift(mel, -1)
    for _ in range(SMALL.f0_layers):
        h = np_elu(h)
    lin = w[0] @ h + 0.3
    assert (lin > 0).any() and (lin < 0).any()
    np.testing.assert_allclose(got, np.abs(lin), rtol=1e-5, atol=1e-6)


def _hift_with(**repl):
    W = init_hift(SMALL, seed=2)
    W.update(repl)
    return oh.HiFT(W, SMALL_DIMS)


@pytest.mark.parametrize("stage", [0, 1, 2])
def test_ups_polyphase_placement(stage):
    """``ups[i]`` is a transposed conv with stride u and padding (k - u) / 2: input frame t through tap j lands on
    output sample u t + j - (k - u) / 2, and T frames give u T samples."""
    u, k = SMALL.up_rates[stage], SMALL.up_kernels[stage]
    cin = ([SMALL.base] + SMALL.stage_channels)[stage]
    cout = SMALL.stage_channels[stage]
    T = 9
    w = torch.zeros(cin, cout, k)
    taps = RNG.normal(0, 1, k)
    for c in range(min(cin, cout)):
        w[c, c] = t64(taps)
    h = _hift_with(**{f"ups.{stage}.weight": w, f"ups.{stage}.bias": torch.zeros(cout)})
    x = RNG.normal(0, 1, (cin, T))
    got = h.ups[stage](t64(x)[None])[0].double().numpy()
    pad = (k - u) // 2
    ref = np.zeros((cout, u * T))
    for t in range(T):
        for j in range(k):
            o = u * t + j - pad
            if 0 <= o < u * T:
                ref[: min(cin, cout), o] += taps[j] * x[: min(cin, cout), t]
    assert got.shape == ref.shape
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("stage", [0, 1, 2])
def test_source_downs_geometry(stage):
    """``source_downs[i]``: kernel 2u, stride u, padding u / 2 (u = 15, 3) and a 1x1 conv for u = 1.  Output frame t
    through tap j reads STFT frame u t + j - u // 2; 120 T + 1 STFT frames (the source of T mel frames) give 8 T,
    40 T and 120 T + 1 frames, the lengths of the upsampled stages they are added to."""
    u = SMALL.down_rates[stage]
    kk = 1 if u == 1 else 2 * u
    nsrc, ch = SMALL.n_fft + 2, SMALL.stage_channels[stage]
    T = 4
    L = 120 * T + 1
    taps = RNG.normal(0, 1, kk)
    w = torch.zeros(ch, nsrc, kk)
    for c in range(min(ch, nsrc)):
        w[c, c] = t64(taps)
    h = _hift_with(**{f"source_downs.{stage}.weight": w, f"source_downs.{stage}.bias": torch.zeros(ch)})
    x = RNG.normal(0, 1, (nsrc, L))
    got = h.source_downs[stage](t64(x)[None])[0].double().numpy()
    want_len = [8 * T, 40 * T, 120 * T + 1][stage]
    assert got.shape == (ch, want_len)
    ref = np.zeros((ch, want_len))
    for t in range(want_len):
        for j in range(kk):
            s = u * t + j - u // 2
            if 0 <= s < L:
                ref[: min(ch, nsrc), t] += taps[j] * x[: min(ch, nsrc), s]
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("name", ["conv_pre", "conv_post"])
@pytest.mark.parametrize("tap", [0, 3, 6])
def test_conv_pre_post_padding(name, tap):
    """``conv_pre`` and ``conv_post`` are kernel-7 convs with padding 3: a delta at tap j reads frame t + j - 3."""
    cin = SMALL.mel if name == "conv_pre" else SMALL.stage_channels[-1]
    cout = SMALL.base if name == "conv_pre" else SMALL.n_fft + 2
    h = _hift_with(**{f"{name}.weight": delta(cout, cin, 7, tap), f"{name}.bias": torch.zeros(cout)})
    x = RNG.normal(0, 1, (cin, 25))
    got = getattr(h, name)(t64(x)[None])[0].double().numpy()
    ref = np.zeros((cout, 25))
    ref[: min(cin, cout)] = np_shift(x[: min(cin, cout)], tap - 3)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_reflection_pad_one_sample_left():
    h = _hift_with()
    x = torch.arange(12, dtype=torch.float32).view(1, 2, 6)
    y = h.reflection_pad(x)
    assert y.shape == (1, 2, 7)
    assert torch.equal(y[..., 0], x[..., 1]) and torch.equal(y[..., 1:], x)


@pytest.mark.parametrize("T", [1, 3, 8])
def test_decoder_lengths(T):
    """Every stage's two branches meet at equal lengths and T mel frames decode to 480 T samples."""
    h = _hift_with()
    mel = t64(RNG.normal(-5, 2, (1, SMALL.mel, T)))
    s = torch.zeros(1, 1, 480 * T)
    assert oh.decode(h, mel, s).shape == (1, 480 * T)


# --- flow encoder -------------------------------------------------------------------------------------------------

FCFG = FlowConfig(vocab=50, dim=16, heads=2, ffn=32, depth1=2, depth2=3, mel=8, spk=4)


@pytest.fixture()
def fw():
    return init_flow(FCFG, seed=5)


def _np(W, k):
    return W[k].double().numpy()


def _set_ffn(W, p, C, F, s):
    """FFN of layer p reduced to s * SiLU(.) on the channels: w_1 = [I; 0], w_2 = [s I, 0], no biases."""
    w1 = torch.zeros(F, C)
    w1[:C] = torch.eye(C)
    w2 = torch.zeros(C, F)
    w2[:, :C] = s * torch.eye(C)
    W[p + ".feed_forward.w_1.weight"], W[p + ".feed_forward.w_1.bias"] = w1, torch.zeros(F)
    W[p + ".feed_forward.w_2.weight"], W[p + ".feed_forward.w_2.bias"] = w2, torch.zeros(C)


def test_linear_embed_norm_then_scale(fw):
    """Linear (a I, constant bias) -> LayerNorm (affine) -> x sqrt(dim): the LayerNorm removes a and the bias, the
    output is (LN(x) g + b) sqrt(C) with LN(a x + c) = a (x - mean) / sqrt(a^2 var + eps).  The scale applied before
    the norm, or no norm, gives rows of another size."""
    d = of.enc_dims_of(fw)
    C, a, c = d.dim, 2.5, 0.7
    fw["encoder.embed.out.0.weight"] = a * torch.eye(C)
    fw["encoder.embed.out.0.bias"] = torch.full((C,), c)
    x = RNG.normal(0, 1, (5, C))
    got = of.linear_embed(fw, "encoder.embed", t64(x)[None], d)[0].double().numpy()
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    ln = a * (x - mu) / np.sqrt(a * a * var + d.eps_embed)
    ref = (ln * _np(fw, "encoder.embed.out.1.weight") + _np(fw, "encoder.embed.out.1.bias")) * math.sqrt(C)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_conformer_layer_prenorm_attention_then_ffn(fw):
    """One frame, no cache: the attention's softmax over its single key is 1, so with to_v = linear_out = I (no biases)
    the attention branch is LN_mha(x).  With the FFN reduced to s SiLU, the layer is
    x1 = x + LN_mha(x); out = x1 + s SiLU(LN_ff(x1)).  Post-norm, the FFN first or ReLU/GELU instead of SiLU fail."""
    d = of.enc_dims_of(fw)
    C, p, s = d.dim, "encoder.encoders.0", 1.7
    fw[p + ".self_attn.linear_v.weight"], fw[p + ".self_attn.linear_v.bias"] = torch.eye(C), torch.zeros(C)
    fw[p + ".self_attn.linear_out.weight"], fw[p + ".self_attn.linear_out.bias"] = torch.eye(C), torch.zeros(C)
    _set_ffn(fw, p, C, d.ffn, s)
    x = RNG.normal(0, 1, (1, C))
    mask = torch.ones(1, 1, 1, dtype=torch.bool)
    cache = torch.zeros(1, d.heads, 0, 2 * d.dk)
    got, _ = of.conformer_layer(fw, p, t64(x)[None], mask, of.rel_pos_table(1, C), cache, d)
    got = got[0].double().numpy()
    x1 = x + np_ln(x, _np(fw, p + ".norm_mha.weight"), _np(fw, p + ".norm_mha.bias"), d.eps_layer)
    ref = x1 + s * np_silu(np_ln(x1, _np(fw, p + ".norm_ff.weight"), _np(fw, p + ".norm_ff.bias"), d.eps_layer))
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_conformer_layer_zero_branches_is_identity(fw):
    """Zero linear_out and w_2 (weights and biases): the layer returns its input exactly (residuals around both)."""
    d = of.enc_dims_of(fw)
    C, p = d.dim, "encoder.up_encoders.1"
    fw[p + ".self_attn.linear_out.weight"], fw[p + ".self_attn.linear_out.bias"] = torch.zeros(C, C), torch.zeros(C)
    fw[p + ".feed_forward.w_2.weight"], fw[p + ".feed_forward.w_2.bias"] = torch.zeros(C, d.ffn), torch.zeros(C)
    x = t64(RNG.normal(0, 1, (1, 4, C)))
    out, _ = of.conformer_layer(fw, p, x, torch.ones(1, 4, 4, dtype=torch.bool), of.rel_pos_table(4, C), torch.zeros(1, d.heads, 0, 2 * d.dk), d)
    assert torch.equal(out, x)


def test_encoder_core_order(fw):
    """``_encoder_core`` (``token2wav_batch.py:42-79``) with every stage reduced to a distinct closed form:
    embed (LN affine, x sqrt C) -> pre-lookahead (zero convs: + conv2's bias) -> d1 layers (attention zeroed, FFN
    s_i SiLU) -> nearest x2 -> upsampling conv (taps 3, 4 = half each: the mean of the previous and the current
    upsampled frame, the cached zeros before the first) + bias -> up_embed (LN affine, x sqrt C) -> d2 layers ->
    after_norm.  Stages that do not commute (LayerNorms with affines, frame mixing) make any reordering, a layer on the
    wrong side of the upsampling or a missing stage fail."""
    d = of.enc_dims_of(fw)
    C, F = d.dim, d.ffn
    for n in ("embed", "up_embed"):
        fw[f"encoder.{n}.out.0.weight"], fw[f"encoder.{n}.out.0.bias"] = torch.eye(C), torch.zeros(C)
    pl = "encoder.pre_lookahead_layer"
    fw[pl + ".conv1.weight"].zero_()
    fw[pl + ".conv1.bias"].zero_()
    fw[pl + ".conv2.weight"].zero_()
    b_pl = _np(fw, pl + ".conv2.bias")
    s1 = [0.9, -1.4][: d.d1]
    s2 = [1.2, -0.6, 2.0][: d.d2]
    for name, ss in (("encoders", s1), ("up_encoders", s2)):
        for i, s in enumerate(ss):
            p = f"encoder.{name}.{i}"
            fw[p + ".self_attn.linear_out.weight"].zero_()
            fw[p + ".self_attn.linear_out.bias"].zero_()
            _set_ffn(fw, p, C, F, s)
    wu = torch.zeros(C, C, 2 * d.stride + 1)
    for c in range(C):
        wu[c, c, 3] = wu[c, c, 4] = 0.5
    fw["encoder.up_layer.conv.weight"] = wu
    b_up = _np(fw, "encoder.up_layer.conv.bias")

    n, T1 = 8, 8 - d.look
    emb = RNG.normal(0, 1, (n, C))
    A1 = torch.zeros(d.d1, 1, d.heads, 0, 2 * d.dk)
    A2 = torch.zeros(d.d2, 1, d.heads, 0, 2 * d.dk)
    m1 = torch.ones(1, T1, T1, dtype=torch.bool)
    m2 = torch.ones(1, 2 * T1, 2 * T1, dtype=torch.bool)
    xs, *_ = of.encoder_core(fw, d, t64(emb)[None], torch.zeros(1, C, 2 + 2 * d.stride), A1, m1, A2, m2, last=False)
    got = xs[0].double().numpy()

    def ln(x, p, eps):
        return np_ln(x, _np(fw, p + ".weight"), _np(fw, p + ".bias"), eps)

    e = ln(emb, "encoder.embed.out.1", d.eps_embed) * math.sqrt(C)
    e = e[:T1] + b_pl
    for i, s in enumerate(s1):
        e = e + s * np_silu(ln(e, f"encoder.encoders.{i}.norm_ff", d.eps_layer))
    u = np.repeat(e, d.stride, axis=0)
    prev = np.concatenate([np.zeros((1, C)), u[:-1]])
    v = 0.5 * (prev + u) + b_up
    e2 = ln(v, "encoder.up_embed.out.1", d.eps_embed) * math.sqrt(C)
    for i, s in enumerate(s2):
        e2 = e2 + s * np_silu(ln(e2, f"encoder.up_encoders.{i}.norm_ff", d.eps_layer))
    ref = ln(e2, "encoder.after_norm", d.eps_after)
    assert got.shape == ref.shape == (2 * T1, C)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


# --- checkpoint folding (product host code; no GPU) -------------------------------------------------------------------

def _weight_normed_checkpoint(W, old_style_every=4):
    """A stepaudio2-like HiFT state dict for the plain weights ``W``: every conv and transposed conv becomes a torch
    module under weight norm (``parametrizations.weight_norm``, or for every ``old_style_every``-th one the older
    ``weight_g`` / ``weight_v`` form) with random magnitudes and directions, Snake alphas stored as logs.  Returns
    (state dict, the weights torch's own parametrization computes)."""
    import warnings

    from torch.nn.utils.parametrizations import weight_norm

    g = torch.Generator().manual_seed(9)
    sd, want = {}, {}
    n = 0
    for k, w in W.items():
        base = k[: -len(".weight")]
        if k.endswith(".weight") and w.dim() == 3:
            ci, co = (w.shape[0], w.shape[1]) if base.startswith("ups.") else (w.shape[1], w.shape[0])
            mod = (torch.nn.ConvTranspose1d if base.startswith("ups.") else torch.nn.Conv1d)(ci, co, w.shape[2])
            if n % old_style_every == old_style_every - 1:
                with warnings.catch_warnings():
                    warnings.simplefilter("ignore")
                    mod = torch.nn.utils.weight_norm(mod)
                mod.weight_v.data = torch.randn(mod.weight_v.shape, generator=g)
                mod.weight_g.data = torch.rand(mod.weight_g.shape, generator=g) + 0.5
                mod(torch.zeros(1, ci, w.shape[2]))  # the forward pre-hook recomputes the weight from g and v
            else:
                mod = weight_norm(mod)
                pw = mod.parametrizations.weight
                pw.original1.data = torch.randn(pw.original1.shape, generator=g)
                pw.original0.data = torch.rand(pw.original0.shape, generator=g) + 0.5
            n += 1
            for kk, vv in mod.state_dict().items():
                if kk != "bias":
                    sd[f"{base}.{kk}"] = vv.clone()
            want[k] = mod.weight.detach().clone()
        elif k.endswith(".alpha"):
            sd[k] = torch.log(w)
            want[k] = w
        else:
            sd[k] = w
            want[k] = w
    return sd, want


def test_fold_weight_norm_matches_torch_parametrizations():
    """Folding a weight-normed HiFT checkpoint gives the weights torch's parametrizations compute (the ones
    ``remove_parametrizations(leave_parametrized=True)`` keeps, ``hift_lean.py:107-134``), and exp of log-scale
    alphas; the oracle vocoder built from the folded dict equals the one built from those weights."""
    from t2w_amd.weights import fold_weight_norm

    W = init_hift(SMALL, seed=4)
    sd, want = _weight_normed_checkpoint(W)
    assert any(k.endswith(".parametrizations.weight.original0") for k in sd) and any(k.endswith(".weight_g") for k in sd)
    got = fold_weight_norm(sd, snake_logscale=True)
    assert set(got) == set(want)
    for k in want:
        if k.endswith(".alpha"):
            torch.testing.assert_close(got[k], want[k], rtol=1e-6, atol=0)
        else:
            assert torch.equal(got[k], want[k]), k
    mel = t64(RNG.normal(-5, 2, (1, SMALL.mel, 4)))
    ri, nz = oh.hift_noise(9, [3], 4 * 480)
    a = oh.forward_noise(oh.HiFT(got, SMALL_DIMS), mel, torch.zeros(1, 1, 0), ri, nz)[0]
    b = oh.forward_noise(oh.HiFT({k: v.detach() for k, v in want.items()}, SMALL_DIMS), mel, torch.zeros(1, 1, 0), ri, nz)[0]
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


def test_fold_weight_norm_plain_dict_unchanged_and_errors():
    from t2w_amd.weights import fold_weight_norm

    W = init_hift(SMALL, seed=4)
    f = fold_weight_norm(W)
    assert set(f) == set(W) and all(torch.equal(f[k], W[k]) for k in W)
    with pytest.raises(ValueError, match="magnitude and the direction"):
        fold_weight_norm({"conv_pre.weight_g": torch.ones(3, 1, 1)})
    with pytest.raises(ValueError, match="does not fit"):
        fold_weight_norm({"c.weight_g": torch.ones(3, 2, 1), "c.weight_v": torch.ones(3, 2, 5)})
