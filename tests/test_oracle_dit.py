"""Pins of the DiT oracle (CPU): closed forms, library routines and invariants, each chosen so that a plausible mistake
(wrong cache order, conv cache taken at the wrong frame, dropped CFG term, wrong noise offset, mask leak) fails."""

import math

import numpy as np
import pytest
import torch

from oracle import dit as od

import t2w_amd  # noqa: F401
from t2w_amd.config import DiTConfig
from t2w_amd.weights import init_dit

TINY = DiTConfig(hidden=128, depth=2, heads=2, ffn=256, steps=4)


@pytest.fixture(scope="module")
def W():
    return init_dit(TINY, seed=7)


def d_of(W, steps=4, cfg=0.7):
    return od.dims_of(W, steps=steps, cfg_rate=cfg)


def test_t_schedule_closed_form():
    ts, dts = od.t_schedule(10)
    k = np.arange(11)
    span = 1 - np.cos(k / 10 * np.pi / 2)
    assert ts[0] == 0.0
    np.testing.assert_allclose(ts, span[:10], atol=2e-7)
    np.testing.assert_allclose(np.array(ts) + np.array(dts), span[1:], atol=3e-7)
    assert abs(sum(dts) - 1.0) < 1e-6


def test_modulated_layer_norm_closed_form():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 64, generator=g) * 3 + 2
    sh, sc = torch.randn(64, generator=g), torch.randn(64, generator=g)
    got = od.modulate(od.layer_norm(x, 1e-6), sh, sc).double().numpy()
    xd = x.double().numpy()
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6) * (1 + sc.double().numpy()) + sh.double().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_mish_closed_form():
    x = torch.linspace(-30, 30, 1001)
    ref = x.double() * torch.tanh(torch.where(x.double() > 20, x.double(), torch.log1p(torch.exp(x.double()))))
    np.testing.assert_allclose(od.mish(x).double().numpy(), ref.numpy(), rtol=1e-6, atol=1e-6)


def test_causal_conv_chunked_equals_full():
    """Carrying the two-frame cache across chunks equals one causal conv over the whole sequence (zero left pad), and
    the cache of a row with fewer real frames than its padded length is taken at its real end."""
    g = torch.Generator().manual_seed(1)
    C, T = 16, 23
    w, b = torch.randn(C, C, 3, generator=g), torch.randn(C, generator=g)
    x = torch.randn(1, C, T, generator=g)
    full = torch.nn.functional.conv1d(torch.nn.functional.pad(x, (2, 0)), w, b)
    cache = torch.zeros(1, C, 2)
    outs = []
    for a, e in ((0, 1), (1, 9), (9, 10), (10, 23)):
        y, cache = od.causal_conv_chunk(w, b, x[:, :, a:e], cache, torch.tensor([e - a]))
        outs.append(y)
    torch.testing.assert_close(torch.cat(outs, 2), full, rtol=1e-5, atol=1e-5)
    # padded row: real length 5 of 8 -> new cache = frames 3, 4
    _, c = od.causal_conv_chunk(w, b, x[:, :, :8], torch.zeros(1, C, 2), torch.tensor([5]))
    torch.testing.assert_close(c, x[:, :, 3:5])


def test_attention_mask_and_cache_order_vs_brute_force(W):
    d = d_of(W)
    g = torch.Generator().manual_seed(2)
    T, L = 7, 5
    a = torch.randn(1, T, d.hidden, generator=g)
    cache = torch.randn(1, d.heads, L, 2 * d.head_dim, generator=g)
    mask = torch.ones(1, T, T + L, dtype=torch.bool)
    mask[0, :, :T] = od.chunk_mask(T, 3)
    out, kv = od.attention_chunk(W, d, 0, a, cache, mask)
    assert torch.equal(kv[:, :, T:], cache)  # [new, cache]
    # brute force from the new keys/values the oracle formed
    p = "blocks.0.attn."
    q = od.layer_norm(torch.nn.functional.linear(a, W[p + "to_q.weight"], W[p + "to_q.bias"]).view(1, T, d.heads, d.head_dim), 1e-6,
                      W[p + "q_norm.weight"], W[p + "q_norm.bias"])
    o = torch.zeros(T, d.heads, d.head_dim)
    for i in range(T):
        for h in range(d.heads):
            keys = [j for j in range(T + L) if (j >= T or (j // 3) <= (i // 3))]
            s = torch.tensor([float(q[0, i, h] @ kv[0, h, j, :d.head_dim]) / math.sqrt(d.head_dim) for j in keys])
            pr = torch.softmax(s, 0)
            o[i, h] = sum(pr[n] * kv[0, h, j, d.head_dim:] for n, j in enumerate(keys))
    ref = torch.nn.functional.linear(o.reshape(1, T, -1), W[p + "proj.weight"], W[p + "proj.bias"])
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("depth", [2, 3])
def test_streaming_equals_full_sequence(W, depth):
    """A prompt setup followed by two kept windows (each attending the previous ones through per-step caches, reading the
    flow noise at its cache offset) equals one whole-sequence solve under the block-causal mask [prompt | w1 | w2].
    Depth 3 as well: the caches' CFG-row and block axes must not be interchangeable."""
    if depth != 2:
        W = init_dit(DiTConfig(hidden=128, depth=depth, heads=2, ffn=256, steps=4), seed=7)
    d = d_of(W)
    g = torch.Generator().manual_seed(3)
    P, T1, T2 = 12, 6, 9
    mu = torch.randn(80, P + T1 + T2, generator=g)
    spk = torch.randn(1, 80, generator=g)
    pc = torch.randn(80, P, generator=g)
    c = od.empty_cache(d, keep=1000)
    outs = [od.solve(W, d, W["rand_noise"], [c], [mu[:, :P]], spk, [pc])[0]]
    outs.append(od.solve(W, d, W["rand_noise"], [c], [mu[:, P:P + T1]], spk, None)[0])
    outs.append(od.solve(W, d, W["rand_noise"], [c], [mu[:, P + T1:]], spk, None)[0])
    assert c.length == P + T1 + T2
    cond = torch.cat([pc, torch.zeros(80, T1 + T2)], 1)
    full = od.solve_full(W, d, W["rand_noise"], mu, spk[0], cond, [P, T1, T2])
    torch.testing.assert_close(torch.cat(outs, 1), full, rtol=2e-4, atol=2e-4)


def test_chunk_mode_equals_streaming_windows(W):
    """chunk > 0 on a whole row equals feeding its chunks as successive kept windows (no trim)."""
    d = d_of(W)
    g = torch.Generator().manual_seed(4)
    mu = torch.randn(80, 15, generator=g)
    spk = torch.randn(1, 80, generator=g)
    whole = od.solve(W, d, W["rand_noise"], [od.empty_cache(d)], [mu], spk, None, [False], chunk=5)[0]
    c = od.empty_cache(d, keep=1000)
    parts = [od.solve(W, d, W["rand_noise"], [c], [mu[:, a:a + 5]], spk, None)[0] for a in (0, 5, 10)]
    torch.testing.assert_close(whole, torch.cat(parts, 1), rtol=2e-4, atol=2e-4)


def test_cfg_zero_is_plain_euler_on_the_conditional_row(W):
    """cfg_rate 0: the solve integrates the conditional row's velocity alone (the unconditional row drops out)."""
    d = d_of(W, cfg=0.0)
    g = torch.Generator().manual_seed(5)
    T = 6
    mu, spk = torch.randn(80, T, generator=g), torch.randn(1, 80, generator=g)
    got = od.solve(W, d, W["rand_noise"], [od.empty_cache(d)], [mu], spk, None, [False])[0]
    ts, dts = od.t_schedule(d.steps)
    x = W["rand_noise"][0, :, :T][None].clone()
    z = lambda *s: torch.zeros(*s)  # noqa: E731
    for s in range(d.steps):
        dphi, _, _ = od.estimator_chunk(W, d, x, mu[None], od.t_embed(W, torch.full((1,), ts[s])), spk, z(1, 80, T), z(d.depth, 1, 2 * d.hidden, 2),
                                        z(d.depth, 1, d.heads, 0, 2 * d.head_dim), torch.ones(1, T, T, dtype=torch.bool), torch.tensor([T]))
        x = x + dts[s] * dphi
    torch.testing.assert_close(got, x[0], rtol=1e-5, atol=1e-5)


def test_euler_cfg_on_a_linear_field(monkeypatch, W):
    """With a velocity field a x (cond) / b x (uncond), x_K = x_0 prod_k (1 + dt_k ((1 + l) a - l b)): the CFG combine, its
    sign and every dt of the schedule appear in the closed form."""
    d = d_of(W, steps=10, cfg=0.7)
    a, b = 0.8, -0.3

    def field(W_, d_, x, mu, temb, spks, cond, cnn, att, mask, tr, pos=None):
        return torch.cat([a * x[:1], b * x[1:]]), cnn[:, :, :, :0], att[:, :, :, :0]

    monkeypatch.setattr(od, "estimator_chunk", field)
    g = torch.Generator().manual_seed(6)
    mu, spk = torch.randn(80, 4, generator=g), torch.randn(1, 80, generator=g)
    got = od.solve(W, d, W["rand_noise"], [od.empty_cache(d)], [mu], spk, None, [False])[0]
    _, dts = od.t_schedule(10)
    f = np.prod([1 + dt * ((1 + 0.7) * a - 0.7 * b) for dt in dts])
    torch.testing.assert_close(got, W["rand_noise"][0, :, :4] * f, rtol=1e-5, atol=1e-6)


def test_noise_is_read_at_the_cache_offset(monkeypatch, W):
    d = d_of(W, steps=1, cfg=0.0)
    seen = []

    def field(W_, d_, x, mu, temb, spks, cond, cnn, att, mask, tr, pos=None):
        seen.append(x[0].clone())
        T = x.shape[2]
        return torch.zeros_like(x), cnn, torch.cat([torch.zeros(att.shape[0], att.shape[1], att.shape[2], T, att.shape[4]), att], 3)

    monkeypatch.setattr(od, "estimator_chunk", field)
    c = od.empty_cache(d, keep=1000)
    od.solve(W, d, W["rand_noise"], [c], [torch.zeros(80, 7)], torch.zeros(1, 80), None)
    od.solve(W, d, W["rand_noise"], [c], [torch.zeros(80, 3)], torch.zeros(1, 80), None)
    torch.testing.assert_close(seen[1], W["rand_noise"][0, :, 7:10])


@pytest.mark.parametrize("keep", [0, 30, 250])
def test_trim_keeps_first_keep_and_last_100(keep):
    order = list(range(400))
    got = od.trim_order(order, keep)
    assert got == (order if 400 <= keep + 100 else order[:keep] + order[-100:])
    att = torch.arange(400.0).view(1, 1, 1, 1, 400, 1).expand(1, 1, 2, 1, 400, 2)
    assert od.trim(att, keep)[0, 0, 0, 0, :, 0].long().tolist() == got


def test_trim_evicts_the_prompt_middle_not_the_newest():
    """Windows are prepended ([new, cache]); after the trim the row holds the newest `keep` frames and the oldest 100 (the
    prompt's tail when the prompt is longer than 100) - what the reference code does, not its docstring."""
    P = 150
    order = [f"p{i}" for i in range(P)]
    for w in range(4):
        order = od.trim_order([f"w{w}_{i}" for i in range(50)] + order, P)
    assert len(order) == P + 100
    assert order[:50] == [f"w3_{i}" for i in range(50)]
    assert order[-100:] == [f"p{i}" for i in range(50, 150)]


def test_rope_closed_forms():
    """The optional rotary embedding (no counterpart in the reference, whose DiT has no positional encoding): the
    frequency table's endpoints, position 0 is the identity, a unit vector on channel 2i turns into (cos, sin) of
    pos * theta^(-2i / 64) on channels (2i, 2i + 1) and nowhere else (consecutive pairs, not halves of the head), pair
    norms are kept, and q.k depends on the difference of the positions only."""
    f = od.rope_freqs(64, 10000.0)
    assert f.dtype == torch.float32 and f.shape == (32,)
    assert float(f[0]) == 1.0 and math.isclose(float(f[31]), 10000.0 ** (-62 / 64), rel_tol=1e-7)
    assert bool((f[1:] < f[:-1]).all())
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 5, 3, 64, generator=g)
    assert torch.equal(od.rope(x, torch.zeros(2, 5, dtype=torch.long), 1e4), x)
    for i in (0, 1, 7, 31):
        e = torch.zeros(1, 1, 1, 64)
        e[..., 2 * i] = 1.0
        y = od.rope(e, torch.tensor([[37]]), 1e4)[0, 0, 0]
        a = 37 * float(f[i])
        want = torch.zeros(64)
        want[2 * i], want[2 * i + 1] = math.cos(a), math.sin(a)
        torch.testing.assert_close(y, want, rtol=0, atol=1e-6)
    pos = torch.randint(0, 5000, (2, 5), generator=g)
    y = od.rope(x, pos, 1e4)
    torch.testing.assert_close(y.view(2, 5, 3, 32, 2).norm(dim=-1), x.view(2, 5, 3, 32, 2).norm(dim=-1), rtol=1e-5, atol=1e-5)
    q, k = torch.randn(1, 1, 1, 64, generator=g), torch.randn(1, 1, 1, 64, generator=g)

    def dot(m, n):
        return float((od.rope(q, torch.tensor([[m]]), 1e4) * od.rope(k, torch.tensor([[n]]), 1e4)).sum())

    assert abs(dot(10, 3) - dot(110, 103)) < 1e-3 and abs(dot(0, 5) - dot(40, 45)) < 1e-3
    assert abs(dot(10, 3) - dot(10, 4)) > 1e-2


def test_rope_streaming_equals_full_sequence(W):
    """With the rotary embedding on, a prompt setup followed by two kept windows still equals the whole-sequence solve
    under the block-causal mask: each window's frames take the stream positions after the kept frames before them, and
    cached keys keep the rotation they were written with.  The embedding changes the result (it is applied)."""
    d = od.dims_of(W, steps=4, rope_theta=10000.0)
    g = torch.Generator().manual_seed(3)
    P, T1, T2 = 12, 6, 9
    mu = torch.randn(80, P + T1 + T2, generator=g)
    spk = torch.randn(1, 80, generator=g)
    pc = torch.randn(80, P, generator=g)
    c = od.empty_cache(d, keep=1000)
    outs = [od.solve(W, d, W["rand_noise"], [c], [mu[:, :P]], spk, [pc])[0]]
    outs.append(od.solve(W, d, W["rand_noise"], [c], [mu[:, P:P + T1]], spk, None)[0])
    outs.append(od.solve(W, d, W["rand_noise"], [c], [mu[:, P + T1:]], spk, None)[0])
    assert c.pos == P + T1 + T2
    cond = torch.cat([pc, torch.zeros(80, T1 + T2)], 1)
    full = od.solve_full(W, d, W["rand_noise"], mu, spk[0], cond, [P, T1, T2])
    torch.testing.assert_close(torch.cat(outs, 1), full, rtol=2e-4, atol=2e-4)
    plain = od.solve_full(W, d_of(W), W["rand_noise"], mu, spk[0], cond, [P, T1, T2])
    assert float((plain - full).abs().max()) > 1e-3


def test_rope_position_survives_the_trim(W):
    """Positions count kept frames, not cached ones: after a trim the cache is shorter than the stream, the next window
    still starts at the stream position, and a window that is not kept does not advance it."""
    d = od.dims_of(W, steps=2, rope_theta=10000.0)
    g = torch.Generator().manual_seed(5)
    c = od.empty_cache(d, keep=10)
    spk = torch.randn(1, 80, generator=g)
    for T, kp in ((10, True), (60, True), (60, True), (20, False)):
        od.solve(W, d, W["rand_noise"], [c], [torch.randn(80, T, generator=g)], spk, None, [kp])
    assert c.pos == 130 and c.length == 10 + 100
