"""Oracle of the flow-matching DiT estimator and the CFG Euler solve (fp32, CPU).

Follows, in the reference repository:

* ``engine/runtime/token2wav_batch.py:787-810`` (``_estimator_temb``: input packing ``[x | mu | spk | cond]``, in_proj,
  blocks, final layer), ``:100-110`` (``_block_chunk``: attention, then causal conv block, then MLP, each a gated residual
  of a modulated norm), ``:82-97`` (``_conv_chunk`` / ``_conv_block_chunk``: kernel-3 causal convs whose two cached frames
  precede the window; new cache = the two frames ending at the row's real end), ``:632-702`` (``_solve``: CFG rows
  ``[cond.., uncond..]`` with ``mu = spk = cond = 0`` on the uncond half, cosine t schedule, Euler/CFG update, new caches
  ``[new frames, old cache]``), ``:36-39`` (``_trim``);
* ``engine/runtime/dit_fast.py:157-178`` (one timestep embedding and adaLN table per step, shared by all rows),
  ``:282-302`` (block order and the Euler line), ``:448-449`` (x0 = the flow's fixed noise read at the row's cache
  offset), ``:480-490`` (trim: ``order = new + old``; above ``keep + 100`` keep ``order[:keep] + order[-100:]``);
* ``engine/runtime/dit_kernels.py`` (LayerNorm then ``x * (1 + scale) + shift``; per-head affine q/k LayerNorm over 64
  values; affine LayerNorm + Mish with softplus threshold 20; GELU-tanh in the MLP).

Not visible in the reference (inside ``stepaudio2``) and defined here, CosyVoice2-style: the timestep embedder
(256-frequency sinusoid of ``1000 t``, ``[cos | sin]``, Linear-SiLU-Linear), adaLN = SiLU + Linear, LayerNorm eps
(1e-6 for the block/final norms and q/k norms, 1e-5 for the conv block's affine norm), attention scale ``1/sqrt(64)``,
no positional encoding.  Against the real stepaudio2 modules these are parity unpinned; the tests pin this oracle's
composition (block order, masks, cache order, conv state, CFG/Euler, trim) with invariants and closed forms.

Rotary position embedding (``rope_theta`` > 0; off by default): an option of this build with no counterpart in the
reference, whose DiT has no positional encoding (``engine/runtime/dit_fast.py:6``).  q and k are rotated after their
LayerNorm, pairs of consecutive head channels (2i, 2i + 1) by the angle ``pos * theta^(-2i / head_dim)`` (RoFormer,
Su et al. 2021, eq. 34), at each frame's position in its stream: frames of kept windows count, so cached keys keep the
angle they were written with and a trim leaves every relative distance as it was.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

TRIM_SUFFIX = 100


@dataclass(frozen=True)
class DiTDims:
    mel: int = 80
    hidden: int = 1024
    depth: int = 22
    heads: int = 16
    head_dim: int = 64
    ffn: int = 2048
    freq: int = 256
    eps_block: float = 1e-6
    eps_qk: float = 1e-6
    eps_conv: float = 1e-5
    eps_final: float = 1e-6
    cfg_rate: float = 0.7
    steps: int = 10
    rope_theta: float = 0.0  # 0: no positional encoding (the reference's DiT)


def dims_of(W: dict, steps: int = 10, cfg_rate: float = 0.7, rope_theta: float = 0.0) -> DiTDims:
    H = W["in_proj.weight"].shape[0]
    depth = sum(1 for k in W if k.endswith(".attn.proj.weight"))
    hd = W["blocks.0.attn.q_norm.weight"].shape[0]
    return DiTDims(mel=W["final_layer.linear.weight"].shape[0], hidden=H, depth=depth, heads=H // hd, head_dim=hd,
                   ffn=W["blocks.0.mlp.fc1.weight"].shape[0], freq=W["t_embedder.mlp.0.weight"].shape[1],
                   cfg_rate=cfg_rate, steps=steps, rope_theta=rope_theta)


def rope_freqs(head_dim: int, theta: float) -> torch.Tensor:
    """Angular frequency of channel pair i: theta^(-2i / head_dim), computed in fp64 and rounded to fp32 (the table the
    GPU path takes)."""
    return (theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float64) / head_dim)).float()


def rope(x: torch.Tensor, pos: torch.Tensor, theta: float) -> torch.Tensor:
    """Rotate consecutive channel pairs of x [B, T, nh, dk] at positions pos [B, T]: (x0, x1) -> (x0 cos a - x1 sin a,
    x0 sin a + x1 cos a), a = pos * freq_i rounded to fp32."""
    B, T, nh, dk = x.shape
    ang = pos.float()[:, :, None] * rope_freqs(dk, theta)[None, None, :]  # fp32 product, as on the GPU
    c, s = torch.cos(ang.double()).float()[:, :, None, :], torch.sin(ang.double()).float()[:, :, None, :]
    xp = x.float().reshape(B, T, nh, dk // 2, 2)
    x0, x1 = xp[..., 0], xp[..., 1]
    return torch.stack([x0 * c - x1 * s, x0 * s + x1 * c], dim=-1).reshape(B, T, nh, dk)


# --- schedule and timestep conditioning -----------------------------------------------------------------------------

def t_schedule(steps: int) -> tuple[list[float], list[float]]:
    """The solver's t values and step sizes: ``t_span = 1 - cos(linspace(0, 1, steps + 1) * pi / 2)``, then
    ``t += dt; dt = t_span[k + 1] - t`` (``token2wav_batch.py:669-693``, ``dit_fast.py:161-178``), in fp32."""
    t_span = torch.linspace(0, 1, steps + 1, dtype=torch.float32)
    t_span = 1 - torch.cos(t_span * 0.5 * torch.pi)
    t, dt = t_span[0].clone(), t_span[1] - t_span[0]
    ts, dts = [], []
    for step in range(1, steps + 1):
        ts.append(float(t))
        dts.append(float(dt))
        t = t + dt
        if step < steps:
            dt = t_span[step + 1] - t
    return ts, dts


def freq_table(freq: int, max_period: float = 10000.0) -> torch.Tensor:
    half = freq // 2
    return torch.exp(-math.log(max_period) * torch.arange(0, half, dtype=torch.float32) / half)


T_SCALE = 1000.0  # the embedder sees 1000 t (t in [0, 1])


def timestep_sinusoid(t: torch.Tensor, dim: int) -> torch.Tensor:
    """The DiT timestep frequency embedding of ``1000 t``: ``[cos(1000 t f_k) | sin(1000 t f_k)]`` with
    ``f_k = 10000^(-k / (dim / 2))``, k = 0 .. dim/2 - 1.  t [B] -> [B, dim]."""
    args = (t.float() * T_SCALE)[:, None] * freq_table(dim)[None]
    return torch.cat([torch.cos(args), torch.sin(args)], dim=-1)


def t_embed(W: dict, t: torch.Tensor) -> torch.Tensor:
    """Timestep embedder: sinusoid -> Linear -> SiLU -> Linear.  t [B] -> [B, H]."""
    emb = timestep_sinusoid(t, W["t_embedder.mlp.0.weight"].shape[1])
    h = F.silu(F.linear(emb, W["t_embedder.mlp.0.weight"], W["t_embedder.mlp.0.bias"]))
    return F.linear(h, W["t_embedder.mlp.2.weight"], W["t_embedder.mlp.2.bias"])


def block_mods(W: dict, b: int, temb: torch.Tensor) -> list[torch.Tensor]:
    """adaLN of block b: SiLU + Linear -> 9 chunks (shift/scale/gate of msa, mlp, conv; ``_block_chunk`` order)."""
    m = F.linear(F.silu(temb), W[f"blocks.{b}.adaLN_modulation.1.weight"], W[f"blocks.{b}.adaLN_modulation.1.bias"])
    return list(m.chunk(9, dim=-1))


def final_mods(W: dict, temb: torch.Tensor) -> list[torch.Tensor]:
    m = F.linear(F.silu(temb), W["final_layer.adaLN_modulation.1.weight"], W["final_layer.adaLN_modulation.1.bias"])
    return list(m.chunk(2, dim=-1))


# --- block pieces ---------------------------------------------------------------------------------------------------

def modulate(x, shift, scale):
    return x * (1 + scale) + shift


def layer_norm(x, eps, w=None, b=None):
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def mish(x):
    return x * torch.tanh(F.softplus(x, beta=1.0, threshold=20.0))


def attention_chunk(W, d: DiTDims, b: int, a: torch.Tensor, att_cache: torch.Tensor, mask: torch.Tensor, pos=None):
    """Attention of one block on a window: a [B, T, H]; att_cache [B, nh, L, 2 dk] (k | v); mask [B, T, T + L] over keys
    ``[new, cache]``; pos [B, T] stream positions of the window's frames (used with ``d.rope_theta`` > 0).  Returns (out
    [B, T, H], new cache [B, nh, T + L, 2 dk])."""
    B, T, H = a.shape
    nh, dk = d.heads, d.head_dim
    p = f"blocks.{b}.attn."
    q = F.linear(a, W[p + "to_q.weight"], W[p + "to_q.bias"]).view(B, T, nh, dk)
    k = F.linear(a, W[p + "to_k.weight"], W[p + "to_k.bias"]).view(B, T, nh, dk)
    v = F.linear(a, W[p + "to_v.weight"], W[p + "to_v.bias"]).view(B, T, nh, dk)
    q = layer_norm(q, d.eps_qk, W[p + "q_norm.weight"], W[p + "q_norm.bias"])
    k = layer_norm(k, d.eps_qk, W[p + "k_norm.weight"], W[p + "k_norm.bias"])
    if d.rope_theta > 0:
        q, k = rope(q, pos, d.rope_theta), rope(k, pos, d.rope_theta)
    q, k = q.transpose(1, 2), k.transpose(1, 2)
    kv = torch.cat([k, v.transpose(1, 2)], dim=-1)  # [B, nh, T, 2 dk]
    kv = torch.cat([kv, att_cache], dim=2)  # [new, cache]
    kk, vv = kv[..., :dk], kv[..., dk:]
    s = torch.matmul(q, kk.transpose(-1, -2)) / math.sqrt(dk)
    s = s.masked_fill(~mask[:, None], float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), vv)  # [B, nh, T, dk]
    o = o.transpose(1, 2).reshape(B, T, H)
    return F.linear(o, W[p + "proj.weight"], W[p + "proj.bias"]), kv


def causal_conv_chunk(w, bias, x: torch.Tensor, cache: torch.Tensor, tr: torch.Tensor):
    """Kernel-3 causal conv with two cached frames (``token2wav_batch.py:82-87``): x [B, C, T], cache [B, C, 2].
    Returns (y [B, Cout, T], new cache [B, C, 2] = the two frames of ``[cache | x]`` ending at ``tr``)."""
    full = torch.cat([cache, x], dim=2)
    y = F.conv1d(full, w, bias)
    idx = (tr[:, None] + torch.arange(2)[None, :])[:, None, :].expand(-1, full.shape[1], -1)
    return y, torch.gather(full, 2, idx)


def conv_block_chunk(W, d: DiTDims, b: int, a: torch.Tensor, cnn_cache: torch.Tensor, tr: torch.Tensor):
    """``_conv_block_chunk`` (``token2wav_batch.py:90-97``): conv, affine LayerNorm, Mish, conv.  a [B, T, H];
    cnn_cache [B, 2H, 2] (first conv's frames | second conv's frames)."""
    H = d.hidden
    p = f"blocks.{b}.conv.block."
    c1, c2 = cnn_cache[:, :H], cnn_cache[:, H:]
    y, n1 = causal_conv_chunk(W[p + "1.weight"], W[p + "1.bias"], a.transpose(1, 2), c1, tr)
    y = mish(layer_norm(y.transpose(1, 2), d.eps_conv, W[p + "3.weight"], W[p + "3.bias"]))
    y, n2 = causal_conv_chunk(W[p + "6.weight"], W[p + "6.bias"], y.transpose(1, 2), c2, tr)
    return y.transpose(1, 2), torch.cat([n1, n2], dim=1)


def mlp(W, b: int, a: torch.Tensor) -> torch.Tensor:
    p = f"blocks.{b}.mlp."
    return F.linear(F.gelu(F.linear(a, W[p + "fc1.weight"], W[p + "fc1.bias"]), approximate="tanh"), W[p + "fc2.weight"], W[p + "fc2.bias"])


def block_chunk(W, d: DiTDims, b: int, h, temb, cnn_cache, att_cache, mask, tr, pos=None):
    """``_block_chunk`` (``token2wav_batch.py:100-110``)."""
    sh_a, sc_a, g_a, sh_m, sc_m, g_m, sh_c, sc_c, g_c = [m[:, None, :] for m in block_mods(W, b, temb)]
    o, new_att = attention_chunk(W, d, b, modulate(layer_norm(h, d.eps_block), sh_a, sc_a), att_cache, mask, pos)
    h = h + g_a * o
    c, new_cnn = conv_block_chunk(W, d, b, modulate(layer_norm(h, d.eps_block), sh_c, sc_c), cnn_cache, tr)
    h = h + g_c * c
    h = h + g_m * mlp(W, b, modulate(layer_norm(h, d.eps_block), sh_m, sc_m))
    return h, new_cnn, new_att


def pack_inputs(x, mu, spks, cond) -> torch.Tensor:
    """The estimator input ``[x | mu | spk | cond]`` per frame (``token2wav_batch.py:801-803``: x and mu packed, then the
    speaker embedding repeated over frames, then cond): x, mu, cond [B, mel, T]; spks [B, mel] -> [B, T, 4 mel]."""
    T = x.shape[2]
    return torch.cat([x, mu, spks[:, :, None].expand(-1, -1, T), cond], dim=1).transpose(1, 2)


def estimator_chunk(W, d: DiTDims, x, mu, temb, spks, cond, cnn_cache, att_cache, mask, tr, pos=None):
    """``_estimator_temb`` (``token2wav_batch.py:787-810``).

    x, mu, cond [B, mel, T]; temb [B, H]; spks [B, mel]; cnn_cache [depth, B, 2H, 2]; att_cache [depth, B, nh, L, 2dk];
    mask [B, T, T + L] bool over keys ``[new, cache]``; tr [B] real frames per row; pos [B, T] stream positions (rope).
    Returns (dphi [B, mel, T], new cnn [depth, B, 2H, 2], new att [depth, B, nh, T + L, 2dk])."""
    h = F.linear(pack_inputs(x, mu, spks, cond), W["in_proj.weight"], W["in_proj.bias"])
    new_cnn, new_att = [], []
    for b in range(d.depth):
        h, c, a = block_chunk(W, d, b, h, temb, cnn_cache[b], att_cache[b], mask, tr, pos)
        new_cnn.append(c)
        new_att.append(a)
    sh, sc = [m[:, None, :] for m in final_mods(W, temb)]
    out = F.linear(modulate(layer_norm(h, d.eps_final), sh, sc), W["final_layer.linear.weight"], W["final_layer.linear.bias"])
    return out.transpose(1, 2), torch.stack(new_cnn), torch.stack(new_att)


# --- streaming state ------------------------------------------------------------------------------------------------

@dataclass
class Cache:
    """One request's estimator caches: att [steps, 2 (cond, uncond), depth, nh, L, 2 dk] in the reference order
    (newest window first), cnn [steps, 2, depth, 2H, 2], the trim length ``keep`` (prompt mel frames), and ``pos``, the
    stream position of the next window's first frame (frames of kept windows so far; rope only)."""
    att: torch.Tensor
    cnn: torch.Tensor
    keep: int = 0
    pos: int = 0

    @property
    def length(self) -> int:
        return self.att.shape[4]


def empty_cache(d: DiTDims, keep: int = 0) -> Cache:
    """Per Euler step, per CFG row (2), per block: keys / values [heads, 0, 2 dk] and conv frames [2 H, 2] (the layout
    ``solve`` stores)."""
    return Cache(torch.zeros(d.steps, 2, d.depth, d.heads, 0, 2 * d.head_dim), torch.zeros(d.steps, 2, d.depth, 2 * d.hidden, 2), keep)


def trim_order(order: list, keep: int) -> list:
    """``dit_fast.py:484-487`` / ``token2wav_batch.py:36-39``: above ``keep + 100`` entries keep the first ``keep`` and
    the last 100."""
    if len(order) > keep + TRIM_SUFFIX:
        return order[:keep] + order[len(order) - TRIM_SUFFIX:]
    return order


def trim(att: torch.Tensor, keep: int, dim: int = 4) -> torch.Tensor:
    if att.shape[dim] > keep + TRIM_SUFFIX:
        return torch.cat([att.narrow(dim, 0, keep), att.narrow(dim, att.shape[dim] - TRIM_SUFFIX, TRIM_SUFFIX)], dim=dim)
    return att


def chunk_mask(T: int, chunk: int) -> torch.Tensor:
    """[T, T] visibility among a row's new frames: full (chunk <= 0) or chunk-causal (frame i sees frames of its own
    and earlier chunks)."""
    if chunk <= 0:
        return torch.ones(T, T, dtype=torch.bool)
    c = torch.arange(T) // chunk
    return c[None, :] <= c[:, None]


def solve(W, d: DiTDims, rand_noise: torch.Tensor, caches: list[Cache], mu: list[torch.Tensor], spks: torch.Tensor,
          cond: list | None = None, keep: list[bool] | None = None, chunk: int = 0) -> list[torch.Tensor]:
    """The CFG Euler solve of one window per request (``token2wav_batch.py:632-702`` with ``dit_fast.py:431-495``'s
    per-request cache bookkeeping and trim).

    mu[i] [mel, T_i]; spks [n, mel]; cond[i] [mel, T_i] or None (zeros); keep[i]: keep the window's keys / conv caches
    (then trim), else leave the caches untouched (final flushes).  ``chunk`` > 0: chunk-causal attention among a row's
    new frames (each frame sees its own and earlier chunks of the window, and the whole cache).  Rows run one request at
    a time (batched == per-request is an invariant of the reference).  Returns mel [mel, T_i] per request and updates
    ``caches`` in place."""
    n = len(caches)
    keep = keep if keep is not None else [True] * n
    ts, dts = t_schedule(d.steps)
    outs = []
    for i in range(n):
        c = caches[i]
        T, L = mu[i].shape[1], c.length
        x = rand_noise[0, :, L:L + T][None].float().clone()
        mu_in = torch.cat([mu[i][None], torch.zeros_like(mu[i][None])]).float()
        spk_in = torch.cat([spks[i:i + 1], torch.zeros_like(spks[i:i + 1])]).float()
        ci = cond[i] if cond is not None and cond[i] is not None else torch.zeros_like(mu[i])
        cond_in = torch.cat([ci[None], torch.zeros_like(ci[None])]).float()
        mask = torch.ones(2, T, T + L, dtype=torch.bool)
        mask[:, :, :T] = chunk_mask(T, chunk)
        tr = torch.full((2,), T, dtype=torch.int64)
        pos = (c.pos + torch.arange(T))[None].expand(2, T)
        new_att, new_cnn = [], []
        for s in range(d.steps):
            temb = t_embed(W, torch.full((2,), ts[s]))
            att = c.att[s].transpose(0, 1)  # [2, depth, ...] -> [depth, 2, ...]
            cnn = c.cnn[s].transpose(0, 1)
            dphi, nc, na = estimator_chunk(W, d, x.repeat(2, 1, 1), mu_in, temb, spk_in, cond_in, cnn, att, mask, tr, pos)
            new_att.append(na.transpose(0, 1))
            new_cnn.append(nc.transpose(0, 1))
            dd, u = dphi.chunk(2, dim=0)
            x = x + dts[s] * ((1.0 + d.cfg_rate) * dd - d.cfg_rate * u)
        if keep[i]:
            c.att = trim(torch.stack(new_att), c.keep)
            c.cnn = torch.stack(new_cnn)
            c.pos += T
        outs.append(x[0])
    return outs


def solve_full(W, d: DiTDims, rand_noise, mu: torch.Tensor, spk: torch.Tensor, cond: torch.Tensor, blocks: list[int]) -> torch.Tensor:
    """One request's whole sequence in one solve under the block-causal mask of ``blocks`` (frame counts of
    ``[prompt | w1 | w2 | ..]``): block j's frames see blocks 0..j.  Equals a prompt setup followed by the windows, each
    with the previous ones as cached keys, as long as no trim happened (stream positions for rope, causal convs)."""
    T = mu.shape[1]
    assert sum(blocks) == T
    bid = torch.repeat_interleave(torch.arange(len(blocks)), torch.tensor(blocks))
    vis = bid[None, :] <= bid[:, None]
    ts, dts = t_schedule(d.steps)
    x = rand_noise[0, :, :T][None].float().clone()
    mu_in = torch.cat([mu[None], torch.zeros_like(mu[None])]).float()
    spk_in = torch.cat([spk[None], torch.zeros_like(spk[None])]).float()
    cond_in = torch.cat([cond[None], torch.zeros_like(cond[None])]).float()
    mask = vis[None].expand(2, T, T).clone()
    tr = torch.full((2,), T, dtype=torch.int64)
    pos = torch.arange(T)[None].expand(2, T)
    att = torch.zeros(d.depth, 2, d.heads, 0, 2 * d.head_dim)
    cnn = torch.zeros(d.depth, 2, 2 * d.hidden, 2)
    for s in range(d.steps):
        temb = t_embed(W, torch.full((2,), ts[s]))
        dphi, _, _ = estimator_chunk(W, d, x.repeat(2, 1, 1), mu_in, temb, spk_in, cond_in, cnn, att, mask, tr, pos)
        dd, u = dphi.chunk(2, dim=0)
        x = x + dts[s] * ((1.0 + d.cfg_rate) * dd - d.cfg_rate * u)
    return x[0]


def estimator_forward(W, d: DiTDims, x, mu, t, spks, cond) -> torch.Tensor:
    """One estimator forward with empty caches and full attention (one block): x, mu, cond [B, mel, T]; t [B]."""
    B, _, T = x.shape
    cnn = torch.zeros(d.depth, B, 2 * d.hidden, 2)
    att = torch.zeros(d.depth, B, d.heads, 0, 2 * d.head_dim)
    mask = torch.ones(B, T, T, dtype=torch.bool)
    tr = torch.full((B,), T, dtype=torch.int64)
    pos = torch.arange(T)[None].expand(B, T)
    return estimator_chunk(W, d, x, mu, t_embed(W, t), spks, cond, cnn, att, mask, tr, pos)[0]
