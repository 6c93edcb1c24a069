"""Oracle of the flow encoder (codec tokens -> ``mu``), fp32, CPU.  Test infrastructure: the product never imports it.

Follows, in the reference repository:

* ``engine/runtime/token2wav_batch.py:42-79`` (``_encoder_core``: embed, the pre-lookahead layer with its two cached
  frames, the first conformer stack on ``[cache | window]`` keys with relative positions, the 2x upsampling with its
  cached frames, the up-embed, the second stack, the final norm; zero lookahead frames for a final window);
* ``:402-444`` (``_encoder``: a stream's packed attention cache ``[d1 + d2, nh, 2 t, 2 dk]`` holds the first stack's t
  frames tiled twice and the second stack's 2 t frames; the first stack reads the first half of the time axis; the new
  cache is ``cat([c1.repeat(2), c2])``), ``:388-400`` (``_flow_finish``: the cache is trimmed along its time axis to the
  first ``keep`` and last 100 entries, keep = the prompt's mel frames), ``:365-386`` (``_flow_encode``: speaker
  embedding ``spk_embed_affine_layer(normalize(spk))``, ``mu = encoder_proj(h)``), ``:556-565`` (``_setup_encoder_one``:
  the prompt plus three silence tokens through an empty-cache chunk, not final), ``:603-611`` (``Upsample1D`` and the
  pre-lookahead layer with empty caches: zero frames);
* the comment at ``token2wav_batch.py:4-7``: the relative position of query i and key j is ``(L - T + i) - j`` for L keys
  and T queries.

Not visible in the reference (inside ``stepaudio2``) and defined here after the published CosyVoice2 / WeNet
``UpsampleConformerEncoder``: width 512, 8 heads of 64, FFN 2048 with SiLU, 6 + 4 layers (pre-norm, no macaron, no conv
module), ESPnet relative-position self-attention (``pos_bias_u`` / ``pos_bias_v``, bias-free ``linear_pos``, the
sinusoid table of relative positions ``L - 1 .. -(L - 1)``), the linear input layer (Linear + LayerNorm, then
``x sqrt(512)``), pre-lookahead layer (conv k = 4 over the window, leaky ReLU 0.01, causal conv k = 3, residual),
``Upsample1D`` (nearest x2, conv k = 5 over 4 cached frames and the upsampled ones), LayerNorm eps 1e-12 in the layers
and 1e-5 in the input layers and the final norm, vocabulary 6561, speaker embedding 192 -> 80.  Against stepaudio2
these are parity unpinned; the tests pin this oracle's composition with closed forms and invariants.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

TRIM_SUFFIX = 100
SILENCE_TOKEN = 4218


@dataclass(frozen=True)
class EncDims:
    vocab: int = 6561
    dim: int = 512
    heads: int = 8
    ffn: int = 2048
    d1: int = 6
    d2: int = 4
    look: int = 3
    stride: int = 2
    mel: int = 80
    spk: int = 192
    eps_layer: float = 1e-12
    eps_embed: float = 1e-5
    eps_after: float = 1e-5
    lrelu: float = 0.01

    @property
    def dk(self) -> int:
        return self.dim // self.heads


def enc_dims_of(W: dict) -> EncDims:
    V, C = W["input_embedding.weight"].shape
    d1 = sum(1 for k in W if k.startswith("encoder.encoders.") and k.endswith(".self_attn.linear_q.weight"))
    d2 = sum(1 for k in W if k.startswith("encoder.up_encoders.") and k.endswith(".self_attn.linear_q.weight"))
    heads = W["encoder.encoders.0.self_attn.pos_bias_u"].shape[0]
    return EncDims(vocab=V, dim=C, heads=heads, ffn=W["encoder.encoders.0.feed_forward.w_1.weight"].shape[0], d1=d1, d2=d2,
                   look=W["encoder.pre_lookahead_layer.conv1.weight"].shape[2] - 1, mel=W["encoder_proj.weight"].shape[0],
                   spk=W["spk_embed_affine_layer.weight"].shape[1])


# --- relative positions -------------------------------------------------------------------------------------------------

def rel_pos_table(size: int, d: int) -> torch.Tensor:
    """The sinusoid of relative positions ``size - 1, size - 2, .., -(size - 1)`` ([2 size - 1, d]; even columns sin,
    odd columns cos of ``pos * 10000^(-2i / d)``)."""
    pos = torch.arange(size - 1, -size, -1, dtype=torch.float64)[:, None]
    div = torch.exp(torch.arange(0, d, 2, dtype=torch.float64) * -(math.log(10000.0) / d))
    pe = torch.zeros(2 * size - 1, d, dtype=torch.float64)
    pe[:, 0::2] = torch.sin(pos * div)
    pe[:, 1::2] = torch.cos(pos * div)
    return pe.float()


def rel_shift(x: torch.Tensor) -> torch.Tensor:
    """[.., T, 2 L - 1] scores over the relative-position table -> [.., T, L] over keys: entry (i, j) takes table
    column ``T - 1 - i + j``, the position ``(L - T + i) - j``."""
    T, P = x.shape[-2], x.shape[-1]
    L = (P + 1) // 2
    i = torch.arange(T)[:, None]
    j = torch.arange(L)[None, :]
    idx = (T - 1 - i + j).expand(*x.shape[:-2], T, L)
    return torch.gather(x, -1, idx)


# --- modules ---------------------------------------------------------------------------------------------------------

def _ln(x, W, p, eps):
    return F.layer_norm(x, (x.shape[-1],), W[p + ".weight"], W[p + ".bias"], eps)


def _lin(x, W, p, bias=True):
    return F.linear(x, W[p + ".weight"], W[p + ".bias"] if bias else None)


def linear_embed(W, p: str, x: torch.Tensor, d: EncDims) -> torch.Tensor:
    """The linear input layer: Linear, LayerNorm, then the positional encoding's ``x sqrt(dim)``."""
    return _ln(_lin(x, W, p + ".out.0"), W, p + ".out.1", d.eps_embed) * math.sqrt(d.dim)


def rel_attention(W, p: str, x: torch.Tensor, mask: torch.Tensor, pos: torch.Tensor, cache: torch.Tensor, d: EncDims):
    """Relative-position self-attention on a window: x [B, T, C]; cache [B, h, Lc, 2 dk] (k | v of earlier frames, in time
    order); mask [B, T, Lc + T] over keys ``[cache, new]``; pos [2 L - 1, C] (L = Lc + T).  Returns (out, new cache
    ``[cache, new]`` [B, h, L, 2 dk])."""
    B, T, C = x.shape
    h, dk = d.heads, d.dk
    q = _lin(x, W, p + ".linear_q").view(B, T, h, dk)
    k = _lin(x, W, p + ".linear_k").view(B, T, h, dk).transpose(1, 2)
    v = _lin(x, W, p + ".linear_v").view(B, T, h, dk).transpose(1, 2)
    kv = torch.cat([cache, torch.cat([k, v], dim=-1)], dim=2)
    kk, vv = kv[..., :dk], kv[..., dk:]
    pp = F.linear(pos, W[p + ".linear_pos.weight"]).view(-1, h, dk).transpose(0, 1)  # [h, 2L - 1, dk]
    qu = (q + W[p + ".pos_bias_u"]).transpose(1, 2)
    qv = (q + W[p + ".pos_bias_v"]).transpose(1, 2)
    ac = torch.matmul(qu, kk.transpose(-1, -2))
    bd = rel_shift(torch.matmul(qv, pp.transpose(-1, -2)[None]))
    s = (ac + bd) / math.sqrt(dk)
    s = s.masked_fill(~mask[:, None], float("-inf"))
    a = torch.softmax(s, dim=-1).masked_fill(~mask[:, None], 0.0)
    o = torch.matmul(a, vv).transpose(1, 2).reshape(B, T, C)
    return _lin(o, W, p + ".linear_out"), kv


def conformer_layer(W, p: str, x, mask, pos, cache, d: EncDims):
    """Pre-norm layer: x += attn(norm_mha x); x += FFN(norm_ff x), FFN = w_2 SiLU(w_1 .)."""
    a, new = rel_attention(W, p + ".self_attn", _ln(x, W, p + ".norm_mha", d.eps_layer), mask, pos, cache, d)
    x = x + a
    f = _lin(F.silu(_lin(_ln(x, W, p + ".norm_ff", d.eps_layer), W, p + ".feed_forward.w_1")), W, p + ".feed_forward.w_2")
    return x + f, new


def pre_lookahead(W, x: torch.Tensor, cache: torch.Tensor, d: EncDims):
    """x [B, T + look, C] (the window with its lookahead frames); cache [B, C, 2] (earlier conv1 outputs).  conv1 (k =
    look + 1, no padding) sees each frame and its lookahead; leaky ReLU; conv2 (k = 3) over ``[cache | .]``; + x[:T].
    Returns (out [B, T, C], new cache = the last two conv1 outputs)."""
    p = "encoder.pre_lookahead_layer"
    o = F.leaky_relu(F.conv1d(x.transpose(1, 2), W[p + ".conv1.weight"], W[p + ".conv1.bias"]), d.lrelu)  # [B, C, T]
    full = torch.cat([cache, o], dim=2)
    y = F.conv1d(full, W[p + ".conv2.weight"], W[p + ".conv2.bias"]).transpose(1, 2)
    return y + x[:, : o.shape[2]], full[:, :, -2:]


def upsample(W, x: torch.Tensor, cache: torch.Tensor, d: EncDims):
    """Nearest x stride, then conv (k = 2 stride + 1) over ``[cache (2 stride frames) | upsampled]``: x [B, C, T] ->
    ([B, C, stride T], new cache = the last 2 stride upsampled frames)."""
    u = F.interpolate(x, scale_factor=float(d.stride), mode="nearest")
    full = torch.cat([cache, u], dim=2)
    y = F.conv1d(full, W["encoder.up_layer.conv.weight"], W["encoder.up_layer.conv.bias"])
    return y, full[:, :, -2 * d.stride:]


def encoder_core(W, d: EncDims, emb: torch.Tensor, cnn: torch.Tensor, A1: torch.Tensor, mask1: torch.Tensor, A2: torch.Tensor,
                 mask2: torch.Tensor, last: bool):
    """``_encoder_core`` (``token2wav_batch.py:42-79``) on token embeddings ``emb`` [B, n, C]; cnn [B, C, 2 + 2 stride];
    A1 [d1, B, h, L1, 2 dk], A2 [d2, B, h, 2 L1, 2 dk] (cached keys in time order); mask1 [B, T1, L1 + T1], mask2
    [B, T2, L2 + T2].  Returns (xs [B, T2, C], new1 [d1, B, h, L1 + T1, 2 dk], new2, new cnn)."""
    L1, L2 = A1.shape[3], A2.shape[3]
    xs = linear_embed(W, "encoder.embed", emb, d)
    if last:
        xs = F.pad(xs, (0, 0, 0, d.look))
    xs, c1 = pre_lookahead(W, xs, cnn[:, :, :2], d)
    pos = rel_pos_table(L1 + xs.shape[1], d.dim)
    new1 = []
    for i in range(d.d1):
        xs, c = conformer_layer(W, f"encoder.encoders.{i}", xs, mask1, pos, A1[i], d)
        new1.append(c)
    up, c2 = upsample(W, xs.transpose(1, 2), cnn[:, :, 2:], d)
    xs = linear_embed(W, "encoder.up_embed", up.transpose(1, 2), d)
    pos = rel_pos_table(L2 + xs.shape[1], d.dim)
    new2 = []
    for i in range(d.d2):
        xs, c = conformer_layer(W, f"encoder.up_encoders.{i}", xs, mask2, pos, A2[i], d)
        new2.append(c)
    xs = _ln(xs, W, "encoder.after_norm", d.eps_after)
    return xs, torch.stack(new1), torch.stack(new2), torch.cat([c1, c2], dim=2)


# --- streams ---------------------------------------------------------------------------------------------------------

@dataclass
class EncState:
    """A stream's encoder caches: att [d1 + d2, h, 2 t, 2 dk] (first stack tiled twice along time, then the second
    stack), cnn [C, 2 + 2 stride], and the trim length ``keep`` (the prompt's mel frames)."""
    att: torch.Tensor
    cnn: torch.Tensor
    keep: int = 0


def empty_state(d: EncDims, keep: int = 0) -> EncState:
    return EncState(torch.zeros(d.d1 + d.d2, d.heads, 0, 2 * d.dk), torch.zeros(d.dim, 2 + 2 * d.stride), keep)


def trim(att: torch.Tensor, keep: int) -> torch.Tensor:
    """``_trim`` along the time axis: above ``keep + 100`` entries keep the first ``keep`` and the last 100."""
    n = att.shape[2]
    if n > keep + TRIM_SUFFIX:
        return torch.cat([att[:, :, :keep], att[:, :, n - TRIM_SUFFIX:]], dim=2)
    return att


def encode_window(W, d: EncDims, st: EncState, tokens: list[int], last: bool, trim_after: bool = True) -> torch.Tensor:
    """One stream's window through the encoder with its caches (``_encoder``, ``token2wav_batch.py:402-444``), the
    caches updated (and trimmed as ``_flow_finish`` does) in place.  Returns the encoder output projected to the mel
    dimension, ``mu`` [mel, T2] (T2 = 2 x the window's tokens after its lookahead, all of them when final)."""
    emb = W["input_embedding.weight"][torch.tensor(tokens)][None]
    off1 = st.att.shape[2] // 2
    A1 = st.att[: d.d1, None, :, :off1]
    A2 = st.att[d.d1:, None]
    T1 = len(tokens) if last else len(tokens) - d.look
    T2 = d.stride * T1
    m1 = torch.ones(1, T1, off1 + T1, dtype=torch.bool)
    m2 = torch.ones(1, T2, A2.shape[3] + T2, dtype=torch.bool)
    xs, new1, new2, cnn = encoder_core(W, d, emb, st.cnn[None], A1, m1, A2, m2, last)
    c1 = new1[:, 0]
    st.att = torch.cat([c1.repeat(1, 1, 2, 1), new2[:, 0]], dim=0)
    st.cnn = cnn[0]
    if trim_after:
        st.att = trim(st.att, st.keep)
    return _lin(xs, W, "encoder_proj")[0].t()


def setup(W, d: EncDims, tokens: list[int]) -> tuple[torch.Tensor, EncState]:
    """A prompt's encoder pass (``_setup_encoder_one``, ``token2wav_batch.py:556-565``): its tokens and three silence
    tokens through an empty-cache chunk, not final.  Returns (mu [mel, 2 n], the stream's starting state; keep = 2 n)."""
    st = empty_state(d, keep=d.stride * len(tokens))
    mu = encode_window(W, d, st, list(tokens) + [SILENCE_TOKEN] * d.look, last=False, trim_after=False)
    return mu, st


def speaker(W, spk: torch.Tensor) -> torch.Tensor:
    """``spk_embed_affine_layer(normalize(spk))``: [B, 192] -> [B, mel]."""
    return F.linear(F.normalize(spk, dim=1), W["spk_embed_affine_layer.weight"], W["spk_embed_affine_layer.bias"])
