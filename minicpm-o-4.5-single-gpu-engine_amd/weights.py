"""Seeded random-init weights of the flow encoder, the DiT estimator and HiFT (fp32 master copies on the host).

No checkpoint is available offline, so every workload runs on random-init weights of the real architecture.  Names
follow the stepaudio2 module attributes the reference reads (``engine/runtime/dit_fast.py:131-145``,
``engine/models/token2wav.py:160-236``; the flow encoder's CosyVoice2 ``UpsampleConformerEncoder`` names,
``engine/runtime/token2wav_batch.py:42-79``).  Linear and conv weights and biases are uniform in ``+-1/sqrt(fan_in)`` (torch's
default init); LayerNorm affines are ``1 + 0.1 N`` / ``0.1 N``; Snake alphas uniform in [0.5, 1.5]; the f0 classifier is
scaled so that a mel of the workloads' statistics gives both voiced (> 10 Hz) and unvoiced frames.
"""

from __future__ import annotations

import math

import torch

from .config import DiTConfig, FlowConfig, HiFTConfig


class _Init:
    def __init__(self, seed: int):
        self.g = torch.Generator().manual_seed(int(seed))

    def uniform(self, shape, bound):
        return (torch.rand(*shape, generator=self.g) * 2 - 1) * bound

    def linear(self, W, name, out_f, in_f, scale=1.0):
        bd = 1.0 / math.sqrt(in_f)
        W[name + ".weight"] = self.uniform((out_f, in_f), bd) * scale
        W[name + ".bias"] = self.uniform((out_f,), bd) * scale

    def conv(self, W, name, out_c, in_c, k):
        bd = 1.0 / math.sqrt(in_c * k)
        W[name + ".weight"] = self.uniform((out_c, in_c, k), bd)
        W[name + ".bias"] = self.uniform((out_c,), bd)

    def conv_t(self, W, name, in_c, out_c, k):
        bd = 1.0 / math.sqrt(out_c * k)
        W[name + ".weight"] = self.uniform((in_c, out_c, k), bd)
        W[name + ".bias"] = self.uniform((out_c,), bd)

    def norm(self, W, name, n):
        W[name + ".weight"] = 1 + 0.1 * torch.randn(n, generator=self.g)
        W[name + ".bias"] = 0.1 * torch.randn(n, generator=self.g)


def init_dit(cfg: DiTConfig = DiTConfig(), seed: int = 0) -> dict[str, torch.Tensor]:
    ini = _Init(seed)
    H, W = cfg.hidden, {}
    ini.linear(W, "t_embedder.mlp.0", H, cfg.freq)
    ini.linear(W, "t_embedder.mlp.2", H, H)
    ini.linear(W, "in_proj", H, cfg.in_dim)
    for b in range(cfg.depth):
        p = f"blocks.{b}."
        ini.linear(W, p + "adaLN_modulation.1", 9 * H, H)
        for n in ("to_q", "to_k", "to_v", "proj"):
            ini.linear(W, p + "attn." + n, H, H)
        ini.norm(W, p + "attn.q_norm", cfg.head_dim)
        ini.norm(W, p + "attn.k_norm", cfg.head_dim)
        ini.conv(W, p + "conv.block.1", H, H, 3)
        ini.norm(W, p + "conv.block.3", H)
        ini.conv(W, p + "conv.block.6", H, H, 3)
        ini.linear(W, p + "mlp.fc1", cfg.ffn, H)
        ini.linear(W, p + "mlp.fc2", H, cfg.ffn)
    ini.linear(W, "final_layer.adaLN_modulation.1", 2 * H, H)
    ini.linear(W, "final_layer.linear", cfg.mel, H)
    W["rand_noise"] = torch.randn(1, cfg.mel, cfg.noise_frames, generator=ini.g)
    return W


def init_hift(cfg: HiFTConfig = HiFTConfig(), seed: int = 0) -> dict[str, torch.Tensor]:
    ini = _Init(seed)
    W = {}
    c = cfg.f0_channels
    for i in range(cfg.f0_layers):
        ini.conv(W, f"f0_predictor.condnet.{2 * i}", c, cfg.mel if i == 0 else c, 3)
    ini.linear(W, "f0_predictor.classifier", 1, c, scale=400.0)
    W["f0_predictor.classifier.bias"] = W["f0_predictor.classifier.bias"].abs() + 20.0
    ini.linear(W, "m_source.l_linear", 1, cfg.harmonics + 1)
    ini.conv(W, "conv_pre", cfg.base, cfg.mel, 7)
    chans = [cfg.base] + cfg.stage_channels
    for i, (u, k) in enumerate(zip(cfg.up_rates, cfg.up_kernels)):
        ini.conv_t(W, f"ups.{i}", chans[i], chans[i + 1], k)
    nsrc = cfg.n_fft + 2
    for i, (u, k) in enumerate(zip(cfg.down_rates, cfg.src_res_kernels)):
        ch = cfg.stage_channels[i]
        ini.conv(W, f"source_downs.{i}", ch, nsrc, 1 if u == 1 else 2 * u)
        _resblock(ini, W, f"source_resblocks.{i}", ch, k, cfg.res_dilations)
    for i, ch in enumerate(cfg.stage_channels):
        for j, k in enumerate(cfg.res_kernels):
            _resblock(ini, W, f"resblocks.{i * len(cfg.res_kernels) + j}", ch, k, cfg.res_dilations)
    ini.conv(W, "conv_post", cfg.n_fft + 2, cfg.stage_channels[-1], 7)
    return W


def fold_weight_norm(sd: dict, snake_logscale: bool = False) -> dict[str, torch.Tensor]:
    """A HiFT state dict as the kernels take it: weight-normalised convolutions folded to their plain weight and Snake
    alphas made linear -- what ``make_lean`` does to the module once (``engine/runtime/hift_lean.py:107-134``).

    * ``<m>.parametrizations.weight.original0`` (g) / ``.original1`` (v) (``torch.nn.utils.parametrizations.weight_norm``)
      and ``<m>.weight_g`` / ``<m>.weight_v`` (the older ``torch.nn.utils.weight_norm``) become ``<m>.weight = g v / |v|``,
      the norm taken over every axis where g has size 1 -- torch's own ``_weight_norm``, so the weight equals the one
      ``remove_parametrizations(..., leave_parametrized=True)`` leaves, bit for bit.
    * ``snake_logscale``: the Snakes were built with ``alpha_logscale`` (a module attribute, not in the state dict), so
      every ``*.alpha`` becomes ``exp(alpha)``; the kernels then take ``1 / (alpha + 1e-9)`` of that, as the reference.
    * Every other entry is passed through (as a float32 tensor).  A plain dict folds to itself.
    """
    out: dict[str, torch.Tensor] = {}
    pairs: dict[str, dict[str, torch.Tensor]] = {}
    for k, v in sd.items():
        for tag, role in ((".parametrizations.weight.original0", "g"), (".parametrizations.weight.original1", "v"),
                          (".weight_g", "g"), (".weight_v", "v")):
            if k.endswith(tag) or k == tag[1:]:
                pairs.setdefault(k[: -len(tag)] if k.endswith(tag) else "", {})[role] = v
                break
        else:
            out[k] = v.detach().float()
    for base, gv in pairs.items():
        if set(gv) != {"g", "v"}:
            raise ValueError(f"weight norm of {base!r}: both the magnitude and the direction are needed, found {sorted(gv)}")
        g, v = gv["g"].detach().float(), gv["v"].detach().float()
        if g.dim() == v.dim() and g.numel() > 1:
            keep = [d for d in range(v.dim()) if g.shape[d] != 1]
            if len(keep) != 1 or g.shape[keep[0]] != v.shape[keep[0]]:
                raise ValueError(f"weight norm of {base!r}: magnitude {tuple(g.shape)} does not fit direction {tuple(v.shape)}")
            dim = keep[0]
        else:
            dim = -1  # one magnitude for the whole tensor
        name = base + ".weight" if base else "weight"
        if name in out:
            raise ValueError(f"{base!r} has both a plain weight and a weight norm")
        out[name] = torch._weight_norm(v, g.reshape(g.shape if dim >= 0 else ()), dim)
    if snake_logscale:
        for k in [k for k in out if k.endswith(".alpha")]:
            out[k] = torch.exp(out[k])
    return out


def _resblock(ini: _Init, W, p, ch, k, dils):
    for j, _ in enumerate(dils):
        ini.conv(W, f"{p}.convs1.{j}", ch, ch, k)
        ini.conv(W, f"{p}.convs2.{j}", ch, ch, k)
        W[f"{p}.activations1.{j}.alpha"] = 0.5 + torch.rand(ch, generator=ini.g)
        W[f"{p}.activations2.{j}.alpha"] = 0.5 + torch.rand(ch, generator=ini.g)


def init_flow(cfg: FlowConfig = FlowConfig(), seed: int = 0) -> dict[str, torch.Tensor]:
    """The flow's token embedding, encoder, ``encoder_proj`` and speaker affine layer.  Embedding rows are N(0, 1) (torch's
    default); ``pos_bias_u`` / ``pos_bias_v`` uniform in ``+-1/sqrt(head_dim)``."""
    ini = _Init(seed)
    C, W = cfg.dim, {}
    W["input_embedding.weight"] = torch.randn(cfg.vocab, C, generator=ini.g)
    ini.linear(W, "encoder.embed.out.0", C, C)
    ini.norm(W, "encoder.embed.out.1", C)
    ini.conv(W, "encoder.pre_lookahead_layer.conv1", C, C, cfg.look + 1)
    ini.conv(W, "encoder.pre_lookahead_layer.conv2", C, C, 3)
    for name, depth in (("encoders", cfg.depth1), ("up_encoders", cfg.depth2)):
        for i in range(depth):
            p = f"encoder.{name}.{i}."
            for n in ("linear_q", "linear_k", "linear_v", "linear_out"):
                ini.linear(W, p + "self_attn." + n, C, C)
            W[p + "self_attn.linear_pos.weight"] = ini.uniform((C, C), 1.0 / math.sqrt(C))
            W[p + "self_attn.pos_bias_u"] = ini.uniform((cfg.heads, cfg.head_dim), 1.0 / math.sqrt(cfg.head_dim))
            W[p + "self_attn.pos_bias_v"] = ini.uniform((cfg.heads, cfg.head_dim), 1.0 / math.sqrt(cfg.head_dim))
            ini.linear(W, p + "feed_forward.w_1", cfg.ffn, C)
            ini.linear(W, p + "feed_forward.w_2", C, cfg.ffn)
            ini.norm(W, p + "norm_mha", C)
            ini.norm(W, p + "norm_ff", C)
    ini.conv(W, "encoder.up_layer.conv", C, C, 2 * cfg.stride + 1)
    ini.linear(W, "encoder.up_embed.out.0", C, C)
    ini.norm(W, "encoder.up_embed.out.1", C)
    ini.norm(W, "encoder.after_norm", C)
    ini.linear(W, "encoder_proj", cfg.mel, C)
    ini.linear(W, "spk_embed_affine_layer", cfg.mel, cfg.spk)
    return W
