"""HiFT vocoder on the MI355X kernels (``t2w_hift_forward``): weights, call plan, workspace, streaming glue.

Host side of ``hift_forward_noise`` (``engine/models/token2wav.py:214-236``) and of the per-stream vocode glue
(``engine/runtime/token2wav_batch.py:813-848``, ``engine/models/token2wav.py:319-332``).  Rows may have different mel
lengths in one call (the reference groups equal lengths); activations are time-major and packed on the device.
Weights are the folded (weight-norm removed) fp32 tensors, conv weights re-laid to [Cout, taps, Cin] and transposed
convs split into their polyphase kernels [u, Cout, ceil(k / u), Cin].
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from .config import MEL_CACHE, SOURCE_CACHE, HiFTConfig
from .weights import fold_weight_norm


def chunk_noise_seed(noise_seed: int, chunk: int) -> int:
    """``engine/models/token2wav.py:108-109``."""
    return (noise_seed * 1_000_003 + chunk) & ((1 << 63) - 1)


# The convs the reference keeps in strict FP32 when it lets the upsampling stages run in TF32 (``decoder_tf32`` /
# ``tf32_stages``, engine/models/token2wav.py:42-55, 195-211): the input and output convs and stage 0's transposed conv.
REFERENCE_FP32_CONVS = ("conv_pre", "ups.0", "conv_post")


class HiFTModel:
    def __init__(self, W: dict, cfg: HiFTConfig = HiFTConfig(), device: str = "cuda", decode_bf16: bool = False,
                 use_graphs: bool = False, max_graphs: int = 32, fp32_convs: tuple = (), resblock_fusion: str = "auto",
                 snake_logscale: bool = False):
        """``W``: plain weights, or a checkpoint's state dict with weight-normalised convolutions (folded here by
        ``fold_weight_norm``; ``snake_logscale`` when its Snakes store log alphas).
        ``decode_bf16``: the decoder convs on bf16 MFMA (fp32 activations); f0 predictor and source stay fp32.
        ``resblock_fusion`` (bf16 only): each ResBlock dilation's two convs as one kernel that keeps the first conv's
        output on chip -- "auto" where the call's grid fills the chip, "on" wherever the channel count allows, "off"
        never (two convs through a scratch buffer).
        ``fp32_convs``: decoder convs that stay fp32 even then (``REFERENCE_FP32_CONVS``: the reference's split).
        ``use_graphs``: calls without overrides replay one captured graph per (row lengths, source-cache length), the
        role of ``HiFTGraphs`` (``engine/runtime/hift_graph.py:22-88``): inputs are copied into the graph's static
        buffers, outputs are returned as copies; at most ``max_graphs`` graphs are kept (least recently used dropped)."""
        W = fold_weight_norm(W, snake_logscale)
        self.cfg, self.device = cfg, device
        self.decode_bf16 = decode_bf16
        if resblock_fusion not in ("auto", "off", "on"):
            raise ValueError(f"resblock_fusion must be auto / off / on, not {resblock_fusion!r}")
        self._mode = {"auto": 1, "off": 2, "on": 3}[resblock_fusion] if decode_bf16 else 0
        self.use_graphs, self.max_graphs = use_graphs, max_graphs
        self.graphs: dict[tuple, dict] = {}
        self.counts = {"graph": 0, "eager": 0}
        f32 = lambda t: t.to(device=device, dtype=torch.float32).contiguous()  # noqa: E731
        self._keep = []

        def keep(t):
            t = f32(t)
            self._keep.append(t)
            return t.data_ptr()

        def keep_bf(w):  # [phases, Cout, taps, Cin] -> bf16, Cout and Cin zero-padded to multiples of 64
            ph, co, tp, ci = w.shape
            pad = torch.zeros(ph, -(-co // 64) * 64, tp, -(-ci // 64) * 64)
            pad[:, :co, :, :ci] = w
            t = pad.to(device=device, dtype=torch.bfloat16).contiguous()
            self._keep.append(t)
            return t.data_ptr()

        def conv(name, bf=True):
            w = W[name + ".weight"].permute(0, 2, 1).contiguous()  # [Cout, taps, Cin]
            return _lib.Conv(keep(w), keep(W[name + ".bias"]), keep_bf(w[None]) if bf and name not in fp32_convs else None)

        def conv_t(name, u):
            w = W[name + ".weight"]  # [Cin, Cout, k]
            cin, cout, k = w.shape
            taps = -(-k // u)
            wp = torch.zeros(u, cout, taps, cin)
            for ph in range(u):
                for m in range(taps):
                    j = ph + m * u
                    if j < k:
                        wp[ph, :, m, :] = w[:, :, j].t()
            return _lib.Conv(keep(wp), keep(W[name + ".bias"]), keep_bf(wp) if name not in fp32_convs else None)

        def resblock(p):
            rb = _lib.ResBlock()
            for j in range(3):
                rb.c1[j] = conv(f"{p}.convs1.{j}")
                rb.c2[j] = conv(f"{p}.convs2.{j}")
                for a, inv, key in ((rb.a1, rb.inv1, "activations1"), (rb.a2, rb.inv2, "activations2")):
                    alpha = W[f"{p}.{key}.{j}.alpha"].float()
                    a[j] = keep(alpha)
                    inv[j] = keep(1.0 / (alpha + 1e-9))
            return rb

        hw = _lib.HiftWeights()
        for i in range(cfg.f0_layers):
            hw.f0[i] = conv(f"f0_predictor.condnet.{2 * i}", bf=False)
        hw.f0_head_w = keep(W["f0_predictor.classifier.weight"][0])
        hw.f0_head_b = keep(W["f0_predictor.classifier.bias"])
        hw.src_w = keep(W["m_source.l_linear.weight"][0])
        hw.src_b = keep(W["m_source.l_linear.bias"])
        hw.conv_pre = conv("conv_pre")
        for i, u in enumerate(cfg.up_rates):
            hw.ups[i] = conv_t(f"ups.{i}", u)
            hw.src_down[i] = conv(f"source_downs.{i}", bf=False)
            hw.src_res[i] = resblock(f"source_resblocks.{i}")
        for i in range(9):
            hw.res[i] = resblock(f"resblocks.{i}")
        hw.conv_post = conv("conv_post")
        hw.window = keep(torch.hann_window(cfg.n_fft, periodic=True, dtype=torch.float32))
        self._w = hw
        dims = _lib.HiftDims(cfg.mel, cfg.base, len(cfg.up_rates), cfg.harmonics, cfg.f0_channels, cfg.f0_layers, cfg.sr, cfg.n_fft, cfg.hop,
                             (C.c_int * 3)(*cfg.up_rates), (C.c_int * 3)(*cfg.up_kernels), (C.c_int * 3)(*cfg.res_kernels),
                             (C.c_int * 3)(*cfg.res_dilations), (C.c_int * 3)(*cfg.src_res_kernels), cfg.sine_amp, cfg.noise_std,
                             cfg.voiced_threshold, cfg.lrelu_slope, cfg.audio_limit)
        h = C.c_void_p()
        _lib.check(_lib.lib().t2w_hift_create(C.byref(dims), C.byref(hw), C.byref(h)), "hift_create")
        self.handle = h
        self._ws = None
        self.dim = cfg.harmonics + 1

    def __del__(self):
        try:
            for g in getattr(self, "graphs", {}).values():
                _lib.lib().t2w_graph_destroy(g["graph"])
            if getattr(self, "handle", None) is not None:
                _lib.lib().t2w_hift_destroy(self.handle)
        except Exception:
            pass

    def noise(self, seeds: list[int], n_samples: int, noise_device: str = "cpu") -> tuple[torch.Tensor, torch.Tensor]:
        """Per-row source noise as the reference draws it (``hift_noise``, ``engine/models/token2wav.py:112-121``): row i
        takes ``rand(1, dim)`` then ``randn(1, dim, n)`` from a generator seeded ``seeds[i]`` on ``noise_device`` (the
        reference draws on the vocoder's device; "cpu" gives the host generator's stream, which the parity tests use),
        returned as (rand_ini [B, dim], noise [B, n, dim]) on the device."""
        gens = [torch.Generator(device=noise_device).manual_seed(int(x)) for x in seeds]
        rand_ini = torch.cat([torch.rand(1, self.dim, generator=g, device=noise_device) for g in gens])
        noise = torch.cat([torch.randn(1, self.dim, n_samples, generator=g, device=noise_device) for g in gens]).transpose(1, 2)
        return rand_ini.to(self.device), noise.to(self.device)

    @torch.inference_mode()
    def __call__(self, mel: torch.Tensor, cache_source: torch.Tensor, seeds: list[int], noise_device: str | None = None):
        """``HiFTGraphs.__call__(mel, cache_source, seeds)`` (``engine/runtime/hift_graph.py:62-88``): the rows' source
        noise drawn from their chunk seeds (on the vocoder's device, as the reference's ``hift_noise``, unless
        ``noise_device`` says otherwise), then ``forward_noise`` -- a captured graph per shape with ``use_graphs``.
        mel [B, 80, T], cache_source [B, 1, S] -> (speech [B, 480 T], source [B, 1, 480 T])."""
        if len(seeds) != mel.shape[0]:
            raise ValueError(f"{len(seeds)} seeds for {mel.shape[0]} rows")
        rand_ini, noise = self.noise(seeds, mel.shape[2] * self.cfg.upsample_scale, noise_device or str(mel.device))
        return self.forward_noise(mel, cache_source, rand_ini, noise)

    def _workspace(self, frames: list[int]) -> torch.Tensor:
        fr = (C.c_int * len(frames))(*frames)
        need = _lib.lib().t2w_hift_workspace_bytes(self.handle, len(frames), fr)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    @torch.inference_mode()
    def forward_packed(self, frames: list[int], mel_tm: torch.Tensor, noise_tm: torch.Tensor, cache_source: torch.Tensor | None, S: int,
                       f0_override=None, source_override=None, want_f0: bool = False):
        """Rows of ``frames[i]`` mel frames, packed time-major: mel [sum T, mel], noise [sum 480 T, dim], cache_source
        [n, S].  Returns (speech [sum 480 T], source [sum 480 T], f0 [sum T] or None)."""
        if self.use_graphs and f0_override is None and source_override is None and not want_f0:
            return self._forward_graph(frames, mel_tm, noise_tm, cache_source, S)
        self.counts["eager"] += 1
        L = _lib.lib()
        n = len(frames)
        fr = (C.c_int * n)(*frames)
        plan = (C.c_int * L.t2w_hift_plan_ints(n))()
        _lib.check(L.t2w_hift_plan(self.handle, n, fr, plan), "hift_plan")
        plan_dev = torch.from_numpy(np.ctypeslib.as_array(plan).copy()).to(self.device)
        ns = sum(frames) * self.cfg.upsample_scale
        speech = torch.empty(ns, device=self.device)
        source = torch.empty(ns, device=self.device)
        f0 = torch.empty(sum(frames), device=self.device) if want_f0 else None
        ws = self._workspace(frames)
        mel_tm = mel_tm.contiguous().float()
        noise_tm = noise_tm.contiguous().float()
        cs = cache_source.contiguous().float() if (cache_source is not None and S > 0) else None
        _lib.check(L.t2w_hift_forward(self.handle, n, fr, plan_dev.data_ptr(), mel_tm.data_ptr(), noise_tm.data_ptr(), _lib.ptr(cs), S,
                                      _lib.ptr(f0_override), _lib.ptr(source_override), speech.data_ptr(), source.data_ptr(), _lib.ptr(f0),
                                      ws.data_ptr(), ws.numel(), self._mode, _lib.stream_handle()), "hift_forward")
        return speech, source, f0

    def _graph(self, frames: list[int], S: int) -> dict:
        """The graph of a (row lengths, source-cache length) shape, captured on first use over its own static buffers;
        the least recently used one is dropped beyond ``max_graphs``."""
        L = _lib.lib()
        key = (tuple(frames), S)
        g = self.graphs.pop(key, None)
        if g is None:
            while len(self.graphs) >= self.max_graphs:
                old = self.graphs.pop(next(iter(self.graphs)))
                L.t2w_graph_destroy(old["graph"])
            n = len(frames)
            fr = (C.c_int * n)(*frames)
            plan = (C.c_int * L.t2w_hift_plan_ints(n))()
            _lib.check(L.t2w_hift_plan(self.handle, n, fr, plan), "hift_plan")
            ns = sum(frames) * self.cfg.upsample_scale
            dev = self.device
            g = {"fr": fr, "plan": torch.from_numpy(np.ctypeslib.as_array(plan).copy()).to(dev),
                 "mel": torch.zeros(sum(frames), self.cfg.mel, device=dev), "noise": torch.zeros(ns, self.dim, device=dev),
                 "cs": torch.zeros(n, S, device=dev) if S > 0 else None,
                 "speech": torch.empty(ns, device=dev), "source": torch.empty(ns, device=dev),
                 "ws": torch.empty(L.t2w_hift_workspace_bytes(self.handle, n, fr), dtype=torch.uint8, device=dev)}
            cap = self._capture_stream()  # capture needs a non-default stream; replays go on the caller's
            cap.wait_stream(torch.cuda.current_stream())
            cst = cap.cuda_stream
            _lib.check(L.t2w_graph_begin(cst), "graph_begin")
            rc = L.t2w_hift_forward(self.handle, n, g["fr"], g["plan"].data_ptr(), g["mel"].data_ptr(), g["noise"].data_ptr(),
                                    _lib.ptr(g["cs"]), S, None, None, g["speech"].data_ptr(), g["source"].data_ptr(), None,
                                    g["ws"].data_ptr(), g["ws"].numel(), self._mode, cst)
            h = C.c_void_p()
            rc2 = L.t2w_graph_end(cst, C.byref(h))
            _lib.check(rc, "hift_forward (capture)")
            _lib.check(rc2, "graph_end")
            torch.cuda.current_stream().wait_stream(cap)
            g["graph"] = h
        self.graphs[key] = g  # most recently used last
        return g

    def _forward_graph(self, frames: list[int], mel_tm: torch.Tensor, noise_tm: torch.Tensor, cache_source, S: int):
        g = self._graph(frames, S)
        g["mel"].copy_(mel_tm)
        g["noise"].copy_(noise_tm)
        if S > 0:
            g["cs"].copy_(cache_source.reshape(len(frames), S))
        _lib.check(_lib.lib().t2w_graph_launch(g["graph"], _lib.stream_handle()), "graph_launch")
        self.counts["graph"] += 1
        return g["speech"].clone(), g["source"].clone(), None

    def _capture_stream(self):
        if getattr(self, "_cap", None) is None:
            self._cap = torch.cuda.Stream()
        return self._cap

    def capture(self, frames: list[int], S: int) -> None:
        """Capture the graph of calls with rows of ``frames`` mel frames and ``S`` cached source samples now."""
        self._graph(list(frames), S)

    def capture_all(self, rows: int = 16, steady: int = MEL_CACHE + 50, first: int = 50) -> int:
        """The graphs of the streaming shapes (``HiFTGraphs.capture_all``, ``engine/runtime/hift_graph.py:52-57``): 1 to
        ``rows`` rows of steady windows (8 cached + 50 new frames, a 3840-sample source cache) and of first windows
        (no cache).  Returns the number of graphs held."""
        self.max_graphs = max(self.max_graphs, 2 * rows + 8)
        for n in range(1, rows + 1):
            self.capture([first] * n, 0)
            self.capture([steady] * n, SOURCE_CACHE)
        return len(self.graphs)

    @torch.inference_mode()
    def forward_noise(self, mel: torch.Tensor, cache_source: torch.Tensor, rand_ini: torch.Tensor, noise: torch.Tensor):
        """``hift_forward_noise`` (``engine/models/token2wav.py:214-236``): mel [B, 80, T], cache_source [B, 1, S],
        rand_ini [B, dim] (it never reaches the output: the frame-rate phase samples skip the first sample),
        noise [B, 480 T, dim] -> (speech [B, 480 T], source [B, 1, 480 T])."""
        B, _, T = mel.shape
        S = cache_source.shape[2]
        mel_tm = mel.permute(0, 2, 1).reshape(B * T, -1)
        noise_tm = noise.reshape(B * noise.shape[1], -1)
        sp, src, _ = self.forward_packed([T] * B, mel_tm, noise_tm, cache_source.reshape(B, S) if S else None, S)
        n = T * self.cfg.upsample_scale
        return sp.view(B, n), src.view(B, 1, n)


class HiftState:
    """A stream's HiFT cache (``engine/models/token2wav.py:319-332``): last 8 mel frames, 3840 source / speech samples."""

    def __init__(self, mel_dim: int = 80, noise_seed: int = 0, device: str = "cuda"):
        self.mel = torch.zeros(1, mel_dim, 0, device=device)
        self.source = torch.zeros(1, 1, 0, device=device)
        self.speech = torch.zeros(1, 0, device=device)
        self.chunks = 0
        self.noise_seed = noise_seed


def fade_in_out(fade_in: torch.Tensor, fade_out: torch.Tensor, window: torch.Tensor) -> torch.Tensor:
    """``engine/models/token2wav.py:81-85``: the first half-window of ``fade_in`` cross-faded with the last of
    ``fade_out`` (the float64 Hamming window as the reference's)."""
    n = int(window.shape[0] / 2)
    out = fade_in.clone()
    out[..., :n] = fade_in[..., :n] * window[:n] + fade_out[..., -n:] * window[n:]
    return out
