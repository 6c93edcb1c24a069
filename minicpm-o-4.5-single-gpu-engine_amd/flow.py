"""The flow encoder on the MI355X kernels: codec tokens -> ``mu`` for many streams' windows in one packed call.

Mirrors the reference's batched encoder (``BatchedToken2Wav._flow_encode`` / ``_encoder`` / ``_encoder_core``,
``engine/runtime/token2wav_batch.py:42-79, 365-444``; the prompt setup's ``_setup_encoder_one`` / ``_setup_encoder_batched``,
``:556-616``) with this build's own state layout:

* Every layer's keys and values live in fp16 slot pools (one slot = one frame, 2 x 512 values per layer).  A frame's
  keys never change once written, so a stream's cache is two lists of slot ids (first stack, second stack) and slots are
  reference counted: a stream made from a prompt shares the prompt's slots, and a trim is a list operation.  The lists
  follow the reference's packed cache exactly: after a kept window the first stack's list is the first half of
  ``trim(list1 + list1)`` (the reference tiles it twice along time and reads the first half) and the second stack's
  ``trim(list2)``, where ``trim`` keeps the first ``keep`` (the prompt's mel frames) and the last 100 entries.
* The two conv caches (two conv1 outputs of the pre-lookahead layer, four upsampled frames) are one slot of a bf16
  pool; a call reads a stream's slot and writes a fresh one, so slots are immutable too.
* Weights-only work is done once: the embed Linear folded into the embedding table, the up_embed Linear composed into
  the upsampling conv, and ``linear_pos`` of the sinusoid tabulated per layer for relative positions +-(rmax - 1).

Windows of any token counts, final or not, ride one call (the reference groups them by count and flag).
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .config import SILENCE_TOKEN, TRIM_SUFFIX, FlowConfig
from .dit import SlotPool, _Upload


C_ref = ctypes.byref


class RefPool(SlotPool):
    """Slot ids with reference counts: a slot goes back to the free stack when no list holds it."""

    def __init__(self, n: int, reserved: int = 0):
        self.ref = np.zeros(int(n), dtype=np.int32)
        super().__init__(n, reserved)

    def alloc(self, k: int) -> np.ndarray:
        ids = super().alloc(k)
        self.ref[ids] = 1
        return ids

    def hold(self, ids) -> None:
        np.add.at(self.ref, np.asarray(ids, dtype=np.int64), 1)

    def drop(self, ids) -> None:
        ids = np.asarray(ids, dtype=np.int64)
        if ids.size == 0:
            return
        np.add.at(self.ref, ids, -1)
        u = np.unique(ids)
        if (self.ref[u] < 0).any():
            raise RuntimeError("flow encoder: slot released more often than held")
        self.release(u[self.ref[u] == 0])


@dataclass
class FlowState:
    """A stream's encoder caches: first- and second-stack key slot lists (time order), its conv-cache slot (0: the
    zero slot of an empty cache) and the trim length ``keep``."""
    k1: np.ndarray
    k2: np.ndarray
    cnn: int
    keep: int


def _trim(ids: np.ndarray, keep: int) -> np.ndarray:
    if ids.size > keep + TRIM_SUFFIX:
        return np.concatenate([ids[:keep], ids[ids.size - TRIM_SUFFIX:]])
    return ids


def rel_sinusoid(rmax: int, dim: int) -> torch.Tensor:
    """[2 rmax - 1, dim] float64: row r + rmax - 1 is the sinusoid of relative position r (sin at even columns, cos at
    odd, frequencies 10000^(-2i / dim))."""
    r = torch.arange(-(rmax - 1), rmax, dtype=torch.float64)[:, None]
    div = torch.exp(torch.arange(0, dim, 2, dtype=torch.float64) * -(math.log(10000.0) / dim))
    pe = torch.zeros(2 * rmax - 1, dim, dtype=torch.float64)
    pe[:, 0::2] = torch.sin(r * div)
    pe[:, 1::2] = torch.cos(r * div)
    return pe


class FlowModel:
    """Device weights of the flow encoder (token embedding, encoder, ``encoder_proj``, speaker affine layer) and the C
    model object."""

    def __init__(self, W: dict, cfg: FlowConfig = FlowConfig(), device: str = "cuda"):
        self.cfg, self.device = cfg, torch.device(device)
        C, dev = cfg.dim, self.device
        if C % 512 or cfg.heads * 64 != C:
            raise ValueError("the flow encoder kernels need a width that is a multiple of 512 and heads of 64")
        f32 = lambda k: W[k].to(dev, torch.float32).contiguous()  # noqa: E731
        bf = lambda t: t.to(torch.bfloat16).contiguous()  # noqa: E731
        taps = lambda w: w.permute(0, 2, 1).reshape(w.shape[0], -1)  # [out, in, k] -> [out, k in], frame-major  # noqa: E731
        with torch.no_grad():
            table = f32("input_embedding.weight") @ f32("encoder.embed.out.0.weight").t() + f32("encoder.embed.out.0.bias")
            wl, wc = f32("encoder.up_embed.out.0.weight"), f32("encoder.up_layer.conv.weight")
            up_w = torch.einsum("oc,cik->oki", wl, wc).reshape(C, -1)
            up_b = wl @ f32("encoder.up_layer.conv.bias") + f32("encoder.up_embed.out.0.bias")
            pe = rel_sinusoid(cfg.rmax, C).to(dev, torch.float32)
            self.g = {
                "embed_table": table.contiguous(), "embed_ln_w": f32("encoder.embed.out.1.weight"), "embed_ln_b": f32("encoder.embed.out.1.bias"),
                "conv1_w": bf(taps(f32("encoder.pre_lookahead_layer.conv1.weight"))), "conv1_b": f32("encoder.pre_lookahead_layer.conv1.bias"),
                "conv2_w": bf(taps(f32("encoder.pre_lookahead_layer.conv2.weight"))), "conv2_b": f32("encoder.pre_lookahead_layer.conv2.bias"),
                "up_w": bf(up_w), "up_b": up_b.contiguous(),
                "up_ln_w": f32("encoder.up_embed.out.1.weight"), "up_ln_b": f32("encoder.up_embed.out.1.bias"),
                "after_w": f32("encoder.after_norm.weight"), "after_b": f32("encoder.after_norm.bias"),
                "proj_w": bf(f32("encoder_proj.weight")), "proj_b": f32("encoder_proj.bias"),
                "spk_w": f32("spk_embed_affine_layer.weight"), "spk_b": f32("spk_embed_affine_layer.bias"),
                "ones": torch.ones(C, dtype=torch.float32, device=dev),
            }
            self.layers = []
            for i in range(cfg.depth1 + cfg.depth2):
                p = f"encoder.encoders.{i}." if i < cfg.depth1 else f"encoder.up_encoders.{i - cfg.depth1}."
                a = p + "self_attn."
                self.layers.append({
                    "qkv_w": bf(torch.cat([f32(a + n + ".weight") for n in ("linear_q", "linear_k", "linear_v")])),
                    "qkv_b": torch.cat([f32(a + n + ".bias") for n in ("linear_q", "linear_k", "linear_v")]).contiguous(),
                    "pos_u": f32(a + "pos_bias_u").reshape(-1).contiguous(), "pos_v": f32(a + "pos_bias_v").reshape(-1).contiguous(),
                    "ptab": (pe @ f32(a + "linear_pos.weight").t()).to(torch.float16).contiguous(),
                    "out_w": bf(f32(a + "linear_out.weight")), "out_b": f32(a + "linear_out.bias"),
                    "ln1_w": f32(p + "norm_mha.weight"), "ln1_b": f32(p + "norm_mha.bias"),
                    "ln2_w": f32(p + "norm_ff.weight"), "ln2_b": f32(p + "norm_ff.bias"),
                    "w1": bf(f32(p + "feed_forward.w_1.weight")), "b1": f32(p + "feed_forward.w_1.bias"),
                    "w2": bf(f32(p + "feed_forward.w_2.weight")), "b2": f32(p + "feed_forward.w_2.bias"),
                })
        L = _lib.lib()
        dims = _lib.FlowDims(cfg.vocab, C, cfg.heads, cfg.ffn, cfg.depth1, cfg.depth2, cfg.look, cfg.stride, cfg.mel, cfg.spk, cfg.rmax,
                             cfg.eps_layer, cfg.eps_embed, cfg.eps_after)
        h = _lib.P()
        _lib.check(L.t2w_flow_create(C_ref(dims), C_ref(h)), "flow create")
        self.handle = h
        for i, lw in enumerate(self.layers):
            s = _lib.FlowLayer(**{k: v.data_ptr() for k, v in lw.items()})
            _lib.check(L.t2w_flow_set_layer(h, i, C_ref(s)), "flow layer")
        _lib.check(L.t2w_flow_set_globals(h, C_ref(_lib.FlowGlobals(**{k: v.data_ptr() for k, v in self.g.items()}))), "flow globals")

    def __del__(self):
        h = getattr(self, "handle", None)
        if h:
            _lib.lib().t2w_flow_destroy(h)
            self.handle = None

    def speaker(self, spk: torch.Tensor) -> torch.Tensor:
        """``spk_embed_affine_layer(F.normalize(spk))``: [R, spk] -> [R, mel] fp32."""
        spk = spk.to(self.device, torch.float32).reshape(-1, self.cfg.spk).contiguous()
        out = torch.empty(spk.shape[0], self.cfg.mel, dtype=torch.float32, device=self.device)
        _lib.check(_lib.lib().t2w_flow_speaker(self.handle, spk.data_ptr(), out.data_ptr(), spk.shape[0], _lib.stream_handle()), "flow speaker")
        return out


class FlowEncoder:
    """Stream caches of the flow encoder and its packed call.  ``n_slots1`` / ``n_slots2``: frames per first / second
    stack pool (each stream's lists hold about keep / 2 + 75 and keep + 150 of them); ``n_cnn``: conv-cache slots.

    ``use_graphs``: window calls replay a captured hipGraph of the whole encoder call (the role of ``EncoderGraphs``,
    ``engine/runtime/dit_graph.py:210-352``), one per call shape -- the row count and the packed row totals, which fix
    every launch of the call; the rows' tables go to the graph's own device arena before each replay (the key lists at
    a fixed capacity of ``rmax`` keys per row, so their lengths do not enter the shape), and ``mu`` is copied out of the
    graph's output buffer.  Prompt setups run eagerly.  At most ``max_graphs`` shapes are kept (least recently used
    dropped)."""

    VAR_TABLES = ("kv1_idx", "kv2_idx")  # tables whose length is not fixed by the call's shape

    def __init__(self, model: FlowModel, n_slots1: int = 32768, n_slots2: int = 65536, n_cnn: int = 4096, use_graphs: bool = False,
                 max_graphs: int = 16):
        cfg, dev = model.cfg, model.device
        self.model, self.cfg, self.device = model, cfg, dev
        C = cfg.dim
        self.pool1 = torch.zeros(cfg.depth1, n_slots1, 2 * C, dtype=torch.float16, device=dev)
        self.pool2 = torch.zeros(cfg.depth2, n_slots2, 2 * C, dtype=torch.float16, device=dev)
        self.cnn_pool = torch.zeros(n_cnn, cfg.cnn_frames, C, dtype=torch.bfloat16, device=dev)
        self.p1, self.p2 = RefPool(n_slots1), RefPool(n_slots2)
        self.pc = RefPool(n_cnn, reserved=1)  # slot 0 stays zero: the empty cache
        self.zero_cnn = int(self.pc.reserved[0])
        self._ws = None
        self.use_graphs, self.max_graphs = use_graphs, max_graphs
        self.graphs: dict[tuple, dict] = {}
        self.counts = {"graph": 0, "eager": 0}
        self._cap = None

    def __del__(self):
        try:
            self.drop_graphs()
        except Exception:
            pass

    # --- states -------------------------------------------------------------------------------------------------------
    def new_state(self, keep: int) -> FlowState:
        e = np.zeros(0, dtype=np.int32)
        return FlowState(e, e.copy(), self.zero_cnn, int(keep))

    def clone(self, st: FlowState) -> FlowState:
        """Another stream from the same caches (shares the slots)."""
        self.p1.hold(st.k1)
        self.p2.hold(st.k2)
        if st.cnn != self.zero_cnn:
            self.pc.hold([st.cnn])
        return FlowState(st.k1.copy(), st.k2.copy(), st.cnn, st.keep)

    def release(self, st: FlowState | None) -> None:
        if st is None or st.k1 is None:
            return
        self.p1.drop(st.k1)
        self.p2.drop(st.k2)
        if st.cnn != self.zero_cnn:
            self.pc.drop([st.cnn])
        st.k1 = st.k2 = None

    def in_use(self) -> tuple[int, int, int]:
        return self.p1.in_use(), self.p2.in_use(), self.pc.in_use() - 1

    # --- the packed call --------------------------------------------------------------------------------------------------
    def _workspace(self, n_in, n_gap, n1, n_up, n2) -> torch.Tensor:
        need = int(_lib.lib().t2w_flow_workspace_bytes(self.model.handle, n_in, n_gap, n1, n_up, n2))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=self.device)
        return self._ws

    # --- graphs -----------------------------------------------------------------------------------------------------
    def _graph_layout(self, parts: dict, R: int) -> tuple[dict, int]:
        """Offsets of the call's tables in a graph arena: the tables whose sizes the call shape fixes, in order, then the
        two key lists at ``R * rmax`` entries each."""
        offs, o = {}, 0
        for k, v in parts.items():
            if k not in self.VAR_TABLES:
                offs[k] = o
                o += max(int(np.asarray(v).size), 1)
        for k in self.VAR_TABLES:
            offs[k] = o
            o += R * self.cfg.rmax
        return offs, o

    def _flow_args(self, shape: tuple, base: int, offs: dict, keys, ws: torch.Tensor, mu: torch.Tensor) -> "_lib.FlowArgs":
        return _lib.FlowArgs(*shape, *[base + 4 * offs[k] for k in keys], self.pool1.data_ptr(), self.pool1[0].numel(),
                             self.pool2.data_ptr(), self.pool2[0].numel(), self.cnn_pool.data_ptr(), mu.data_ptr(), ws.data_ptr(),
                             ws.numel())

    def _graph_call(self, shape: tuple, parts: dict) -> torch.Tensor:
        """Replay (capturing on first use) the graph of a call of this ``shape`` = (R, n_in, n_gap, n1, n_up, n2,
        tiles1, tiles2) with the call's tables; returns a copy of its mu [n2, mel]."""
        L = _lib.lib()
        R, n2 = shape[0], shape[5]
        g = self.graphs.pop(shape, None)
        if g is None:
            while len(self.graphs) >= self.max_graphs:
                L.t2w_graph_destroy(self.graphs.pop(next(iter(self.graphs)))["graph"])
            offs, size = self._graph_layout(parts, R)
            need = int(L.t2w_flow_workspace_bytes(self.model.handle, *shape[1:6]))
            g = {"offs": offs, "arena": torch.zeros(size, dtype=torch.int32, device=self.device),
                 "ws": torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=self.device),
                 "mu": torch.empty(n2, self.cfg.mel, dtype=torch.float32, device=self.device), "graph": None}
        host = np.zeros(g["arena"].numel(), dtype=np.int32)
        for k, v in parts.items():
            v = np.asarray(v)
            host[g["offs"][k]:g["offs"][k] + v.size] = v
        _Upload.into(g["arena"], host)
        if g["graph"] is None:
            if self._cap is None:
                self._cap = torch.cuda.Stream()
            self._cap.wait_stream(torch.cuda.current_stream())
            cst = self._cap.cuda_stream
            args = self._flow_args(shape, g["arena"].data_ptr(), g["offs"], parts, g["ws"], g["mu"])
            _lib.check(L.t2w_graph_begin(cst), "graph_begin")
            rc = L.t2w_flow_encode(self.model.handle, C_ref(args), cst)
            h = _lib.P()
            rc2 = L.t2w_graph_end(cst, C_ref(h))
            _lib.check(rc, "flow encode (capture)")
            _lib.check(rc2, "graph_end")
            torch.cuda.current_stream().wait_stream(self._cap)
            g["graph"] = h
        self.graphs[shape] = g  # most recently used last
        _lib.check(L.t2w_graph_launch(g["graph"], _lib.stream_handle()), "graph_launch")
        self.counts["graph"] += 1
        return g["mu"].clone()

    def drop_graphs(self) -> None:
        for g in self.graphs.values():
            if g["graph"] is not None:
                _lib.lib().t2w_graph_destroy(g["graph"])
        self.graphs = {}

    @torch.inference_mode()
    def encode(self, states: list[FlowState], windows: list, lasts: list[bool], graph: bool | None = None
               ) -> tuple[torch.Tensor, list[int], list[int]]:
        """One call over every stream's window (token lists; a non-final window carries ``look`` lookahead tokens at its
        end).  Returns (mu [sum T2, mel] fp32 on the device, each stream's first row, each stream's T2) and advances the
        states (a final window's state is released).  ``graph``: replay a captured graph of the call's shape (default
        ``use_graphs``)."""
        cfg = self.cfg
        look, s, C = cfg.look, cfg.stride, cfg.dim
        R = len(states)
        toks = [np.asarray(w, dtype=np.int64).ravel() for w in windows]
        T1 = np.array([t.size if last else t.size - look for t, last in zip(toks, lasts)], dtype=np.int64)
        if R == 0:
            return torch.zeros(0, cfg.mel, device=self.device), [], []
        if (T1 < 1).any():
            raise ValueError("flow encoder: a window needs at least one frame (a non-final window more than the lookahead tokens)")
        for t in toks:
            if t.size and (t.min() < 0 or t.max() >= cfg.vocab):
                raise ValueError(f"flow encoder: token ids must be in [0, {cfg.vocab})")
        T2 = s * T1
        L1 = np.array([st.k1.size for st in states], dtype=np.int64) + T1
        L2 = np.array([st.k2.size for st in states], dtype=np.int64) + T2
        if L1.max() > cfg.rmax or L2.max() > cfg.rmax:
            raise ValueError(f"flow encoder: {int(max(L1.max(), L2.max()))} keys exceed the relative-position table (rmax {cfg.rmax})")
        n1, n2 = int(T1.sum()), int(T2.sum())
        n_in, n_gap, n_up = n1 + look * R, n1 + 2 * R, n2 + 2 * s * R
        new1 = self.p1.alloc(n1)
        new2 = wr = None
        try:  # every slot this call takes goes back if anything before the kernels' launch fails
            new2 = self.p2.alloc(n2)
            wr = self.pc.alloc(R)
            cs = lambda n: np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)  # noqa: E731
            in0, g0, o1, u0, o2 = cs(T1 + look), cs(T1 + 2), cs(T1), cs(T2 + 2 * s), cs(T2)
            sid1 = np.repeat(np.arange(R), T1)            # stream of each stack-1 row
            t_in1 = np.arange(n1) - o1[sid1]              # its frame index
            sid2 = np.repeat(np.arange(R), T2)
            f2 = np.arange(n2) - o2[sid2]
            # conv1 input rows: the window's tokens (a final window: then `look` zero rows); h1 rows for the first T1
            tok = np.full(n_in, -1, dtype=np.int64)
            res = np.full(n_in, -1, dtype=np.int64)
            for r in range(R):
                tok[in0[r]:in0[r] + toks[r].size] = toks[r]
                res[in0[r]:in0[r] + T1[r]] = np.arange(o1[r], o1[r] + T1[r])
            c1_src = np.repeat(in0, T1 + 2)
            gi = np.arange(n_gap) - np.repeat(g0, T1 + 2)  # position in the stream's gapped block: 0, 1 cache, then frames
            c1_src = c1_src + np.maximum(gi - 2, 0)
            c2_src = g0[sid1] + t_in1
            up_dst = u0[sid1] + 2 * s + s * t_in1
            up_src = u0[sid2] + f2
            kv1 = np.concatenate([np.concatenate([st.k1, new1[o1[r]:o1[r] + T1[r]]]) for r, st in enumerate(states)])
            kv2 = np.concatenate([np.concatenate([st.k2, new2[o2[r]:o2[r] + T2[r]]]) for r, st in enumerate(states)])
            kv1_off, kv2_off = cs(L1), cs(L2)
            tiles1 = np.array([(r, q) for r in range(R) for q in range(0, int(T1[r]), 32)], dtype=np.int64).reshape(-1, 2)
            tiles2 = np.array([(r, q) for r in range(R) for q in range(0, int(T2[r]), 32)], dtype=np.int64).reshape(-1, 2)
            rd = np.array([st.cnn for st in states], dtype=np.int64)
            parts = {"tok": tok, "res": res, "c1_src": c1_src, "gofs": g0, "t1": T1, "c2_src": c2_src, "up_dst": up_dst, "uofs": u0,
                     "o1": o1, "up_src": up_src, "o2": o2, "t2": T2, "cnn_rd": rd, "cnn_wr": wr, "new1": new1, "new2": new2,
                     "kv1_idx": kv1, "kv1_off": kv1_off, "kv1_len": L1, "tiles1": tiles1.ravel(), "kv2_idx": kv2, "kv2_off": kv2_off,
                     "kv2_len": L2, "tiles2": tiles2.ravel()}
            shape = (R, n_in, n_gap, n1, n_up, n2, tiles1.shape[0], tiles2.shape[0])
            if self.use_graphs if graph is None else graph:
                mu = self._graph_call(shape, parts)
            else:
                offs, o = {}, 0
                for k, v in parts.items():
                    offs[k] = o
                    o += max(int(np.asarray(v).size), 1)
                host = np.zeros(o, dtype=np.int32)
                for k, v in parts.items():
                    host[offs[k]:offs[k] + np.asarray(v).size] = v
                meta = _Upload.new(host, self.device)
                ws = self._workspace(n_in, n_gap, n1, n_up, n2)
                mu = torch.empty(n2, cfg.mel, dtype=torch.float32, device=self.device)
                args = self._flow_args(shape, meta.data_ptr(), offs, parts, ws, mu)
                _lib.check(_lib.lib().t2w_flow_encode(self.model.handle, C_ref(args), _lib.stream_handle()), "flow encode")
                self.counts["eager"] += 1
        except Exception:
            self.p1.drop(new1)
            if new2 is not None:
                self.p2.drop(new2)
            if wr is not None:
                self.pc.drop(wr)
            raise
        # advance the lists: [cache, new]; the first stack as the first half of the trimmed tiled list
        for r, st in enumerate(states):
            c1 = kv1[kv1_off[r]:kv1_off[r] + L1[r]]
            c2 = kv2[kv2_off[r]:kv2_off[r] + L2[r]]
            old1, old2, oldc = st.k1, st.k2, st.cnn
            if lasts[r]:
                st.k1, st.k2, st.cnn = np.zeros(0, np.int32), np.zeros(0, np.int32), self.zero_cnn
            else:
                p1 = _trim(np.concatenate([c1, c1]), st.keep)
                st.k1 = p1[: p1.size // 2].astype(np.int32)
                st.k2 = _trim(c2, st.keep).astype(np.int32)
                st.cnn = int(wr[r])
                self.p1.hold(st.k1)
                self.p2.hold(st.k2)
                self.pc.hold([st.cnn])
            self.p1.drop(old1)
            self.p2.drop(old2)
            if oldc != self.zero_cnn:
                self.pc.drop([oldc])
        # the call's own references to its new slots
        self.p1.drop(new1)
        self.p2.drop(new2)
        self.pc.drop(wr)
        return mu, [int(x) for x in o2], [int(x) for x in T2]

    def setup(self, prompts: list) -> tuple[list[FlowState], torch.Tensor, list[int], list[int]]:
        """Prompt setups in one call: each prompt's tokens plus ``look`` silence tokens through an empty cache, not final
        (``_setup_encoder_one``, ``token2wav_batch.py:556-565``).  Returns (states with keep = stride x tokens, mu, first
        rows, frames)."""
        cfg = self.cfg
        toks = [np.asarray(p, dtype=np.int64).ravel() for p in prompts]
        states = [self.new_state(cfg.stride * t.size) for t in toks]
        windows = [np.concatenate([t, np.full(cfg.look, SILENCE_TOKEN, dtype=np.int64)]) for t in toks]
        try:
            mu, rows, frames = self.encode(states, windows, [False] * len(states), graph=False)
        except Exception:
            for st in states:
                self.release(st)
            raise
        return states, mu, rows, frames
