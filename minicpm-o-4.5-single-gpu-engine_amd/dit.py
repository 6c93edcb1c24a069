"""The DiT estimator and its CFG Euler solve on the MI355X kernels: weights, streaming key/conv state, call planning.

Host side of ``t2w_dit_solve`` (``include/t2w.h``).  It mirrors the reference's fast solve
(``engine/runtime/dit_fast.py:99-495``): packed ragged rows ``[cond rows | uncond rows]``, one key slot per cached frame
in a shared pool per (Euler step, block), the reference's tensor order kept as a host list of slot ids so trimming
evicts the same frames (``:480-490``), conv caches of two frames per (step, block, row) in row slots.  Differences by
design: the residual stream and the Euler state are fp32 (bf16 GEMM operands), the key pool is bf16, conv caches are
double-buffered per row (read one slot, write the other, swap after a kept window) so no staging copy is needed, and
the attention's per-row key lists and 64-query tiles are planned here and uploaded with the other tables in one copy.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .config import TRIM_SUFFIX, DiTConfig

MAX_STEPS = 16


def t_schedule(steps: int) -> tuple[list[float], list[float]]:
    """t and dt of each Euler step: ``t_span = 1 - cos(linspace(0, 1, steps + 1) pi / 2)``, ``t += dt``,
    ``dt = t_span[k + 1] - t`` in fp32 (``engine/runtime/dit_fast.py:161-178``; fp32 instead of the flow's fp16)."""
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
    return torch.exp(-np.log(max_period) * torch.arange(0, half, dtype=torch.float32) / half)


def quantize_e4m3(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel fp8 weights (the reference's fp8 convention, ``engine/runtime/fp8.py:15-37``): scale
    max|w_n| / 448, codes = round-to-nearest-even e4m3 of w / scale.  w [N, K] -> (uint8 codes [N, K], fp32 scales [N])."""
    wf = w.float()
    sc = (wf.abs().amax(dim=1) / 448.0).clamp_min(1e-30)
    q = (wf / sc[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    return q.contiguous(), sc.contiguous()


class DiTModel:
    """Weights on the GPU (bf16 GEMM operands, fp32 biases / norm affines) and the per-step adaLN tables.  With
    ``fp8`` the six block GEMMs also get e4m3 weights (per-output-channel scales) for fp8 solves."""

    def __init__(self, W: dict, cfg: DiTConfig = DiTConfig(), device: str = "cuda", fp8: bool = False):
        self.cfg, self.device = cfg, device
        H, D = cfg.hidden, cfg.depth
        bf = lambda t: t.to(device=device, dtype=torch.bfloat16).contiguous()  # noqa: E731
        f32 = lambda t: t.to(device=device, dtype=torch.float32).contiguous()  # noqa: E731
        self.t = {"in_w": bf(W["in_proj.weight"]), "in_b": f32(W["in_proj.bias"]),
                  "out_w": bf(W["final_layer.linear.weight"]), "out_b": f32(W["final_layer.linear.bias"])}
        self.blocks = []
        for b in range(D):
            p = f"blocks.{b}."
            a = p + "attn."
            conv = lambda w: bf(w.permute(0, 2, 1).reshape(w.shape[0], -1))  # noqa: E731  [out, k * in], frame-major
            self.blocks.append({
                "qkv_w": bf(torch.cat([W[a + "to_q.weight"], W[a + "to_k.weight"], W[a + "to_v.weight"]])),
                "qkv_b": f32(torch.cat([W[a + "to_q.bias"], W[a + "to_k.bias"], W[a + "to_v.bias"]])),
                "qn_w": f32(W[a + "q_norm.weight"]), "qn_b": f32(W[a + "q_norm.bias"]),
                "kn_w": f32(W[a + "k_norm.weight"]), "kn_b": f32(W[a + "k_norm.bias"]),
                "proj_w": bf(W[a + "proj.weight"]), "proj_b": f32(W[a + "proj.bias"]),
                "c1_w": conv(W[p + "conv.block.1.weight"]), "c1_b": f32(W[p + "conv.block.1.bias"]),
                "cln_w": f32(W[p + "conv.block.3.weight"]), "cln_b": f32(W[p + "conv.block.3.bias"]),
                "c2_w": conv(W[p + "conv.block.6.weight"]), "c2_b": f32(W[p + "conv.block.6.bias"]),
                "fc1_w": bf(W[p + "mlp.fc1.weight"]), "fc1_b": f32(W[p + "mlp.fc1.bias"]),
                "fc2_w": bf(W[p + "mlp.fc2.weight"]), "fc2_b": f32(W[p + "mlp.fc2.bias"])})
        self.rand_noise = f32(W["rand_noise"][0])  # [mel, frames]
        L = _lib.lib()
        dims = _lib.DitDims(cfg.mel, H, D, cfg.heads, cfg.head_dim, cfg.ffn, cfg.freq, cfg.steps, cfg.eps_block, cfg.eps_qk,
                            cfg.eps_conv, cfg.eps_final, cfg.cfg_rate)
        h = C.c_void_p()
        _lib.check(L.t2w_dit_create(C.byref(dims), C.byref(h)), "dit_create")
        self.handle = h
        for b, blk in enumerate(self.blocks):
            s = _lib.DitBlock(*[blk[n].data_ptr() for n, _ in _lib.DitBlock._fields_])
            _lib.check(L.t2w_dit_set_block(h, b, C.byref(s)), "set_block")
        self.fp8 = fp8
        self.blocks8 = []
        if fp8:
            for b in range(D):
                p = f"blocks.{b}."
                a = p + "attn."
                src = {"qkv": torch.cat([W[a + "to_q.weight"], W[a + "to_k.weight"], W[a + "to_v.weight"]]),
                       "proj": W[a + "proj.weight"],
                       "c1": W[p + "conv.block.1.weight"].permute(0, 2, 1).reshape(H, -1),
                       "c2": W[p + "conv.block.6.weight"].permute(0, 2, 1).reshape(H, -1),
                       "fc1": W[p + "mlp.fc1.weight"], "fc2": W[p + "mlp.fc2.weight"]}
                blk8 = {}
                for k, w in src.items():
                    q, sc = quantize_e4m3(w.to(device))
                    blk8[k + "_w8"], blk8[k + "_ws"] = q, sc
                self.blocks8.append(blk8)
                s8 = _lib.DitBlockFp8(*[blk8[n].data_ptr() for n, _ in _lib.DitBlockFp8._fields_])
                _lib.check(L.t2w_dit_set_block_fp8(h, b, C.byref(s8)), "set_block_fp8")
        self.ts, self.dts = t_schedule(cfg.steps)
        # timestep / adaLN tables of the schedule, computed on the GPU from fp32 copies of those weights
        self._mod_w = {"freqs": f32(freq_table(cfg.freq)), "te0_w": f32(W["t_embedder.mlp.0.weight"]), "te0_b": f32(W["t_embedder.mlp.0.bias"]),
                       "te2_w": f32(W["t_embedder.mlp.2.weight"]), "te2_b": f32(W["t_embedder.mlp.2.bias"]),
                       "ada_w": f32(torch.cat([W[f"blocks.{b}.adaLN_modulation.1.weight"] for b in range(D)])),
                       "ada_b": f32(torch.cat([W[f"blocks.{b}.adaLN_modulation.1.bias"] for b in range(D)])),
                       "fin_w": f32(W["final_layer.adaLN_modulation.1.weight"]), "fin_b": f32(W["final_layer.adaLN_modulation.1.bias"])}
        self.mods, self.final_mods = self.tables(self.ts)
        self._dts = (C.c_float * cfg.steps)(*self.dts)
        g = _lib.DitGlobals(self.t["in_w"].data_ptr(), self.t["in_b"].data_ptr(), self.t["out_w"].data_ptr(), self.t["out_b"].data_ptr(),
                            self.mods.data_ptr(), self.final_mods.data_ptr(), C.cast(self._dts, _lib.FP))
        _lib.check(L.t2w_dit_set_globals(h, C.byref(g)), "set_globals")

    def tables(self, ts: list[float]) -> tuple[torch.Tensor, torch.Tensor]:
        """adaLN tables for the given t values: mods [S, depth, 9, H] (shift, 1 + scale, gate of msa, mlp, conv) and
        final [S, 2, H] (``engine/runtime/dit_fast.py:157-178``)."""
        cfg, L = self.cfg, _lib.lib()
        S, H, D = len(ts), cfg.hidden, cfg.depth
        assert 0 < S <= MAX_STEPS
        mods = torch.empty(S, D, 9, H, device=self.device)
        fin = torch.empty(S, 2, H, device=self.device)
        tsd = torch.tensor(ts, dtype=torch.float32, device=self.device)
        ws = torch.empty(L.t2w_dit_mods_workspace_bytes(self.handle, S), dtype=torch.uint8, device=self.device)
        mw = _lib.ModWeights(*[self._mod_w[n].data_ptr() for n, _ in _lib.ModWeights._fields_])
        _lib.check(L.t2w_dit_build_mods(self.handle, C.byref(mw), tsd.data_ptr(), S, mods.data_ptr(), fin.data_ptr(), ws.data_ptr(),
                                        _lib.stream_handle()), "build_mods")
        return mods, fin

    def drop_table_weights(self) -> None:
        """Free the fp32 adaLN weights (only needed to build tables)."""
        self._mod_w = None

    def __del__(self):
        try:
            if getattr(self, "handle", None) is not None:
                _lib.lib().t2w_dit_destroy(self.handle)
        except Exception:
            pass


# --- stream state ---------------------------------------------------------------------------------------------------

class SlotPool:
    """Host free list of key slots (``engine/runtime/dit_fast.py:58-78``)."""

    def __init__(self, n: int):
        self.n = n
        self.free = list(range(n - 1, -1, -1))

    def alloc(self, k: int) -> list[int]:
        if k > len(self.free):
            raise RuntimeError(f"Token2Wav cache pool exhausted ({k} slots wanted, {len(self.free)} free of {self.n})")
        out = self.free[len(self.free) - k:][::-1] if k else []
        del self.free[len(self.free) - k:]
        return out

    def release(self, ids: list[int]) -> None:
        self.free.extend(ids)

    def in_use(self) -> int:
        return self.n - len(self.free)


@dataclass
class FastRow:
    """One CFG row: key slots in the reference tensor order (newest window first) and its two conv-cache row slots
    (the current one is read, the other written)."""
    order: list[int] = field(default_factory=list)
    cnn: tuple[int, int] = (-1, -1)
    cur: int = 0


@dataclass
class FastCache:
    """A request's estimator caches (conditional and unconditional row) and its trim length (prompt mel frames)."""
    rows: tuple[FastRow, FastRow]
    keep: int = 0

    @property
    def length(self) -> int:
        return len(self.rows[0].order)


def plan_call(rows: list[FastRow], Ts: list[int], new: list[list[int]], keep: list[bool], cnn_scratch: int) -> dict:
    """Host plan of one call (``engine/runtime/dit_fast.py:223-266``): rows ``[cond 0..n-1 | uncond 0..n-1]`` each with
    its window's ``Ts[i]`` tokens and freshly allocated key slots ``new[r]``.  Returns the device tables (in
    ``t2w_solve_args`` order; kv_idx last because its length varies) and the bookkeeping the solve needs afterwards."""
    n = len(Ts)
    lens = Ts + Ts
    tok_row, tok_pos, new_slot = [], [], []
    row_start, row_kv_off, row_kv_len, rd, wr, kv, tiles = [], [], [], [], [], [], []
    o = 0
    for r, (row, t, nw) in enumerate(zip(rows, lens, new)):
        row_start.append(o)
        tok_row += [r] * t
        tok_pos += list(range(t))
        new_slot += nw
        row_kv_off.append(len(kv))
        kv += nw + row.order  # the row's new frames first (masking is by position), then its cache
        row_kv_len.append(t + len(row.order))
        rd.append(row.cnn[row.cur])
        wr.append(row.cnn[1 - row.cur] if keep[r % n] else cnn_scratch)
        tiles += [v for q0 in range(0, t, 64) for v in (r, q0)]
        o += t
    a_src = [i + 2 * r for i, r in enumerate(tok_row)]
    parts = [tok_row, tok_pos, a_src, new_slot, row_start, lens, row_kv_off, row_kv_len, rd, wr, tiles, kv]
    return {"n_tok": o, "n_rows": 2 * n, "half": o // 2, "n_tiles": len(tiles) // 2, "parts": parts, "new": new, "rows": rows}


ROW_BUCKETS = (2, 4, 8, 16, 32, 64)  # request rows (both CFG halves) of a graph bucket, padding rows excluded
MAX_GRAPH_T = 56  # frames per row of the streaming windows the row buckets are sized for
SETUP_TOKENS = 4096  # row buckets up to SETUP_ROWS also take whole-prompt setups up to this many tokens
SETUP_ROWS = 8


def token_buckets(rb: int) -> list[int]:
    """Token buckets (both halves) of row bucket ``rb`` (``token_buckets``, ``engine/runtime/dit_fast.py:43-55``):
    multiples of 128 below 512, then of 256, up to the bucket's top (``MAX_GRAPH_T`` frames per row, at least
    ``SETUP_TOKENS`` for small buckets), which is a bucket itself."""
    top = max(rb * MAX_GRAPH_T, SETUP_TOKENS if rb <= SETUP_ROWS else 0)
    return [b for b in list(range(128, 512, 128)) + list(range(512, top, 256)) if b < top] + [top]


def bucket_of(n_rows: int, n_tok: int) -> tuple[int, int] | None:
    """The smallest row bucket holding ``n_rows`` request rows with a token bucket for ``n_tok`` tokens, and that token
    bucket (``FastDiT._bucket``, ``engine/runtime/dit_fast.py:212-221``); None when no bucket fits."""
    for rb in ROW_BUCKETS:
        if rb >= n_rows:
            nb = next((b for b in token_buckets(rb) if b >= n_tok), None)
            if nb is not None:
                return rb, nb
    return None


def bucket_tiles(rb: int, nb: int) -> int:
    """Attention tiles of a bucket's graph: a half's real rows of T_i tokens take sum ceil(T_i / 64) tiles, at most
    (tokens + 63 rows) / 64, so tokens / 64 + rows per half (the padding row included) covers every call."""
    return 2 * ((nb // 2 + 63) // 64 + rb // 2 + 1)


def pad_plan(p: dict, rb: int, nb: int, kv_scratch: int, cnn_scratch: int) -> dict:
    """Pads a call's plan to bucket ``(rb, nb)`` (the layout of ``FastDiT._plan``, ``engine/runtime/dit_fast.py:223-263``):
    each CFG half holds its request rows, ``rb / 2 - n`` empty rows and one padding row carrying the half's
    ``nb / 2 - half`` padding tokens.  Padding tokens have zero inputs, write their keys and values to one scratch slot
    and attend to it alone; empty and padding rows read and write the scratch conv-cache slot; their outputs are
    discarded.  No real row reads padding data, since every kernel works within a token or a row.  The attention tile
    list is filled up to ``bucket_tiles`` with tiles past a row's end, which the kernel skips."""
    tok_row, tok_pos, _, new_slot, row_start, lens, kv_off, kv_len, rd, wr, tiles, kv = p["parts"]
    n = p["n_rows"] // 2
    hr, half_b = rb // 2 + 1, nb // 2
    pad = half_b - p["half"]
    row_tiles: dict[int, list[int]] = {}
    for i in range(0, len(tiles), 2):
        row_tiles.setdefault(tiles[i], []).append(tiles[i + 1])
    out = [[] for _ in range(12)]
    t_row, t_pos, _, t_slot, t_start, t_len, t_kvo, t_kvl, t_rd, t_wr, t_tiles, t_kv = out
    o = 0
    for h in range(2):  # cond half, then uncond half
        for j in range(hr):
            r_new = h * hr + j
            if j < n:  # a request row
                r = h * n + j
                s0, T = row_start[r], lens[r]
                t_pos += tok_pos[s0:s0 + T]
                t_slot += new_slot[s0:s0 + T]
                t_kvo.append(len(t_kv))
                t_kv += kv[kv_off[r]:kv_off[r] + kv_len[r]]
                t_kvl.append(kv_len[r])
                t_rd.append(rd[r])
                t_wr.append(wr[r])
                q0s = row_tiles.get(r, [])
            else:  # empty rows, then the padding row
                T = pad if j == hr - 1 else 0
                t_pos += list(range(T))
                t_slot += [kv_scratch] * T
                t_kvo.append(len(t_kv))
                t_kv += [kv_scratch] * T
                t_kvl.append(T)
                t_rd.append(cnn_scratch)
                t_wr.append(cnn_scratch)
                q0s = list(range(0, T, 64))
            t_row += [r_new] * T
            t_tiles += [v for q0 in q0s for v in (r_new, q0)]
            t_start.append(o)
            t_len.append(T)
            o += T
    n_tiles = bucket_tiles(rb, nb)
    if len(t_tiles) // 2 > n_tiles:
        raise AssertionError("attention tiles beyond the bucket's bound")
    t_tiles += [hr - 1, 1 << 30] * (n_tiles - len(t_tiles) // 2)
    out[2] = [i + 2 * r for i, r in enumerate(t_row)]
    q = dict(p)
    q.update({"n_tok": o, "n_rows": 2 * hr, "half": half_b, "n_tiles": n_tiles, "parts": out, "real_half": p["half"]})
    return q


def advance_row(r: FastRow, new: list[int], keep: bool, keep_len: int) -> list[int]:
    """After a solve: a kept window's slots join the row as ``[new, cache]`` (the reference's concatenation order), then
    the order is trimmed to its first ``keep_len`` and last 100 entries (``engine/runtime/dit_fast.py:480-490``) and
    the conv caches swap to the slot just written; a window that is not kept leaves the row as it was.  Returns the
    slots to release."""
    if not keep:
        return list(new)
    order = new + r.order
    freed = []
    if len(order) > keep_len + TRIM_SUFFIX:
        freed = order[keep_len:len(order) - TRIM_SUFFIX]
        order = order[:keep_len] + order[len(order) - TRIM_SUFFIX:]
    r.order = order
    r.cur = 1 - r.cur
    return freed


def _pad_halves(x: torch.Tensor, real: int, padded: int) -> torch.Tensor:
    """Conditional-token rows [real, C] padded with zero rows to [padded, C] (the padding rows come last)."""
    if padded == real:
        return x
    return torch.cat([x, x.new_zeros(padded - real, x.shape[1])])


class FastDiT:
    """The packed ragged CFG Euler solve over per-request caches (``FastDiT`` of ``engine/runtime/dit_fast.py``)."""

    def __init__(self, model: DiTModel, n_slots: int = 32768, max_streams: int = 96, use_graphs: bool = False, fp8: bool = False,
                 buckets: bool = True):
        """``fp8``: solves run the block GEMMs on fp8 MFMA (the model must have been built with fp8 weights).
        ``buckets`` (with ``use_graphs``): a call that fits a (rows, tokens) bucket is padded to it, so that one captured
        graph serves every call of the bucket; other calls (and every call without ``buckets``) take a graph keyed by
        their exact shape."""
        self.buckets = buckets
        if fp8 and not model.fp8:
            raise ValueError("fp8 solves need a DiTModel built with fp8=True")
        self.fp8 = fp8
        cfg = model.cfg
        self.model, self.cfg, self.device = model, cfg, model.device
        S, D, H = cfg.steps, cfg.depth, cfg.hidden
        self.pool = SlotPool(n_slots - 1)
        self.kv_scratch = n_slots - 1  # key slot written by padding tokens, outside the pool
        self.n_slots = n_slots
        self.k_pool = torch.zeros(S * D, n_slots, H, dtype=torch.bfloat16, device=self.device)
        self.v_pool = torch.zeros_like(self.k_pool)
        n_rs = 4 * max_streams + 2
        self.conv_pool = torch.zeros(n_rs, S, D, 2, 2, H, dtype=torch.bfloat16, device=self.device)
        self.cnn_free = list(range(n_rs - 1, -1, -1))
        self.cnn_scratch = self.cnn_free.pop()  # write slot of rows whose caches are not kept
        self.use_graphs = use_graphs
        self.graphs: dict[tuple, tuple] = {}
        self._ws = None
        self.counts = {"graph": 0, "eager": 0}

    # --- caches -----------------------------------------------------------------------------------------------------
    def new_cache(self, keep: int = 0) -> FastCache:
        if len(self.cnn_free) < 4:
            raise RuntimeError("Token2Wav conv-cache row slots exhausted")
        rows = []
        for _ in range(2):
            a, b = self.cnn_free.pop(), self.cnn_free.pop()
            self.conv_pool[a].zero_()
            rows.append(FastRow(cnn=(a, b)))
        return FastCache((rows[0], rows[1]), keep)

    def release(self, c: FastCache) -> None:
        for r in c.rows:
            self.pool.release(r.order)
            r.order = []
            if r.cnn[0] >= 0:
                self.cnn_free.extend(r.cnn)
                r.cnn = (-1, -1)

    def clone(self, c: FastCache) -> FastCache:
        """An independent copy (new slots holding the same keys, values and conv caches)."""
        out = self.new_cache(c.keep)
        for src, dst in zip(c.rows, out.rows):
            self.conv_pool[dst.cnn[0]] = self.conv_pool[src.cnn[src.cur]]
            dst.order = self.pool.alloc(len(src.order))
            if src.order:
                s = torch.tensor(src.order, device=self.device)
                d = torch.tensor(dst.order, device=self.device)
                self.k_pool[:, d] = self.k_pool[:, s]
                self.v_pool[:, d] = self.v_pool[:, s]
        return out

    # --- planning ---------------------------------------------------------------------------------------------------
    def _plan(self, caches: list[FastCache], Ts: list[int], keep: list[bool]) -> dict:
        rows = [c.rows[0] for c in caches] + [c.rows[1] for c in caches]
        new = [self.pool.alloc(t) for t in Ts + Ts]
        return plan_call(rows, Ts, new, keep, self.cnn_scratch)

    def _workspace(self, N: int, R: int) -> torch.Tensor:
        need = _lib.lib().t2w_dit_workspace_bytes(self.model.handle, N, R)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def _args(self, p: dict, tables: torch.Tensor, x0, stat, out, ws, chunk: int, in_rows=None) -> _lib.SolveArgs:
        offs = np.cumsum([0] + [len(x) for x in p["parts"]])
        tp = lambda i: tables.data_ptr() + 4 * int(offs[i])  # noqa: E731
        H = self.cfg.hidden
        return _lib.SolveArgs(p["n_tok"], p["n_rows"], p["half"], p["n_tiles"], int(chunk), _lib.ptr(x0), _lib.ptr(stat), _lib.ptr(in_rows),
                              out.data_ptr(), tp(0), tp(1), tp(2), tp(3), tp(4), tp(5), tp(6), tp(7), tp(8), tp(9), tp(11), tp(10),
                              self.k_pool.data_ptr(), self.v_pool.data_ptr(), self.n_slots * H, self.conv_pool.data_ptr(),
                              ws.data_ptr(), ws.numel(), int(self.fp8))

    @staticmethod
    def _tables(p: dict, device) -> torch.Tensor:
        flat = np.concatenate([np.asarray(x, dtype=np.int32) for x in p["parts"]]) if p["n_tok"] else np.zeros(1, np.int32)
        return torch.from_numpy(flat).to(device)

    # --- solve ------------------------------------------------------------------------------------------------------
    @torch.inference_mode()
    def solve(self, caches: list[FastCache], mu: list[torch.Tensor], spks: torch.Tensor, cond: list | None,
              keep: list[bool], chunk: int = 0) -> list[torch.Tensor]:
        """The CFG Euler solve of one window per request (``FastDiT.solve``, ``engine/runtime/dit_fast.py:431-495``).

        ``mu[i]`` [mel, T_i]; ``spks`` [n, mel] (after the speaker affine layer); ``cond[i]`` [mel, T_i] or None;
        ``keep[i]``: keep the window's keys and conv caches (then trim as the reference does), else leave the caches
        untouched (final flushes).  ``chunk`` > 0: chunk-causal attention among each row's new frames.  Returns each
        request's mel [mel, T_i] in fp32."""
        n = len(caches)
        Ts = [int(m.shape[1]) for m in mu]
        lens = [c.length for c in caches]
        p = self._plan(caches, Ts, keep)
        half, dev, mel = p["half"], self.device, self.cfg.mel
        noise = self.model.rand_noise
        if max(o + t for o, t in zip(lens, Ts)) > noise.shape[1]:
            raise RuntimeError("window beyond the flow's noise buffer")
        x0 = torch.cat([noise[:, o:o + t].t() for o, t in zip(lens, Ts)])
        mu_t = torch.cat([m.t() for m in mu]).to(dev, torch.float32)
        spk_t = torch.cat([spks[i:i + 1].to(dev, torch.float32).expand(t, -1) for i, t in enumerate(Ts)])
        cond_t = torch.cat([(c.t() if c is not None else mu_t.new_zeros(t, mel)) for c, t in zip(cond, Ts)]).to(dev, torch.float32) \
            if cond is not None else torch.zeros_like(mu_t)
        stat = torch.cat([mu_t, spk_t, cond_t], dim=1).contiguous()
        out = self._run(p, x0.contiguous(), stat, chunk)
        for i, c in enumerate(caches):
            for r, nw in ((p["rows"][i], p["new"][i]), (p["rows"][n + i], p["new"][n + i])):
                self.pool.release(advance_row(r, nw, keep[i], c.keep))
        res, o = [], 0
        for t in Ts:
            res.append(out[o:o + t].t())
            o += t
        return res

    def _run(self, p: dict, x0: torch.Tensor, stat: torch.Tensor, chunk: int) -> torch.Tensor:
        L = _lib.lib()
        N, R = p["n_tok"], p["n_rows"]
        st = _lib.stream_handle()
        if not self.use_graphs:
            tables = self._tables(p, self.device)
            out = torch.empty(p["half"], self.cfg.mel, device=self.device)
            ws = self._workspace(N, R)
            a = self._args(p, tables, x0, stat, out, ws, chunk)
            _lib.check(L.t2w_dit_solve(self.model.handle, C.byref(a), st), "dit_solve")
            self.counts["eager"] += 1
            return out
        real_half = p["half"]
        bucket = bucket_of(R, N) if self.buckets else None
        if bucket is not None:
            p = pad_plan(p, *bucket, self.kv_scratch, self.cnn_scratch)
            x0 = _pad_halves(x0, real_half, p["half"])
            stat = _pad_halves(stat, real_half, p["half"])
            N, R = p["n_tok"], p["n_rows"]
        key = (N, R, p["n_tiles"], chunk, self.fp8)
        flat = np.concatenate([np.asarray(x, dtype=np.int32) for x in p["parts"]])
        g = self.graphs.get(key)
        if g is not None and g["tables"].numel() < flat.size:  # more cached keys than this graph's table holds
            L.t2w_graph_destroy(g["graph"])
            g = None
        if g is None:
            g = {"tables": torch.zeros(flat.size + max(8192, flat.size), dtype=torch.int32, device=self.device), "x0": torch.empty_like(x0),
                 "stat": torch.empty_like(stat), "out": torch.empty(p["half"], self.cfg.mel, device=self.device),
                 "ws": torch.empty(L.t2w_dit_workspace_bytes(self.model.handle, N, R), dtype=torch.uint8, device=self.device),
                 "graph": None}
            self.graphs[key] = g
        # every table but kv_idx has a size fixed by the key; kv_idx is last, so all offsets the graph reads are stable
        g["tables"][:flat.size].copy_(torch.from_numpy(flat))
        g["x0"].copy_(x0)
        g["stat"].copy_(stat)
        if g["graph"] is None:
            a = self._args(p, g["tables"], g["x0"], g["stat"], g["out"], g["ws"], chunk)
            cap = self._capture_stream()  # capture needs a non-default stream; replays go on the caller's
            cst = cap.cuda_stream
            _lib.check(L.t2w_graph_begin(cst), "graph_begin")
            rc = L.t2w_dit_solve(self.model.handle, C.byref(a), cst)
            h = C.c_void_p()
            rc2 = L.t2w_graph_end(cst, C.byref(h))
            _lib.check(rc, "dit_solve (capture)")
            _lib.check(rc2, "graph_end")
            g["graph"] = h
        _lib.check(L.t2w_graph_launch(g["graph"], st), "graph_launch")
        self.counts["graph"] += 1
        return g["out"][:real_half].clone()

    def _capture_stream(self):
        if getattr(self, "_cap", None) is None:
            self._cap = torch.cuda.Stream()
        return self._cap

    # --- single estimator evaluation (no cache, full attention) ------------------------------------------------------
    @torch.inference_mode()
    def estimator_forward(self, x: torch.Tensor, mu: torch.Tensor, t: float, spks: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
        """One estimator forward (``_estimator_temb``, ``engine/runtime/token2wav_batch.py:787-810``) of B independent
        rows with empty caches and full attention: x, mu, cond [B, mel, T]; spks [B, mel]; t a scalar.  Returns dphi
        [B, mel, T] fp32."""
        B, mel, T = x.shape
        dev = self.device
        rows = torch.cat([x, mu, spks[:, :, None].expand(-1, -1, T), cond], dim=1).to(dev, torch.float32)  # [B, 4 mel, T]
        in_rows = rows.permute(0, 2, 1).reshape(B * T, 4 * mel).contiguous()
        slots = self.pool.alloc(B * T)
        try:
            tok_row = [r for r in range(B) for _ in range(T)]
            parts = [tok_row, [p for _ in range(B) for p in range(T)], [i + 2 * r for i, r in enumerate(tok_row)], slots,
                     [r * T for r in range(B)], [T] * B, [r * T for r in range(B)], [T] * B, [self.cnn_scratch] * B, [self.cnn_scratch] * B,
                     [v for r in range(B) for q0 in range(0, T, 64) for v in (r, q0)], slots]
            self.conv_pool[self.cnn_scratch].zero_()
            p = {"n_tok": B * T, "n_rows": B, "half": 0, "n_tiles": len(parts[10]) // 2, "parts": parts}
            tables = self._tables(p, dev)
            out = torch.empty(B * T, mel, device=dev)
            mods, fin = self.model.tables([float(t)])
            ws = self._workspace(B * T, B)
            a = self._args(p, tables, None, None, out, ws, 0, in_rows=in_rows)
            _lib.check(_lib.lib().t2w_dit_forward(self.model.handle, C.byref(a), 0, mods.data_ptr(), fin.data_ptr(), _lib.stream_handle()),
                       "dit_forward")
            torch.cuda.current_stream().synchronize()
        finally:
            self.pool.release(slots)
        return out.view(B, T, mel).permute(0, 2, 1).contiguous()
