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
        # optional rotary embedding of q and k (none in the reference): pair i turns at theta^(-2i / head_dim) rad per frame
        self.rope_freq = None
        if cfg.rope_theta > 0:
            i = torch.arange(0, cfg.head_dim, 2, dtype=torch.float64)
            self.rope_freq = f32((cfg.rope_theta ** (-i / cfg.head_dim)).float())
        g = _lib.DitGlobals(self.t["in_w"].data_ptr(), self.t["in_b"].data_ptr(), self.t["out_w"].data_ptr(), self.t["out_b"].data_ptr(),
                            self.mods.data_ptr(), self.final_mods.data_ptr(), C.cast(self._dts, _lib.FP),
                            _lib.ptr(self.rope_freq))
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
    """Slot ids of the key/value pools (a slot holds one cached frame of one CFG row in every (Euler step, block) pool).

    Free ids live in one int32 array used as a stack (``_stack[:_top]``, the next id handed out on top).  ``reserved``
    ids are taken once at construction and never returned: padding tokens of bucketed calls write their keys there.
    They count as in use, as the reference's reserved padding slots do (callers subtract ``FastDiT.scratch``)."""

    def __init__(self, n: int, reserved: int = 0):
        self.n = int(n)
        self._stack = np.arange(self.n - 1, -1, -1, dtype=np.int32)
        self._top = self.n
        self.reserved = self.alloc(reserved)

    def alloc(self, k: int) -> np.ndarray:
        k = int(k)
        if k > self._top:
            raise RuntimeError(f"Token2Wav key/value slots exhausted: {k} needed, {self._top} of {self.n} free")
        self._top -= k
        return self._stack[self._top:self._top + k][::-1].copy()

    def release(self, ids) -> None:
        ids = np.asarray(ids, dtype=np.int32).ravel()
        self._stack[self._top:self._top + ids.size] = ids
        self._top += ids.size

    def in_use(self) -> int:
        return self.n - self._top

    @property
    def n_free(self) -> int:
        return self._top


_NO_SLOTS = np.zeros(0, dtype=np.int32)


@dataclass
class FastRow:
    """Cached frames of one CFG row of a stream.  ``slots``: key/value slot ids, the newest window's frames first (the
    order the reference concatenates ``[new, cache]`` in, which the trim relies on).  ``conv``: two row slots of the
    conv-cache pool; ``conv[cur]`` holds the two cached frames per (step, block, conv), a kept window writes the other
    one and flips ``cur``.  ``pos``: the stream position of the next window's first frame (frames of kept windows so
    far), the angle origin of the optional rotary embedding."""
    slots: np.ndarray = field(default_factory=lambda: _NO_SLOTS)
    conv: tuple = (-1, -1)
    cur: int = 0
    pos: int = 0

    @property
    def order(self) -> list[int]:
        return self.slots.tolist()


@dataclass
class FastCache:
    """Estimator state of one stream: its conditional and unconditional rows, and ``keep``, the number of cached frames
    the trim always keeps from the newest end (the prompt's mel frames)."""
    rows: tuple
    keep: int = 0

    @property
    def length(self) -> int:
        return int(self.rows[0].slots.size)


def _tile_list(lens: np.ndarray) -> np.ndarray:
    """(row, first query) of every 64-query attention tile of rows with ``lens`` tokens, interleaved."""
    per = (lens + 63) // 64
    rows = np.repeat(np.arange(lens.size, dtype=np.int64), per)
    first = np.arange(rows.size, dtype=np.int64) - np.repeat(np.cumsum(per) - per, per)
    return np.stack([rows, 64 * first], 1).ravel()


def _layout(lens, new, kv, rd, wr, pos0=None) -> list[np.ndarray]:
    """The device tables of a call (``t2w_solve_args`` order, then the stream positions, ``kv_idx`` last: every table but
    the key lists has a size fixed by the call's token and row counts) from its rows in call order: token counts
    ``lens``, new key slots ``new[r]``, key lists ``kv[r]``, conv-cache read / write slots and the stream position of
    each row's first new frame (``pos0``, default 0)."""
    lens = np.asarray(lens, dtype=np.int64)
    starts = np.cumsum(lens) - lens
    tok_row = np.repeat(np.arange(lens.size, dtype=np.int64), lens)
    idx = np.arange(tok_row.size, dtype=np.int64)
    tok_pos = idx - starts[tok_row]
    pos0 = np.zeros(lens.size, dtype=np.int64) if pos0 is None else np.asarray(pos0, dtype=np.int64)
    kv_len = np.array([x.size for x in kv], dtype=np.int64)
    cat = lambda xs: np.concatenate(xs) if len(xs) else _NO_SLOTS  # noqa: E731
    return [tok_row, tok_pos, idx + 2 * tok_row, cat(new), starts, lens, np.cumsum(kv_len) - kv_len, kv_len,
            np.asarray(rd, dtype=np.int64), np.asarray(wr, dtype=np.int64), _tile_list(lens), pos0[tok_row] + tok_pos, cat(kv)]


ATTN_ROW_KMAX = 512  # key-list length up to which the attention holds a row's keys in LDS (t2w_solve_args.kv_max)


def _kv_max(p: dict) -> int:
    """A call's ``kv_max``: 256 or 512 (the row-resident attention's LDS sizes; lists up to 256 keys let two of its
    workgroups share a CU) when every row's key list fits, else 0 (no bound).  Exact-shape graphs are keyed by it, so a
    replay never breaks the bound its capture stated.

    Bucketed calls always state 0: their rows are streaming windows of at most ``MAX_GRAPH_T`` frames or small setup
    batches, which never meet the row-resident attention's launch condition (at least 16 rows of three or more 64-query
    tiles on average: a bucket's tiles per row stay below that for every bucket of the table), so the bound would
    select nothing and would only split one bucket's graph by its rows' cached lengths."""
    if p.get("bucket") is not None:
        return 0
    kv = p["parts"][7]
    top = int(kv.max()) if kv.size else 0
    return 256 if top <= 256 else ATTN_ROW_KMAX if top <= ATTN_ROW_KMAX else 0


def plan_call(rows: list[FastRow], Ts: list[int], new: list[np.ndarray], keep: list[bool], cnn_scratch: int, cnn_zero: int | None = None,
              bucket: tuple[int, int] | None = None, kv_scratch: int | None = None) -> dict:
    """Host plan of one call over ``n`` requests (``engine/runtime/dit_fast.py:223-266``): rows ``[cond 0..n-1 | uncond
    0..n-1]``, row r with its window's ``Ts[r % n]`` tokens and freshly allocated key slots ``new[r]``; a row's keys are
    its new frames, then its cache (masking is by position).  A kept window's conv caches go to the row's other conv
    slot, others to ``cnn_scratch``.

    ``bucket = (rb, nb)`` pads the call to a graph bucket: each CFG half then holds its requests, ``rb / 2 - n`` empty
    rows and one padding row with the half's ``nb / 2 - sum(Ts)`` padding tokens, which write their keys to slot
    ``kv_scratch`` and attend to it alone; empty and padding rows read the zero conv slot ``cnn_zero`` and write
    ``cnn_scratch``; the tile list is filled to ``bucket_tiles`` with tiles past a row's end (skipped by the kernel).
    No real row reads padding data: every kernel works within a token or a row.

    Returns the tables (``parts``) and what the solve needs afterwards."""
    n = len(Ts)
    half = int(sum(Ts))
    lens, nw, kv, rd, wr, p0 = [], [], [], [], [], []
    pad = 0 if bucket is None else bucket[1] // 2 - half
    extra = 0 if bucket is None else bucket[0] // 2 - n  # empty rows per half
    zero = cnn_scratch if cnn_zero is None else cnn_zero
    for h in range(2):
        for i in range(n):
            r = rows[h * n + i]
            lens.append(Ts[i])
            nw.append(new[h * n + i])
            kv.append(np.concatenate([new[h * n + i], r.slots]))
            rd.append(r.conv[r.cur])
            wr.append(r.conv[1 - r.cur] if keep[i] else cnn_scratch)
            p0.append(r.pos)
        if bucket is not None:
            for j in range(extra + 1):
                T = pad if j == extra else 0
                pads = np.full(T, kv_scratch, dtype=np.int32)
                lens.append(T)
                nw.append(pads)
                kv.append(pads)
                rd.append(zero)
                wr.append(cnn_scratch)
                p0.append(0)
    parts = _layout(lens, nw, kv, rd, wr, p0)
    R = len(lens)
    n_tiles = parts[10].size // 2
    if bucket is not None:
        rb, nb = bucket
        want = bucket_tiles(rb, nb)
        if n_tiles > want:
            raise AssertionError("attention tiles beyond the bucket's bound")
        fill = np.tile(np.array([R - 1, 1 << 30], dtype=np.int64), want - n_tiles)
        parts[10] = np.concatenate([parts[10], fill])
        n_tiles = want
    return {"n_tok": int(sum(lens)), "n_rows": R, "half": half + pad, "real_half": half, "n_tiles": n_tiles, "parts": parts,
            "new": new, "rows": rows, "bucket": bucket}


ROW_BUCKETS = (2, 4, 8, 16, 32, 64)  # request rows (both CFG halves) of a graph bucket, padding rows excluded
MAX_GRAPH_T = 56  # frames per row of the streaming windows the row buckets are sized for
SETUP_TOKENS = 4096  # row buckets up to SETUP_ROWS also take whole-prompt setups up to this many tokens
SETUP_ROWS = 8


def bucket_top(rb: int) -> int:
    """The most tokens (both halves) a row bucket takes: ``MAX_GRAPH_T`` frames per row, and whole prompt setups up to
    ``SETUP_TOKENS`` in the small buckets (``bucket_top``, ``engine/runtime/dit_fast.py:37-45``)."""
    return max(rb * MAX_GRAPH_T, SETUP_TOKENS if rb <= SETUP_ROWS else 0)


def token_buckets(rb: int) -> list[int]:
    """Token buckets (both halves) of row bucket ``rb`` (``token_buckets``, ``engine/runtime/dit_fast.py:48-55``): steps of
    128 below 512, of 256 from there, and the bucket's top."""
    top = bucket_top(rb)
    steps = [b for b in range(128, 512, 128)] + [b for b in range(512, top, 256)]
    return [b for b in steps if b < top] + [top]


def bucket_of(n_rows: int, n_tok: int) -> tuple[int, int] | None:
    """The (row bucket, token bucket) a call of ``n_rows`` request rows and ``n_tok`` tokens pads to: the first row
    bucket with room for both, and its smallest token bucket that holds the call; None when none does."""
    for rb in (b for b in ROW_BUCKETS if b >= n_rows):
        fits = [b for b in token_buckets(rb) if b >= n_tok]
        if fits:
            return rb, fits[0]
    return None


def bucket_tiles(rb: int, nb: int) -> int:
    """Attention tiles of a bucket's graph: a half's real rows of T_i tokens take sum ceil(T_i / 64) tiles, at most
    (tokens + 63 rows) / 64, so tokens / 64 + rows per half (the padding row included) covers every call."""
    return 2 * ((nb // 2 + 63) // 64 + rb // 2 + 1)


def bucket_graph_key(bucket: tuple[int, int], chunk: int, fp8: int) -> tuple:
    """The key of a bucket's graph: the bucket, the chunk mask and the GEMM format (0 bf16, 1 fp8 MFMA, 2 e4m3
    weights) -- nothing that depends on the rows' cached lengths, so a graph captured on a padding-only plan serves
    every call that pads to its bucket."""
    return (tuple(bucket), int(chunk), int(fp8))


def all_buckets() -> list[tuple[int, int]]:
    return [(rb, nb) for rb in ROW_BUCKETS for nb in token_buckets(rb)]


def advance_row(r: FastRow, new: np.ndarray, keep: bool, keep_len: int) -> np.ndarray:
    """A row after its window was solved.  A kept window's frames go in front of the cache (``[new, cache]``); a cache
    longer than ``keep_len + 100`` then drops the entries between its first ``keep_len`` and its last 100
    (``engine/runtime/dit_fast.py:480-490``), and the conv slots flip.  A window that is not kept leaves the row alone.
    Returns the slot ids to give back to the pool."""
    if not keep:
        return new
    merged = np.concatenate([new, r.slots])
    cut = merged.size - TRIM_SUFFIX
    if cut > keep_len:
        freed = merged[keep_len:cut].copy()
        merged = np.concatenate([merged[:keep_len], merged[cut:]])
    else:
        freed = _NO_SLOTS
    r.slots = merged
    r.cur ^= 1
    r.pos += int(new.size)
    return freed


class _Upload:
    """Host tables to the device without a wait: a pinned staging copy, then an asynchronous copy on the current
    stream (the caching host allocator keeps the pinned block until that copy has run)."""

    @staticmethod
    def into(dst: torch.Tensor, host: np.ndarray) -> None:
        src = torch.from_numpy(host)
        if dst.is_cuda:
            src = src.pin_memory()
        dst[:host.size].copy_(src, non_blocking=True)

    @staticmethod
    def new(host: np.ndarray, device) -> torch.Tensor:
        out = torch.empty(max(host.size, 1), dtype=torch.int32, device=device)
        _Upload.into(out, host)
        return out


class FastDiT:
    """The packed ragged CFG Euler solve over per-stream caches (the ``FastDiT`` surface of
    ``engine/runtime/dit_fast.py``: ``new_cache / release / clone / solve / capture / capture_all``, attributes ``pool``,
    ``scratch``, ``cnn_free``, ``counts``, ``use_graphs``)."""

    FP8_MODES = {False: 0, None: 0, "bf16": 0, True: 1, "mx": 1, "weights": 2}

    def __init__(self, model: DiTModel, n_slots: int = 32768, max_streams: int = 96, use_graphs: bool = False, fp8: bool | str = False,
                 buckets: bool = True, max_exact_graphs: int = 8):
        """``n_slots`` cached frames per pool (one CFG row's frame each).  ``fp8``: True / "mx": the block GEMMs on fp8
        MFMA (e4m3 weights, MX fp8 activations); "weights": e4m3 weights with per-output-channel scales, dequantized to
        bf16 just before each block GEMM, bf16 activations and MFMA (both need a model built with fp8 weights).  ``use_graphs``: every call replays a captured hipGraph of its whole 10-step solve; with
        ``buckets`` a call that fits a (rows, tokens) bucket is padded to it, so one graph serves all its calls
        (``capture_all`` makes them all up front); other calls take a graph of their exact shape (the last
        ``max_exact_graphs`` are kept)."""
        if fp8 not in self.FP8_MODES:
            raise ValueError(f"fp8 must be False, True / 'mx' or 'weights', not {fp8!r}")
        mode = self.FP8_MODES[fp8]
        if mode and not model.fp8:
            raise ValueError("fp8 solves need a DiTModel built with fp8=True")
        cfg = model.cfg
        self.model, self.cfg, self.device, self.fp8 = model, cfg, model.device, mode
        self.use_graphs, self.buckets, self.max_exact_graphs = use_graphs, buckets, max_exact_graphs
        S, D, H = cfg.steps, cfg.depth, cfg.hidden
        self.pool = SlotPool(n_slots, reserved=1)
        self.kv_scratch = int(self.pool.reserved[0])
        self.scratch = self.pool.reserved.size  # reserved slots counted by pool.in_use()
        self.n_slots = n_slots
        self.k_pool = torch.zeros(S * D, n_slots, H, dtype=torch.bfloat16, device=self.device)
        self.v_pool = torch.zeros_like(self.k_pool)
        n_rs = 4 * max_streams + 2
        self.conv_pool = torch.zeros(n_rs, S, D, 2, 2, H, dtype=torch.bfloat16, device=self.device)
        self.cnn_free = list(range(n_rs))
        self.cnn_zero = self.cnn_free.pop()     # stays zero: read by rows without a cache of their own
        self.cnn_scratch = self.cnn_free.pop()  # written by rows whose conv caches are not kept
        self.graphs: dict[tuple, dict] = {}
        self.exact: dict[tuple, dict] = {}
        self._arena = None
        self._ws = None
        self._cap = None
        self.counts = {"graph": 0, "eager": 0}

    # --- caches -----------------------------------------------------------------------------------------------------
    def new_cache(self, keep: int = 0) -> FastCache:
        if len(self.cnn_free) < 4:
            raise RuntimeError("Token2Wav conv-cache row slots exhausted")
        rows = []
        for _ in range(2):
            conv = (self.cnn_free.pop(), self.cnn_free.pop())
            self.conv_pool[conv[0]].zero_()
            rows.append(FastRow(conv=conv))
        return FastCache(tuple(rows), keep)

    def release(self, c: FastCache) -> None:
        for r in c.rows:
            self.pool.release(r.slots)
            r.slots = _NO_SLOTS
            if r.conv[0] >= 0:
                self.cnn_free += list(r.conv)
                r.conv = (-1, -1)

    def clone(self, c: FastCache) -> FastCache:
        """A copy with its own slots holding the same keys, values and conv frames (one gather per pool)."""
        out = self.new_cache(c.keep)
        for src, dst in zip(c.rows, out.rows):
            self.conv_pool[dst.conv[0]].copy_(self.conv_pool[src.conv[src.cur]])
            dst.slots = self.pool.alloc(src.slots.size)
            dst.pos = src.pos
        n = c.length
        if n:
            ids = _Upload.new(np.concatenate([r.slots for r in c.rows] + [r.slots for r in out.rows]), self.device).long()
            s, d = ids[:2 * n], ids[2 * n:]
            for pool in (self.k_pool, self.v_pool):
                pool.index_copy_(1, d, pool.index_select(1, s))
        return out

    # --- inputs -----------------------------------------------------------------------------------------------------
    def _inputs(self, caches: list[FastCache], mu: list[torch.Tensor], spks: torch.Tensor, cond: list | None, Ts: list[int]):
        """x0 (the flow's noise buffer read from each stream's cache length on) and the per-token conditioning
        ``[mu | spk | cond]`` of the conditional half, token-major fp32 (the unconditional half is zero)."""
        noise, mel, dev = self.model.rand_noise, self.cfg.mel, self.device
        n, half = len(Ts), int(sum(Ts))
        starts = np.array([c.length for c in caches], dtype=np.int64)
        if int((starts + np.asarray(Ts)).max()) > noise.shape[1]:
            raise RuntimeError("window beyond the flow's noise buffer")
        # one upload: the noise column and the stream of every conditional token
        lens = np.asarray(Ts, dtype=np.int64)
        req = np.repeat(np.arange(n, dtype=np.int64), lens)
        col = np.arange(half, dtype=np.int64) - np.repeat(np.cumsum(lens) - lens, lens) + starts[req]
        idx = _Upload.new(np.concatenate([col, req]).astype(np.int32), dev).long()
        x0 = noise.index_select(1, idx[:half]).t().contiguous()
        spk_t = spks.to(dev, torch.float32).reshape(n, mel).index_select(0, idx[half:])
        mu_t = torch.cat([m.to(dev, torch.float32) for m in mu], dim=1).t()
        if cond is None or all(c is None for c in cond):
            cond_t = torch.zeros_like(mu_t)
        else:
            cond_t = torch.cat([(c.to(dev, torch.float32) if c is not None else m.new_zeros(mel, m.shape[1], dtype=torch.float32))
                                for c, m in zip(cond, mu)], dim=1).t()
        return x0, torch.cat([mu_t, spk_t, cond_t], dim=1)

    # --- solve ------------------------------------------------------------------------------------------------------
    @torch.inference_mode()
    def solve(self, caches: list[FastCache], mu: list[torch.Tensor], spks: torch.Tensor, cond: list | None,
              keep: list[bool], chunk: int = 0) -> list[torch.Tensor]:
        """The CFG Euler solve of one window per stream (``FastDiT.solve``, ``engine/runtime/dit_fast.py:431-495``).

        ``mu[i]`` [mel, T_i]; ``spks`` [n, mel] (after the speaker affine layer); ``cond[i]`` [mel, T_i] or None;
        ``keep[i]``: keep the window's keys and conv caches (then trim as the reference does), else leave the caches
        untouched (final flushes).  ``chunk`` > 0: chunk-causal attention among each row's new frames.  Returns each
        stream's mel [mel, T_i] in fp32.  Nothing waits for the GPU."""
        return self._solve(caches, mu, spks, cond, keep, chunk)

    @torch.inference_mode()
    def solve_timed(self, caches: list[FastCache], mu: list[torch.Tensor], spks: torch.Tensor, cond: list | None,
                    keep: list[bool], chunk: int = 0, cap: int = 8192) -> tuple[list[torch.Tensor], list[tuple]]:
        """``solve`` run eagerly (no graph) under the library's launch timer: (mels, [(kind, ms, bytes)] of every
        instrumented launch -- the dense gated-residual tile GEMMs, proj and fc2 of every block at calls of more than
        128 tokens -- timed by HIP events around the launch).  A measurement aid; waits for the GPU."""
        with _lib.LaunchTimer(cap) as t:
            out = self._solve(caches, mu, spks, cond, keep, chunk, eager=True)
        return out, t.launches

    def _solve(self, caches, mu, spks, cond, keep, chunk, eager: bool = False):
        Ts = [int(m.shape[1]) for m in mu]
        x0, stat = self._inputs(caches, mu, spks, cond, Ts)
        rows = [c.rows[0] for c in caches] + [c.rows[1] for c in caches]
        new = [self.pool.alloc(t) for t in Ts + Ts]
        bucket = bucket_of(2 * len(Ts), 2 * sum(Ts)) if (self.use_graphs and self.buckets and not eager) else None
        p = plan_call(rows, Ts, new, keep, self.cnn_scratch, self.cnn_zero, bucket, self.kv_scratch)
        out = self._run(p, x0, stat, chunk, bucket, eager)
        n = len(caches)
        for i, c in enumerate(caches):
            for h in range(2):
                self.pool.release(advance_row(c.rows[h], new[h * n + i], keep[i], c.keep))
        offs = np.cumsum([0] + Ts)
        return [out[offs[i]:offs[i + 1]].t() for i in range(n)]

    def _args(self, p: dict, tables: torch.Tensor, x0, stat, out, ws, chunk: int, in_rows=None) -> _lib.SolveArgs:
        offs = np.cumsum([0] + [x.size for x in p["parts"]])
        tp = lambda i: tables.data_ptr() + 4 * int(offs[i])  # noqa: E731
        return _lib.SolveArgs(p["n_tok"], p["n_rows"], p["half"], p["n_tiles"], int(chunk), _lib.ptr(x0), _lib.ptr(stat), _lib.ptr(in_rows),
                              out.data_ptr(), tp(0), tp(1), tp(2), tp(3), tp(4), tp(5), tp(6), tp(7), tp(8), tp(9), tp(12), tp(10),
                              self.k_pool.data_ptr(), self.v_pool.data_ptr(), self.n_slots * self.cfg.hidden, self.conv_pool.data_ptr(),
                              ws.data_ptr(), ws.numel(), int(self.fp8), tp(11), _kv_max(p))

    def _workspace(self, N: int, R: int) -> torch.Tensor:
        need = _lib.lib().t2w_dit_workspace_bytes(self.model.handle, N, R)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._ws

    @staticmethod
    def _flat(p: dict) -> np.ndarray:
        return np.concatenate([x.astype(np.int32, copy=False) for x in p["parts"]])

    def _run(self, p: dict, x0: torch.Tensor, stat: torch.Tensor, chunk: int, bucket, eager: bool = False) -> torch.Tensor:
        L, st = _lib.lib(), _lib.stream_handle()
        if not self.use_graphs or eager:
            tables = _Upload.new(self._flat(p), self.device)
            out = torch.empty(p["half"], self.cfg.mel, device=self.device)
            a = self._args(p, tables, x0, stat, out, self._workspace(p["n_tok"], p["n_rows"]), chunk)
            _lib.check(L.t2w_dit_solve(self.model.handle, C.byref(a), st), "dit_solve")
            self.counts["eager"] += 1
            return out
        flat = self._flat(p)
        g = self._bucket_graph(bucket, chunk, flat.size) if bucket is not None else self._exact_graph(p, chunk, flat.size)
        _Upload.into(g["tables"], flat)
        half = p["real_half"]
        g["x0"][:half].copy_(x0)
        g["stat"][:half].copy_(stat)
        if p["half"] > half:  # padding tokens: zero inputs
            g["x0"][half:p["half"]].zero_()
            g["stat"][half:p["half"]].zero_()
        if g["graph"] is None:
            g["graph"] = self._capture(p, g, chunk)
        _lib.check(L.t2w_graph_launch(g["graph"], st), "graph_launch")
        self.counts["graph"] += 1
        return g["out"][:half].clone()

    def _capture(self, p: dict, g: dict, chunk: int):
        """Capture the solve of plan ``p`` over the graph's buffers on a side stream (capture needs a non-default
        stream; replays go on the caller's)."""
        L = _lib.lib()
        a = self._args(p, g["tables"], g["x0"], g["stat"], g["out"], g["ws"], chunk)
        if self._cap is None:
            self._cap = torch.cuda.Stream()
        self._cap.wait_stream(torch.cuda.current_stream())
        cst = self._cap.cuda_stream
        _lib.check(L.t2w_graph_begin(cst), "graph_begin")
        rc = L.t2w_dit_solve(self.model.handle, C.byref(a), cst)
        h = C.c_void_p()
        rc2 = L.t2w_graph_end(cst, C.byref(h))
        _lib.check(rc, "dit_solve (capture)")
        _lib.check(rc2, "graph_end")
        torch.cuda.current_stream().wait_stream(self._cap)
        return h

    # --- graphs -----------------------------------------------------------------------------------------------------
    # Bucket graphs share one arena (tables, inputs, output, workspace) sized for the largest bucket: replays are ordered
    # on the caller's stream and each output is copied out before the next call writes the arena.
    KV_ROW_CAP = 2048  # cached keys per row the shared table arena is sized for (a larger call regrows it)

    def _arena_for(self, n_ints: int) -> dict:
        a = self._arena
        if a is None or a["tables"].numel() < n_ints:
            if a is not None:  # every bucket graph points into the old arena
                self.drop_graphs(exact=False)
            top = max(nb for _, nb in all_buckets())
            rows = 2 * (ROW_BUCKETS[-1] // 2 + 1)
            cap = max(n_ints, 16 * top + 2 * rows * (self.KV_ROW_CAP + 8))
            ws = max(_lib.lib().t2w_dit_workspace_bytes(self.model.handle, nb, 2 * (rb // 2 + 1)) for rb, nb in all_buckets())
            dev, mel = self.device, self.cfg.mel
            a = {"tables": torch.zeros(cap, dtype=torch.int32, device=dev), "x0": torch.zeros(top // 2, mel, device=dev),
                 "stat": torch.zeros(top // 2, 3 * mel, device=dev), "out": torch.zeros(top // 2, mel, device=dev),
                 "ws": torch.empty(ws, dtype=torch.uint8, device=dev)}
            self._arena = a
        return a

    def _bucket_graph(self, bucket, chunk: int, n_ints: int) -> dict:
        arena = self._arena_for(n_ints)
        key = bucket_graph_key(bucket, chunk, self.fp8)
        g = self.graphs.get(key)
        if g is None:
            g = dict(arena, graph=None)
            self.graphs[key] = g
        return g

    def _exact_graph(self, p: dict, chunk: int, n_ints: int) -> dict:
        key = (p["n_tok"], p["n_rows"], p["n_tiles"], chunk, self.fp8, _kv_max(p))
        g = self.exact.pop(key, None)
        if g is not None and g["tables"].numel() < n_ints:  # more cached keys than this graph's tables hold
            _lib.lib().t2w_graph_destroy(g["graph"])
            g = None
        if g is None:
            while len(self.exact) >= self.max_exact_graphs:
                old = self.exact.pop(next(iter(self.exact)))
                _lib.lib().t2w_graph_destroy(old["graph"])
            dev, mel, half = self.device, self.cfg.mel, p["half"]
            g = {"tables": torch.zeros(2 * n_ints + 8192, dtype=torch.int32, device=dev), "x0": torch.empty(half, mel, device=dev),
                 "stat": torch.empty(half, 3 * mel, device=dev), "out": torch.empty(half, mel, device=dev),
                 "ws": torch.empty(_lib.lib().t2w_dit_workspace_bytes(self.model.handle, p["n_tok"], p["n_rows"]), dtype=torch.uint8, device=dev),
                 "graph": None}
        self.exact[key] = g  # most recently used last
        return g

    @torch.inference_mode()
    def capture(self, rb: int, nb: int, chunk: int = 0) -> None:
        """Capture the graph of bucket (``rb`` request rows, ``nb`` tokens) now (``FastDiT.capture``,
        ``engine/runtime/dit_fast.py:392-422``), on a plan whose tokens are all padding."""
        if not self.use_graphs:
            raise RuntimeError("capture needs use_graphs=True")
        p = plan_call([], [], [], [], self.cnn_scratch, self.cnn_zero, (rb, nb), self.kv_scratch)
        flat = self._flat(p)
        g = self._bucket_graph((rb, nb), chunk, flat.size)
        if g["graph"] is None:
            _Upload.into(g["tables"], flat)
            g["graph"] = self._capture(p, g, chunk)

    def capture_all(self, row_buckets=ROW_BUCKETS) -> int:
        """Every bucket's graph (``FastDiT.capture_all``, ``engine/runtime/dit_fast.py:424-428``); returns the count."""
        for rb in row_buckets:
            for nb in token_buckets(rb):
                self.capture(rb, nb)
        return len(self.graphs)

    def drop_graphs(self, exact: bool = True) -> None:
        L = _lib.lib()
        for g in self.graphs.values():
            if g["graph"] is not None:
                L.t2w_graph_destroy(g["graph"])
        self.graphs = {}
        if exact:
            for g in self.exact.values():
                if g["graph"] is not None:
                    L.t2w_graph_destroy(g["graph"])
            self.exact = {}

    def __del__(self):
        try:
            self.drop_graphs()
        except Exception:
            pass

    # --- single estimator evaluation (no cache, full attention) ------------------------------------------------------
    @torch.inference_mode()
    def estimator_forward(self, x: torch.Tensor, mu: torch.Tensor, t: float, spks: torch.Tensor, cond: torch.Tensor) -> torch.Tensor:
        """One estimator forward (``_estimator_temb``, ``engine/runtime/token2wav_batch.py:787-810``) of B independent
        rows with empty caches and full attention: x, mu, cond [B, mel, T]; spks [B, mel]; t a scalar.  Returns dphi
        [B, mel, T] fp32.  Rows read the zero conv slot and write the scratch one, so no row sees another's frames."""
        B, mel, T = x.shape
        dev = self.device
        rows = torch.cat([x, mu, spks[:, :, None].expand(-1, -1, T), cond], dim=1).to(dev, torch.float32)  # [B, 4 mel, T]
        in_rows = rows.permute(0, 2, 1).reshape(B * T, 4 * mel).contiguous()
        slots = self.pool.alloc(B * T)
        try:
            new = [slots[r * T:(r + 1) * T] for r in range(B)]
            parts = _layout([T] * B, new, new, [self.cnn_zero] * B, [self.cnn_scratch] * B)
            p = {"n_tok": B * T, "n_rows": B, "half": 0, "n_tiles": parts[10].size // 2, "parts": parts}
            tables = _Upload.new(self._flat(p), dev)
            out = torch.empty(B * T, mel, device=dev)
            mods, fin = self.model.tables([float(t)])
            a = self._args(p, tables, None, None, out, self._workspace(B * T, B), 0, in_rows=in_rows)
            _lib.check(_lib.lib().t2w_dit_forward(self.model.handle, C.byref(a), 0, mods.data_ptr(), fin.data_ptr(), _lib.stream_handle()),
                       "dit_forward")
        finally:
            self.pool.release(slots)
        return out.view(B, T, mel).permute(0, 2, 1).contiguous()

    @torch.inference_mode()
    def estimator_chunk(self, x: torch.Tensor, mu: torch.Tensor, t: float, spks: torch.Tensor, cond: torch.Tensor,
                        cnn_cache: torch.Tensor, att_cache: torch.Tensor, chunk: int = 0):
        """The estimator on dense caches, as the reference module's ``_estimator`` / ``_estimator_temb`` take them
        (``engine/runtime/token2wav_batch.py:782-810``): B rows of T new frames, every row's T frames real, with the
        solve's mask (every cached frame visible; new frames full, or chunk-causal with ``chunk`` > 0).

        x, mu, cond [B, mel, T]; spks [B, mel]; t a scalar; cnn_cache [depth, B, 2H, 2] (conv1's two cached frames,
        then conv2's, oldest first); att_cache [depth, B, heads, L, 2 * head_dim] (k | v, newest frames first).
        Returns (dphi [B, mel, T], new cnn_cache [depth, B, 2H, 2], new att_cache [depth, B, heads, T + L,
        2 * head_dim] with the new frames first), the caches rounded to bf16 as the pools hold them.  The caches go
        through the step-0 layers of this object's pools (slots and conv rows borrowed for the call)."""
        cfg, dev = self.cfg, self.device
        B, mel, T = x.shape
        D, H, nh, dk = cfg.depth, cfg.hidden, cfg.heads, cfg.head_dim
        L = int(att_cache.shape[3])
        if tuple(att_cache.shape) != (D, B, nh, L, 2 * dk) or tuple(cnn_cache.shape) != (D, B, 2 * H, 2):
            raise ValueError(f"caches of shape {tuple(att_cache.shape)} / {tuple(cnn_cache.shape)} do not fit depth {D}, "
                             f"{B} rows, {nh} heads, hidden {H}")
        if len(self.cnn_free) < 2 * B:
            raise RuntimeError("Token2Wav conv-cache row slots exhausted")
        rows = torch.cat([x, mu, spks[:, :, None].expand(-1, -1, T), cond], dim=1).to(dev, torch.float32)
        in_rows = rows.permute(0, 2, 1).reshape(B * T, 4 * mel).contiguous()
        conv = [self.cnn_free.pop() for _ in range(2 * B)]
        rd, wr = conv[:B], conv[B:]
        slots = self.pool.alloc(B * (T + L))
        try:
            new = [slots[r * T:(r + 1) * T] for r in range(B)]
            old = [slots[B * T + r * L:B * T + (r + 1) * L] for r in range(B)]
            lists = [np.concatenate([new[r], old[r]]) for r in range(B)]
            if L:
                ids = torch.as_tensor(np.concatenate(old).astype(np.int64), device=dev)
                kv = att_cache.to(dev).permute(0, 1, 3, 2, 4).reshape(D, B * L, nh, 2 * dk)  # [depth, B L, heads, 2 dk]
                self.k_pool[:D].index_copy_(1, ids, kv[..., :dk].reshape(D, B * L, H).to(torch.bfloat16))
                self.v_pool[:D].index_copy_(1, ids, kv[..., dk:].reshape(D, B * L, H).to(torch.bfloat16))
            rd_ids = torch.as_tensor(rd, device=dev)
            # conv_pool[row, step 0, block, conv, frame, :] = cnn_cache[block, row, conv * H : (conv + 1) * H, frame]
            self.conv_pool[rd_ids, 0] = cnn_cache.to(dev).view(D, B, 2, H, 2).permute(1, 0, 2, 4, 3).to(torch.bfloat16)
            parts = _layout([T] * B, new, lists, rd, wr)
            p = {"n_tok": B * T, "n_rows": B, "half": 0, "n_tiles": parts[10].size // 2, "parts": parts}
            tables = _Upload.new(self._flat(p), dev)
            out = torch.empty(B * T, mel, device=dev)
            mods, fin = self.model.tables([float(t)])
            a = self._args(p, tables, None, None, out, self._workspace(B * T, B), int(chunk), in_rows=in_rows)
            _lib.check(_lib.lib().t2w_dit_forward(self.model.handle, C.byref(a), 0, mods.data_ptr(), fin.data_ptr(), _lib.stream_handle()),
                       "dit_forward")
            all_ids = torch.as_tensor(np.concatenate(lists).astype(np.int64), device=dev)
            k = self.k_pool[:D].index_select(1, all_ids).view(D, B, T + L, nh, dk)
            v = self.v_pool[:D].index_select(1, all_ids).view(D, B, T + L, nh, dk)
            new_att = torch.cat([k, v], dim=-1).permute(0, 1, 3, 2, 4).float().contiguous()
            new_cnn = self.conv_pool[torch.as_tensor(wr, device=dev), 0].permute(1, 0, 2, 4, 3).reshape(D, B, 2 * H, 2).float()
        finally:
            self.pool.release(slots)
            self.cnn_free += conv
        return out.view(B, T, mel).permute(0, 2, 1).contiguous(), new_cnn, new_att
