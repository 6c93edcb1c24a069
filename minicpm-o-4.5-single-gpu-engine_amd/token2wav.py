"""The Token2Wav module surface the reference's worker calls, over the MI355X DiT solve and HiFT.

Mirrors ``BatchedToken2Wav`` (``engine/runtime/token2wav_batch.py:151-309, 480-554``) as its worker drives it
(``engine/runtime/t2w_worker.py:448-560, 642-665, 826-838``; ``FakeBT`` in ``tests/engine_api/test_t2w_worker_loop.py:52-82``
pins the minimal contract): ``setup_many``, ``setup_encode`` / ``release_presetup``, ``new_stream`` (with ``adopt``),
``decode(items, async_result=False, setups=None)``, ``release_stream``, ``release_prompt``, ``capture_graphs``, and the
attributes the loop reads (``max_flow_streams``, ``fuse_setup_frames``, ``fast``, ``profile``, ``trace``).

Prompt features keep the reference's tuple layout ``(tokens, tokens_len, spk, mels, mels_len)`` (``Token2Wav.features``,
``engine/models/token2wav.py:266-276``): ``tokens`` [1, n] codec tokens, ``spk`` [1, 192] the speaker embedding,
``mels`` [1, 2n, mel] the prompt mel (it sets the trim length).  A window is ``(stream, tokens, last)`` with the
chunker's tokens (a non-final window ends with 3 lookahead tokens).  Every call runs the flow encoder once over all its
token windows and token prompts (``FlowEncoder``), as ``_flow_encode`` does per group.

The encoder can be bypassed: a feature tuple whose first entry is the encoder's output ``mu`` [1, P, mel] (floating
point) and whose ``spk`` is already through the affine layer [1, mel] (``prompt_features`` builds one), and a window
``(stream, mu [mel, T], last)``, go straight to the solve (DiT + HiFT measurements and tests use this).

Per call: the flow encoder over the token windows, one packed ragged CFG Euler solve over every window (and fused prompt
setups), then HiFT over all windows in
one ragged call per source-cache length, then the per-stream glue of ``engine/models/token2wav.py:319-332`` (8 cached
mel frames, 3840 cached source / speech samples, Hamming cross-fade, first non-final chunk shifted by 3840 zeros,
non-final chunks hold back their last 3840 samples), and one device-to-host copy — synchronous, or through a pinned
buffer and an event (``PendingAudio``) so the caller does not wait for the GPU.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .config import MEL_CACHE, SOURCE_CACHE
from .dit import FastCache, FastDiT
from .flow import FlowEncoder, FlowState
from .hift import HiFTModel, HiftState, chunk_noise_seed, fade_in_out


def _is_tokens(x) -> bool:
    """Codec tokens (a list, an integer array or tensor) rather than an encoder output (a floating-point tensor)."""
    if isinstance(x, torch.Tensor):
        return not torch.is_floating_point(x)
    if isinstance(x, np.ndarray):
        return np.issubdtype(x.dtype, np.integer)
    return isinstance(x, (list, tuple))


def _token_list(x) -> list[int]:
    if isinstance(x, torch.Tensor):
        return x.reshape(-1).tolist()
    return np.asarray(x, dtype=np.int64).reshape(-1).tolist()


def prompt_features(mu: torch.Tensor, spk: torch.Tensor, mels: torch.Tensor) -> tuple:
    """A prompt-feature tuple in the reference layout for this module: ``mu`` [mel, P] (flow-encoder output of the
    prompt), ``spk`` [mel] (after the speaker affine layer), ``mels`` [mel, P] (the prompt mel)."""
    P = int(mels.shape[-1])
    n = torch.tensor([P], dtype=torch.int32)
    return (mu.t().reshape(1, P, -1), n, spk.reshape(1, -1), mels.t().reshape(1, P, -1), n)


@dataclass
class Prompt:
    """A set-up prompt: its features, speaker embedding (after the affine layer), estimator caches and flow-encoder
    caches (None for an encoder-output prompt)."""
    feats: tuple
    spk: torch.Tensor       # [1, mel]
    cache: FastCache | None
    flow: FlowState | None = None

    @property
    def mels(self) -> torch.Tensor:
        return self.feats[3]

    @property
    def frames(self) -> int:
        return int(self.feats[3].shape[1])


@dataclass
class PreSetup:
    """A prompt setup whose inputs are staged and caches allocated, not solved yet (``setup_encode``): ``decode(setups=)``
    and ``setup_many`` take it in place of the features; an unused one goes back with ``release_presetup``."""
    feats: tuple
    cache: FastCache | None
    mu: torch.Tensor        # [mel, P]
    spk: torch.Tensor       # [1, mel]
    cond: torch.Tensor      # [mel, P]
    flow: FlowState | None = None


@dataclass
class StreamState:
    prompt: Prompt
    cache: FastCache | None
    hift: HiftState = field(default_factory=HiftState)
    flow: FlowState | None = None

    @property
    def chunks(self) -> int:
        return self.hift.chunks

    @property
    def noise_seed(self) -> int:
        return self.hift.noise_seed


class _PinnedBlocks:
    """Reusable pinned host blocks for asynchronous results.  Blocks come in power-of-two sizes (at least 64 Ki
    samples); a block handed back after its copy finished serves the next result of its size class, so a steady
    decode loop stops allocating pinned memory after its first calls."""

    MIN = 1 << 16

    def __init__(self):
        self.free: dict[int, list[torch.Tensor]] = {}

    def take(self, n: int) -> torch.Tensor:
        size = max(self.MIN, 1 << max(0, int(n) - 1).bit_length())
        spare = self.free.get(size)
        return spare.pop() if spare else torch.empty(size, dtype=torch.float32, pin_memory=True)

    def give(self, block: torch.Tensor) -> None:
        self.free.setdefault(block.numel(), []).append(block)


class PendingAudio:
    """One decode call's samples on their way to the host (``async_result``; the worker's ``ready`` / ``result``
    contract, ``token2wav_batch.py:113-136``).  The packed samples are copied into a pinned block of the module's pool
    on the current stream, with an event behind the copy; the streams' host-side state is already advanced.
    ``ready()`` polls the event; ``result()`` waits for it once, splits the samples per item and hands the block back
    to the pool (later calls return the same arrays)."""

    def __init__(self, flat: torch.Tensor | None, lengths: list[int], blocks: _PinnedBlocks):
        self.lengths = [int(n) for n in lengths]
        self._blocks = blocks
        self._block = None
        self._out: list[np.ndarray] | None = None
        total = sum(self.lengths)
        if flat is not None and total:
            self._block = blocks.take(total)
            self._block[:total].copy_(flat, non_blocking=True)
        self.event = torch.cuda.Event()
        self.event.record()

    def ready(self) -> bool:
        return self._out is not None or self.event.query()

    def result(self) -> list[np.ndarray]:
        if self._out is None:
            self.event.synchronize()
            cuts = np.cumsum(self.lengths)[:-1]
            data = self._block.numpy()[: sum(self.lengths)] if self._block is not None else np.zeros(0, np.float32)
            self._out = [a.copy() for a in np.split(data, cuts)] if self.lengths else []
            if self._block is not None:
                self._blocks.give(self._block)
                self._block = None
        return self._out


class BatchedToken2Wav:
    def __init__(self, dit: FastDiT, hift: HiFTModel, flow: FlowEncoder | None = None, noise_device: str = "cuda", fuse_setup_frames: int = 0,
                 max_flow_streams: int = 32):
        """``flow``: the flow encoder (needed for codec-token prompts and windows).  ``noise_device``: where the
        per-chunk HiFT source noise is drawn ("cuda" as the reference's ``hift_noise``; "cpu" reproduces a host-generator
        draw bit for bit, used by the parity tests).  ``fuse_setup_frames``: prompt setups of up to this many mel frames
        in all may ride a decode call's solve (``decode(setups=...)``).  ``max_flow_streams``: requests per packed solve
        (larger calls run in slices)."""
        self.fast, self.hift, self.flow = dit, hift, flow
        self.device = dit.device
        self.noise_device = noise_device
        self.window = torch.from_numpy(np.hamming(2 * SOURCE_CACHE)).to(self.device)  # float64, as the reference's
        self.max_flow_streams = int(max_flow_streams)
        self.fuse_setup_frames = int(fuse_setup_frames)
        self.profile: dict | None = None  # stage -> [calls, seconds, items] when set (stages timed by events)
        self.trace = None
        self._open_stages: list[tuple] = []
        self._blocks = _PinnedBlocks()

    def _prof(self, name: str, n: int, fn, *a):
        """Run one stage of a call.  With ``profile`` set (a dict: stage -> [calls, seconds, items], the layout the
        reference's worker reads, ``token2wav_batch.py:197``), the stage is bracketed by two timing events on the
        current stream and its seconds are the GPU-side span between them: from the moment the stream reaches the
        stage (its earlier work done) to the stage's last kernel, host launch gaps included.  Nothing synchronises
        until the call's end, where ``_settle`` reads the events of every stage of the call."""
        if self.profile is None:
            return fn(*a)
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        r = fn(*a)
        t1.record()
        self._open_stages.append((name, int(n), t0, t1))
        return r

    def _settle(self) -> None:
        """Fold the timed stages of the finished call into ``profile``."""
        if not self._open_stages:
            return
        self._open_stages[-1][3].synchronize()
        for name, n, t0, t1 in self._open_stages:
            acc = self.profile.setdefault(name, [0, 0.0, 0]) if self.profile is not None else [0, 0.0, 0]
            acc[0] += 1
            acc[1] += t0.elapsed_time(t1) * 1e-3
            acc[2] += n
        self._open_stages = []

    # --- prompts ------------------------------------------------------------------------------------------------------
    def _stage_mu(self, feats: tuple) -> PreSetup:
        mu, _, spk, mels, _ = feats
        P = int(mels.shape[1])
        if mu.shape[1] != P:
            raise ValueError(f"prompt mu has {mu.shape[1]} frames, its mel {P}")
        dev = self.device
        return PreSetup(feats, self.fast.new_cache(keep=P), mu[0].to(dev, torch.float32).t(), spk.to(dev, torch.float32).reshape(1, -1),
                        mels[0].to(dev, torch.float32).t())

    def _stage_tokens(self, feats_list: list[tuple]) -> list[PreSetup]:
        """Token prompts: the flow encoder over every prompt (plus 3 silence tokens) in one call and the speaker affine
        layer over their embeddings (``_setup_encoder_batched``, ``token2wav_batch.py:567-616``)."""
        if self.flow is None:
            raise ValueError("codec-token prompts need the flow encoder (BatchedToken2Wav(flow=...))")
        toks = [_token_list(f[0]) for f in feats_list]
        for t, f in zip(toks, feats_list):
            if 2 * len(t) != int(f[3].shape[1]):
                raise ValueError(f"prompt of {len(t)} tokens needs a mel of {2 * len(t)} frames, got {int(f[3].shape[1])}")
        states, mu, rows, frames = self.flow.setup(toks)
        out: list[PreSetup] = []
        try:
            spk = self.flow.model.speaker(torch.cat([f[2].reshape(1, -1).to(self.device, torch.float32) for f in feats_list]))
            dev = self.device
            for i, f in enumerate(feats_list):
                P = frames[i]
                out.append(PreSetup(f, self.fast.new_cache(keep=P), mu[rows[i]:rows[i] + P].t(), spk[i:i + 1],
                                    f[3][0].to(dev, torch.float32).t(), states[i]))
        except Exception:  # give back every cache made so far and every encoder state (a pool ran out, say)
            for p in out:
                self.release_presetup(p)
            for st in states[len(out):]:
                self.flow.release(st)
            raise
        return out

    @torch.inference_mode()
    def setup_encode(self, feats_list: list[tuple]) -> list[PreSetup]:
        """Prompt setups staged ahead of their solve (``setup_encode``, ``token2wav_batch.py:480-485``): the flow encoder
        of token prompts run (one call for all), inputs on the device and empty estimator caches allocated."""
        out: list = [None] * len(feats_list)
        try:
            tok_idx = [i for i, f in enumerate(feats_list) if _is_tokens(f[0])]
            for i, p in zip(tok_idx, self._stage_tokens([feats_list[i] for i in tok_idx]) if tok_idx else []):
                out[i] = p
            for i, f in enumerate(feats_list):
                if out[i] is None:
                    out[i] = self._stage_mu(f)
        except Exception:
            for p in out:
                self.release_presetup(p)
            raise
        return out

    def release_presetup(self, p: PreSetup) -> None:
        if p is None:
            return
        if p.cache is not None:
            self.fast.release(p.cache)
            p.cache = None
        if p.flow is not None:
            self.flow.release(p.flow)
            p.flow = None

    def _presetups(self, setups: list) -> list[PreSetup]:
        raw = [s for s in setups if not isinstance(s, PreSetup)]
        staged = iter(self.setup_encode(raw) if raw else ())
        return [s if isinstance(s, PreSetup) else next(staged) for s in setups]

    @staticmethod
    def _prompt(p: PreSetup) -> Prompt:
        pr = Prompt(p.feats, p.spk, p.cache, p.flow)
        p.cache = p.flow = None  # the prompt owns the caches now
        return pr

    @torch.inference_mode()
    def setup_many(self, feats_list: list) -> list[Prompt]:
        """Prompt setups: one solve over every prompt's frames with its prompt mel as condition and empty caches
        (``token2wav_batch.py:507-554``, the fast-DiT branch).  Entries may be ``PreSetup``."""
        pre = self._presetups(feats_list)
        for a in range(0, len(pre), self.max_flow_streams):
            part = pre[a:a + self.max_flow_streams]
            self.fast.solve([p.cache for p in part], [p.mu for p in part], torch.cat([p.spk for p in part]), [p.cond for p in part],
                            [True] * len(part))
        return [self._prompt(p) for p in pre]

    def setup(self, feats) -> Prompt:
        return self.setup_many([feats])[0]

    # --- streams ------------------------------------------------------------------------------------------------------
    def new_stream(self, prompt: Prompt, noise_seed: int = 0, adopt: bool = False) -> StreamState:
        """A stream with its own copy of the prompt's caches, or taking them over (``adopt``: the prompt is used once).
        Flow-encoder caches are shared slot lists, so a copy costs no device work."""
        if adopt:
            cache, prompt.cache = prompt.cache, None
            flow, prompt.flow = prompt.flow, None
        else:
            cache = self.fast.clone(prompt.cache)
            flow = self.flow.clone(prompt.flow) if prompt.flow is not None else None
        return StreamState(prompt, cache, HiftState(noise_seed=noise_seed, device=self.device), flow)

    def release_stream(self, st: StreamState | None) -> None:
        if st is None:
            return
        if st.cache is not None:
            self.fast.release(st.cache)
            st.cache = None
        if st.flow is not None:
            self.flow.release(st.flow)
            st.flow = None

    def release_prompt(self, p: Prompt | None) -> None:
        if p is None:
            return
        if p.cache is not None:
            self.fast.release(p.cache)
            p.cache = None
        if p.flow is not None:
            self.flow.release(p.flow)
            p.flow = None

    @torch.inference_mode()
    def capture_graphs(self, prompt: Prompt | None = None) -> dict:
        """Capture every graph up front (``capture_graphs``, ``token2wav_batch.py:292-309``): the DiT's (rows, tokens)
        buckets and HiFT's steady shapes.  ``prompt`` is accepted for the reference's signature and not needed."""
        n = {}
        if self.fast.use_graphs:
            n["dit"] = self.fast.capture_all()
        if self.hift.use_graphs:
            n["hift"] = self.hift.capture_all()
        return n

    # --- decode -------------------------------------------------------------------------------------------------------
    def _encode_windows(self, items: list[tuple]) -> list[tuple]:
        """Items with codec tokens through the flow encoder (one call): ``(stream, mu [mel, T], last)`` for every item
        (``_flow_encode``, ``token2wav_batch.py:365-386``)."""
        idx = [i for i, (_, w, _) in enumerate(items) if _is_tokens(w)]
        if not idx:
            return items
        if self.flow is None:
            raise ValueError("codec-token windows need the flow encoder (BatchedToken2Wav(flow=...))")
        for i in idx:
            if items[i][0].flow is None:
                raise ValueError("a codec-token window needs a stream set up from a codec-token prompt")
        mu, rows, frames = self._prof("encoder", len(idx), self.flow.encode, [items[i][0].flow for i in idx],
                                      [_token_list(items[i][1]) for i in idx], [bool(items[i][2]) for i in idx])
        out = list(items)
        for k, i in enumerate(idx):
            st, _, last = items[i]
            out[i] = (st, mu[rows[k]:rows[k] + frames[k]].t(), last)
        return out

    @torch.inference_mode()
    def decode(self, items: list[tuple], async_result: bool = False, setups: list | None = None):
        """``items[i] = (stream, tokens, last)`` -> float32 24 kHz samples per item (``decode``,
        ``token2wav_batch.py:220-255``); ``tokens`` are the window's codec tokens (or the encoder's output ``mu``
        [mel, T]).  ``async_result``: a ``PendingAudio`` instead, without waiting for the GPU.  ``setups``
        (``fuse_setup_frames``): prompt features (or ``PreSetup``) set up in the same packed solve; then the result is
        ``(samples, prompts)``."""
        if setups:
            frames = sum(int((s.feats if isinstance(s, PreSetup) else s)[3].shape[1]) for s in setups)
            if not self.fuse_setup_frames or frames > self.fuse_setup_frames or len(items) + len(setups) > self.max_flow_streams:
                raise ValueError(f"fused setups: {len(setups)} prompts of {frames} frames with {len(items)} windows exceed "
                                 f"fuse_setup_frames={self.fuse_setup_frames} / max_flow_streams={self.max_flow_streams}")
        self._open_stages = []  # stage events of an earlier call that raised are dropped
        pre = self._presetups(setups) if setups else []
        items = self._encode_windows(items)
        rows = [(p.cache, p.mu, p.spk, p.cond, True) for p in pre]
        rows += [(st.cache, mu.to(self.device), st.prompt.spk, None, not last) for st, mu, last in items]
        mels = []
        for a in range(0, len(rows), self.max_flow_streams):
            part = rows[a:a + self.max_flow_streams]
            conds = [r[3] for r in part] if any(r[3] is not None for r in part) else None
            mels += self._prof("solve", len(part), self.fast.solve, [r[0] for r in part], [r[1] for r in part],
                               torch.cat([r[2] for r in part]), conds, [r[4] for r in part])
        prompts = [self._prompt(p) for p in pre]
        out = self._prof("vocode", len(items), self._vocode, items, mels[len(pre):], async_result)
        self._settle()
        return (out, prompts) if setups else out

    def _noise(self, seeds: list[int], n: int):
        dim = self.hift.dim
        gens = [torch.Generator(device=self.noise_device).manual_seed(int(s)) for s in seeds]
        rand_ini = torch.cat([torch.rand(1, dim, generator=g, device=self.noise_device) for g in gens])
        noise = torch.cat([torch.randn(1, dim, n, generator=g, device=self.noise_device) for g in gens]).transpose(1, 2)
        return rand_ini.to(self.device), noise.to(self.device)

    def _vocode(self, items, mels, async_result: bool = False):
        """HiFT per source-cache length (first windows have none), rows of different lengths in one call, then the
        reference's cross-fade, cache update and hold-back per stream (``token2wav_batch.py:813-848``)."""
        up = self.hift.cfg.upsample_scale
        full = [torch.cat([st.hift.mel, m[None].float()], dim=2) for (st, _, _), m in zip(items, mels)]
        groups: dict[int, list[int]] = {}
        for i, (st, _, _) in enumerate(items):
            groups.setdefault(int(st.hift.source.shape[2]), []).append(i)
        speech_of: dict[int, torch.Tensor] = {}
        source_of: dict[int, torch.Tensor] = {}
        for S, idx in groups.items():
            frames = [int(full[i].shape[2]) for i in idx]
            mel_tm = torch.cat([full[i][0].t() for i in idx])
            noises = [self._noise([chunk_noise_seed(items[i][0].noise_seed, items[i][0].chunks)], f * up) for i, f in zip(idx, frames)]
            noise_tm = torch.cat([nz[0] for _, nz in noises])
            cs = torch.cat([items[i][0].hift.source.reshape(1, -1) for i in idx]) if S else None
            sp, src, _ = self.hift.forward_packed(frames, mel_tm, noise_tm, cs, S)
            o = 0
            for i, f in zip(idx, frames):
                speech_of[i] = sp[o:o + f * up][None]
                source_of[i] = src[o:o + f * up].view(1, 1, -1)
                o += f * up
        pieces = []
        for i, (st, _, last) in enumerate(items):
            h = st.hift
            speech, source = speech_of[i], source_of[i]
            first = h.speech.shape[-1] == 0
            if not first:
                speech = fade_in_out(speech, h.speech, self.window)
            h.mel = full[i][..., -MEL_CACHE:].clone()
            h.source = source[:, :, -SOURCE_CACHE:].clone()
            h.speech = speech[:, -SOURCE_CACHE:].clone()
            h.chunks += 1
            sp = speech[0]
            if not last:
                sp = torch.cat([torch.zeros(SOURCE_CACHE, device=sp.device, dtype=sp.dtype), sp[:-SOURCE_CACHE]]) if first else sp[:-SOURCE_CACHE]
            pieces.append(sp)
        lengths = [int(p.numel()) for p in pieces]
        flat = torch.cat(pieces).float() if pieces else None
        if async_result:
            return PendingAudio(flat, lengths, self._blocks)
        host = flat.cpu().numpy() if flat is not None else np.zeros(0, np.float32)
        ends = np.cumsum(lengths)
        return [host[e - n:e] for n, e in zip(lengths, ends)]
