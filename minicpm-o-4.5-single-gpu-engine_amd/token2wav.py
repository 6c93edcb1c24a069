"""The Token2Wav module surface the reference's worker calls, over the MI355X DiT solve and HiFT.

Mirrors ``BatchedToken2Wav`` (``engine/runtime/token2wav_batch.py:151-309, 480-554``) as its worker uses it
(``FakeBT`` in ``tests/engine_api/test_t2w_worker_loop.py:52-82`` pins that contract): ``setup_many``, ``new_stream``
(with ``adopt``), ``decode``, ``release_stream``, ``release_prompt``.  The flow encoder (codec tokens -> ``mu``) is the
next stage to be built, so windows and prompts enter as encoder outputs: a window is ``(stream, mu [mel, T], last)`` and
a prompt setup is ``(mu [mel, P], spk [mel] (after the speaker affine layer), prompt mel [mel, P])``.

Per call: one packed ragged CFG Euler solve over every window (``keep`` = not last, as the reference's
``_flow_finish``/``dit_fast.solve``), then HiFT over all windows in one ragged call per source-cache length (first
windows have no cache), then the per-stream glue of ``engine/models/token2wav.py:319-332`` (8 cached mel frames, 3840
cached source / speech samples, Hamming cross-fade, first non-final chunk shifted by 3840 zeros, non-final chunks hold
back their last 3840 samples), and one device-to-host copy (``token2wav_batch.py:847``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .config import MEL_CACHE, SOURCE_CACHE
from .dit import FastCache, FastDiT
from .hift import HiFTModel, HiftState, chunk_noise_seed, fade_in_out


@dataclass
class Prompt:
    spk: torch.Tensor            # [mel] after the speaker affine layer
    frames: int                  # prompt mel frames (the trim length)
    cache: FastCache | None      # estimator caches after the setup solve


@dataclass
class StreamState:
    prompt: Prompt
    cache: FastCache | None
    hift: HiftState = field(default_factory=HiftState)

    @property
    def chunks(self) -> int:
        return self.hift.chunks

    @property
    def noise_seed(self) -> int:
        return self.hift.noise_seed


class BatchedToken2Wav:
    def __init__(self, dit: FastDiT, hift: HiFTModel, noise_device: str = "cuda"):
        """``noise_device``: where the per-chunk HiFT source noise is drawn ("cuda" as the reference's ``hift_noise``;
        "cpu" reproduces a host-generator draw bit for bit, used by the parity tests)."""
        self.fast, self.hift = dit, hift
        self.device = dit.device
        self.noise_device = noise_device
        self.window = torch.from_numpy(np.hamming(2 * SOURCE_CACHE)).to(self.device)  # float64, as the reference's
        self.max_flow_streams = 32
        self.fuse_setup_frames = 0
        self.profile = None
        self.trace = None

    # --- prompts and streams ------------------------------------------------------------------------------------------
    @torch.inference_mode()
    def setup_many(self, feats: list[tuple]) -> list[Prompt]:
        """Prompt setups: one solve over every prompt's frames with its prompt mel as condition and empty caches
        (``token2wav_batch.py:507-554``, the fast-DiT branch)."""
        caches = [self.fast.new_cache(keep=int(mu.shape[1])) for mu, _, _ in feats]
        spks = torch.stack([s.to(self.device, torch.float32).reshape(-1) for _, s, _ in feats])
        self.fast.solve(caches, [mu.to(self.device) for mu, _, _ in feats], spks, [c.to(self.device) for _, _, c in feats],
                        [True] * len(feats))
        return [Prompt(spks[i], int(mu.shape[1]), c) for i, ((mu, _, _), c) in enumerate(zip(feats, caches))]

    def new_stream(self, prompt: Prompt, noise_seed: int = 0, adopt: bool = False) -> StreamState:
        """A stream with its own copy of the prompt's caches, or taking them over (``adopt``: the prompt is used once)."""
        if adopt:
            cache, prompt.cache = prompt.cache, None
        else:
            cache = self.fast.clone(prompt.cache)
        return StreamState(prompt, cache, HiftState(noise_seed=noise_seed, device=self.device))

    def release_stream(self, st: StreamState | None) -> None:
        if st is not None and st.cache is not None:
            self.fast.release(st.cache)
            st.cache = None

    def release_prompt(self, p: Prompt | None) -> None:
        if p is not None and p.cache is not None:
            self.fast.release(p.cache)
            p.cache = None

    # --- decode -------------------------------------------------------------------------------------------------------
    @torch.inference_mode()
    def decode(self, items: list[tuple[StreamState, torch.Tensor, bool]]) -> list[np.ndarray]:
        """``items[i] = (stream, mu [mel, T_i], last)`` -> float32 24 kHz samples per item."""
        if not items:
            return []
        mels = []
        for a in range(0, len(items), self.max_flow_streams):
            part = items[a:a + self.max_flow_streams]
            mels += self.fast.solve([st.cache for st, _, _ in part], [mu.to(self.device) for _, mu, _ in part],
                                    torch.stack([st.prompt.spk for st, _, _ in part]), None, [not last for _, _, last in part])
        return self._vocode(items, mels)

    def _noise(self, seeds: list[int], n: int):
        dim = self.hift.dim
        gens = [torch.Generator(device=self.noise_device).manual_seed(int(s)) for s in seeds]
        rand_ini = torch.cat([torch.rand(1, dim, generator=g, device=self.noise_device) for g in gens])
        noise = torch.cat([torch.randn(1, dim, n, generator=g, device=self.noise_device) for g in gens]).transpose(1, 2)
        return rand_ini.to(self.device), noise.to(self.device)

    def _vocode(self, items, mels) -> list[np.ndarray]:
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
        flat = torch.cat(pieces).float().cpu().numpy()
        out, o = [], 0
        for p in pieces:
            out.append(flat[o:o + p.numel()])
            o += p.numel()
        return out
