"""Co-scheduling the Token2Wav module with other work of the same process on one GPU, without CUDA MPS.

The reference gives Token2Wav a worker process of its own and shares the GPU with the Thinker/Talker process through
MPS (``engine/runtime/t2w_worker.py:858-924``, ``scripts/serve_engine.sh:1-45``, ``docs/architecture.md:54-62``).  On
the MI355X the module can live in the engine's process instead: its launches (graph replays included) go to the
current stream, so running it under a stream of its own lets the engine's other streams proceed beside it, and a
CU-masked stream (``t2w_stream_create_cu_mask``) bounds the CUs it may occupy, which leaves the rest to the other
work.  Every kernel of the module is an ordinary grid whose results do not depend on how many CUs run it, so the
outputs on a masked stream equal those on the default stream bit for bit.
"""

from __future__ import annotations

import ctypes as C

import torch

from . import _lib


def device_cus() -> int:
    n = C.c_int()
    _lib.check(_lib.lib().t2w_device_cus(C.byref(n)), "device_cus")
    return n.value


MIN_GROUP_CUS = 8  # CUs a 32-CU group of a mask holds at least, when it holds any (the runtime refuses fewer)


def spread_mask(n_cus: int, total: int | None = None) -> list[int]:
    """A CU mask (32-bit words, bit i of word w = CU 32 w + i) of ``n_cus`` of the device's ``total`` CUs: as many
    32-CU groups as can hold ``MIN_GROUP_CUS`` each (all of them for shares of 64 CUs and more at 256) take equal
    shares (the first ones one more when the share does not divide), each as a run of consecutive CUs from the group's
    first.  The runtime refuses masks that interleave single CUs or leave a group fewer than 8 CUs."""
    total = device_cus() if total is None else int(total)
    n_cus = int(n_cus)
    sizes = [min(32, total - 32 * w) for w in range((total + 31) // 32)]
    if not MIN_GROUP_CUS <= n_cus <= total:
        raise ValueError(f"a share of {n_cus} CUs of {total} (at least {MIN_GROUP_CUS})")
    groups = max(1, min(len(sizes), n_cus // MIN_GROUP_CUS))
    per, extra = divmod(n_cus, groups)
    words = [0] * len(sizes)
    taken = 0
    for w in range(groups):
        k = min(sizes[w], per + (1 if w < extra else 0))
        words[w] = (1 << k) - 1
        taken += k
    for w, size in enumerate(sizes):  # groups that could not take their share (a short last group): others take the rest
        if taken >= n_cus:
            break
        k = bin(words[w]).count("1")
        add = min(size - k, n_cus - taken) if k else (min(size, n_cus - taken) if n_cus - taken >= MIN_GROUP_CUS else 0)
        words[w] = (1 << (k + add)) - 1
        taken += add
    if taken != n_cus:
        raise ValueError(f"no mask of {n_cus} CUs fits groups of {sizes} with at least {MIN_GROUP_CUS} CUs each")
    return words


class CUStream:
    """A stream of the current device restricted to a set of CUs (default priority).  ``with cs:`` makes it torch's
    current stream, so every launch of the module in the block goes there; ``close()`` (or garbage collection)
    releases it after waiting for its work."""

    def __init__(self, n_cus: int | None = None, mask: list[int] | None = None):
        if (n_cus is None) == (mask is None):
            raise ValueError("give either n_cus or mask")
        words = spread_mask(n_cus) if mask is None else [int(w) & 0xFFFFFFFF for w in mask]
        arr = (C.c_uint32 * len(words))(*words)
        h = C.c_void_p()
        _lib.check(_lib.lib().t2w_stream_create_cu_mask(arr, len(words), C.byref(h)), "stream_create_cu_mask")
        self.handle = h
        self.mask = words
        self.n_cus = sum(bin(w).count("1") for w in words)
        self.stream = torch.cuda.ExternalStream(h.value)
        self._ctx = None

    def __enter__(self):
        self._ctx = torch.cuda.stream(self.stream)
        self._ctx.__enter__()
        return self

    def __exit__(self, *exc):
        ctx, self._ctx = self._ctx, None
        return ctx.__exit__(*exc)

    def close(self) -> None:
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.stream.synchronize()
            _lib.lib().t2w_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
