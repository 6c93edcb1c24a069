"""Co-scheduling without MPS: the module's work on a CU-masked stream of the engine's process gives the same bits as on
the default stream (every kernel's result is independent of how many CUs run its grid), for the packed 16 x 400
solve (bucket-less exact-shape graph) and for the worker-facing decode path (bucketed graphs, HiFT graphs)."""

import time

import numpy as np
import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd.config import DiTConfig, HiFTConfig
from t2w_amd.cosched import CUStream, device_cus
from t2w_amd.dit import DiTModel, FastDiT
from t2w_amd.hift import HiFTModel
from t2w_amd.token2wav import BatchedToken2Wav, prompt_features
from t2w_amd.weights import init_dit, init_hift

pytestmark = pytest.mark.gpu

TINY = DiTConfig(hidden=256, depth=2, heads=4, ffn=512)


def _on(n_cus, fn):
    if n_cus is None:
        out = fn()
        torch.cuda.synchronize()
        return out
    cs = CUStream(n_cus)
    try:
        with cs:
            out = fn()
        cs.stream.synchronize()
    finally:
        cs.close()
    return out


def test_packed_solve_same_bits_on_cu_masked_streams(dev):
    total = device_cus()
    model = DiTModel(init_dit(DiTConfig(), seed=2), DiTConfig())
    g = torch.Generator().manual_seed(3)
    mus = [torch.randn(80, 400, generator=g).cuda() for _ in range(16)]
    spks = torch.randn(16, 80, generator=g).cuda()
    outs, times = {}, {}
    for n_cus in (None, total // 2, total // 8):
        fd = FastDiT(model, n_slots=16 * 800 + 4096, max_streams=16, use_graphs=True)
        caches = [fd.new_cache() for _ in range(16)]

        def run():
            fd.solve(caches, mus, spks, None, [False] * 16, chunk=50)  # capture + first replay
            torch.cuda.current_stream().synchronize()
            t0 = time.perf_counter()
            o = fd.solve(caches, mus, spks, None, [False] * 16, chunk=50)
            torch.cuda.current_stream().synchronize()
            times[n_cus] = time.perf_counter() - t0
            return torch.cat(o, 1).cpu()

        outs[n_cus] = _on(n_cus, run)
        fd.drop_graphs()
    print("16 x 400 solve ms by CU share:", {k or total: round(v * 1e3, 1) for k, v in times.items()})
    ref = outs[None]
    assert all(torch.equal(v, ref) for v in outs.values())


def test_decode_same_bits_on_cu_masked_stream(dev):
    W, Wh = init_dit(TINY, seed=5), init_hift(HiFTConfig(), seed=6)
    model = DiTModel(W, TINY)
    g = torch.Generator().manual_seed(7)
    prompt = (torch.randn(80, 120, generator=g), torch.randn(80, generator=g), torch.randn(80, 120, generator=g))
    wins = [torch.randn(80, 50, generator=g) for _ in range(4)]
    audio = {}
    for n_cus in (None, 48):
        fd = FastDiT(model, n_slots=8192, max_streams=4, use_graphs=True)
        bt = BatchedToken2Wav(fd, HiFTModel(Wh, HiFTConfig(), use_graphs=True), noise_device="cpu")

        def run():
            st = bt.new_stream(bt.setup(prompt_features(*(x.cuda() for x in prompt))), noise_seed=3, adopt=True)
            out = [bt.decode([(st, w.cuda(), i == len(wins) - 1)])[0] for i, w in enumerate(wins)]
            bt.release_stream(st)
            return np.concatenate(out)

        audio[n_cus] = _on(n_cus, run)
        assert fd.counts["graph"] > 0
    assert audio[None].size > 0 and np.array_equal(audio[None], audio[48])


def test_interleaved_mask_refused(dev):
    """Masks that interleave single CUs or give a 32-CU group fewer than 8 are refused before any queue is made (the
    runtime would fail on them and the failure would stick to the process); a run-shaped mask works afterwards."""
    for bad in ([0x55555555] * 8, [0xF] * 8):
        with pytest.raises(RuntimeError, match="at least 8 consecutive CUs"):
            CUStream(mask=bad)
    cs = CUStream(mask=[0x0000FFFF] * 8)
    with cs:
        x = torch.ones(1024, device="cuda") * 3
    cs.stream.synchronize()
    cs.close()
    assert float(x.sum()) == 3072.0
