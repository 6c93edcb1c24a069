"""The library's launch timer (``t2w_timer_arm`` / ``t2w_timer_read``): it times the instrumented launches of an eager
call with HIP events and leaves the results unchanged; graph replays and capture are not timed."""

import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd import _lib
from t2w_amd.config import DiTConfig, HiFTConfig
from t2w_amd.dit import DiTModel, FastDiT
from t2w_amd.hift import HiFTModel
from t2w_amd.weights import init_dit, init_hift

pytestmark = pytest.mark.gpu

TINY = DiTConfig(hidden=256, depth=2, heads=4, ffn=512)


def test_solve_timed_counts_and_bits(dev):
    """A 2 x 700-frame solve (2,800 tokens: tile GEMMs) times 2 launches (proj, fc2) per block and step, and its mels
    equal an untimed eager solve's bit for bit."""
    model = DiTModel(init_dit(TINY, seed=12), TINY)
    g = torch.Generator().manual_seed(2)
    mus = [torch.randn(80, 700, generator=g).cuda() for _ in range(2)]
    spks = torch.randn(2, 80, generator=g).cuda()
    outs = []
    for timed in (False, True):
        fd = FastDiT(model, n_slots=8192, max_streams=2)
        caches = [fd.new_cache() for _ in range(2)]
        if timed:
            mels, launches = fd.solve_timed(caches, mus, spks, None, [False, False], chunk=50)
        else:
            mels = fd.solve(caches, mus, spks, None, [False, False], chunk=50)
        outs.append(torch.cat(mels, 1).cpu())
    assert torch.equal(outs[0], outs[1])
    assert len(launches) == 2 * TINY.depth * TINY.steps
    assert all(k == "resid_gemm" and ms > 0 and by > 0 for k, ms, by in launches)
    print("timed proj/fc2 launches", len(launches), "mean ms", sum(m for _, m, _ in launches) / len(launches))


def test_hift_stages_timed_and_graphs_untimed(dev):
    """HiFT's elementwise stages are timed in an eager call (strict fp32: Snake too); a graph replay records nothing."""
    W = init_hift(HiFTConfig(), seed=5)
    mel = torch.randn(2, 80, 30, generator=torch.Generator().manual_seed(1)).cuda() * 2 - 5
    src = torch.zeros(2, 1, 0, device="cuda")
    hm = HiFTModel(W, HiFTConfig())
    ri, nz = hm.noise([1, 2], 30 * 480)
    ref = hm.forward_noise(mel, src, ri, nz)[0]
    with _lib.LaunchTimer() as t:
        got = hm.forward_noise(mel, src, ri, nz)[0]
    assert torch.equal(ref, got)
    kinds = {k for k, _, _ in t.launches}
    assert {"hift_phase", "hift_source", "hift_stft", "hift_istft", "hift_reflect", "hift_f0_head", "hift_snake"} <= kinds
    hg = HiFTModel(W, HiFTConfig(), use_graphs=True)
    hg.forward_noise(mel, src, ri, nz)
    with _lib.LaunchTimer() as t2:
        hg.forward_noise(mel, src, ri, nz)
    assert t2.launches == [] and hg.counts["graph"] == 2
