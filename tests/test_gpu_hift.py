"""HiFT on the GPU against the fp32 CPU oracle (same seeded random-init weights, mel and source noise).

Stages are checked separately so that each bound measures one kernel family: the f0 predictor; the NSF source given the
oracle's f0 (the frame-rate phase reaches ~1e5 rad over a 400-frame row, so any f0 difference is amplified by sin); the
decoder + ISTFT given the oracle's source.  End to end, the strict-fp32 bound of the reference
(``tests/engine/test_token2wav_stream.py:54``: waveform rel-L2 1e-4) holds for the decoder; the strict-fp32 chain end
to end is held to 5e-4 (it measures ~4e-5: its f0 matches the oracle's to 2e-6, too little for the phase to amplify),
the bf16 decoders to the reference's reduced-precision HiFT bound of 1e-2 (``tests/engine/test_hift_tf32.py:227``).
"""

import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd.config import HiFTConfig
from t2w_amd.hift import HiFTModel
from t2w_amd.weights import init_hift
from oracle import hift as oh
from conftest import rel

pytestmark = pytest.mark.gpu

LENS = [50, 58, 123, 17]


@pytest.fixture(scope="module")
def case():
    W = init_hift(HiFTConfig(), seed=3)
    g = torch.Generator().manual_seed(3)
    mels = [torch.randn(1, 80, t, generator=g) * 2 - 5 for t in LENS]
    noise = [oh.hift_noise(9, [100 + i], t * 480) for i, t in enumerate(LENS)]
    h = oh.HiFT(W)
    return W, h, HiFTModel(W, HiFTConfig()), mels, noise


def _packed(mels, noise):
    mel_tm = torch.cat([m[0].t() for m in mels]).cuda()
    noise_tm = torch.cat([nz[0] for _, nz in noise]).cuda()
    return mel_tm, noise_tm


def test_f0_predictor(dev, case):
    W, h, gm, mels, noise = case
    mel_tm, noise_tm = _packed(mels, noise)
    _, _, f0 = gm.forward_packed(LENS, mel_tm, noise_tm, None, 0, want_f0=True)
    ref = torch.cat([h.f0_predictor(m)[0] for m in mels])
    e = rel(f0.cpu(), ref)
    print("f0 rel-L2", e)
    assert e < 1e-5


def test_source_given_f0(dev, case):
    W, h, gm, mels, noise = case
    mel_tm, noise_tm = _packed(mels, noise)
    f0s = [h.f0_predictor(m) for m in mels]
    f0_tm = torch.cat([f[0] for f in f0s]).cuda()
    _, src, _ = gm.forward_packed(LENS, mel_tm, noise_tm, None, 0, f0_override=f0_tm)
    ref = torch.cat([oh.source(h, m, torch.zeros(1, 1, 0), ri, nz, f0=f)[0, 0] for m, (ri, nz), f in zip(mels, noise, f0s)])
    e = rel(src.cpu(), ref)
    print("source rel-L2 (oracle f0)", e, "max-abs", float((src.cpu() - ref).abs().max()))
    assert e < 1e-4


def test_decoder_given_source(dev, case):
    W, h, gm, mels, noise = case
    mel_tm, noise_tm = _packed(mels, noise)
    srcs = [oh.source(h, m, torch.zeros(1, 1, 0), ri, nz) for m, (ri, nz) in zip(mels, noise)]
    s_tm = torch.cat([s[0, 0] for s in srcs]).cuda()
    sp, _, _ = gm.forward_packed(LENS, mel_tm, noise_tm, None, 0, source_override=s_tm)
    ref = torch.cat([oh.decode(h, m, s)[0] for m, s in zip(mels, srcs)])
    e = rel(sp.cpu(), ref)
    print("decoder rel-L2 (oracle source)", e)
    assert e < 1e-4


def test_forward_noise_end_to_end_with_cache(dev, case):
    """Equal-length rows through ``forward_noise`` with a 3840-sample source cache (a steady 58-frame window), strict
    fp32 end to end: f0, source and decoder agree with the oracle closely enough that the phase integration does not
    amplify anything (measured rel-L2 3.8e-5 speech, 5.0e-5 source), so the bound is 5e-4 rather than the
    reduced-precision 1e-2 of the bf16 tests."""
    W, h, gm, mels, noise = case
    g = torch.Generator().manual_seed(8)
    mel = torch.randn(3, 80, 58, generator=g) * 2 - 5
    cs = torch.randn(3, 1, 3840, generator=g) * 0.01
    ri, nz = oh.hift_noise(9, [5, 6, 7], 58 * 480)
    sp, src = gm.forward_noise(mel.cuda(), cs.cuda(), ri.cuda(), nz.cuda())
    rsp, rsrc = oh.forward_noise(h, mel, cs, ri, nz)
    e_sp, e_src = rel(sp.cpu(), rsp), rel(src.cpu(), rsrc)
    print("end-to-end speech rel-L2", e_sp, "source rel-L2", e_src)
    assert torch.equal(src[:, :, :3840].cpu(), cs)
    assert e_sp < 5e-4 and e_src < 5e-4


@pytest.mark.parametrize("fusion", ["auto", "on"])
def test_decoder_bf16_given_source(dev, case, fusion):
    """The bf16-MFMA decoder (fp32 activations and accumulation) against the strict-fp32 oracle on the oracle's source:
    the reference's reduced-precision HiFT bound, waveform rel-L2 <= 1e-2 (``tests/engine/test_hift_tf32.py:227``).
    "on" runs every ResBlock dilation as one kernel (rows of 17 to 123 frames: one to thirty workgroups per row)."""
    W, h, gm, mels, noise = case
    gb = HiFTModel(W, HiFTConfig(), decode_bf16=True, resblock_fusion=fusion)
    mel_tm, noise_tm = _packed(mels, noise)
    srcs = [oh.source(h, m, torch.zeros(1, 1, 0), ri, nz) for m, (ri, nz) in zip(mels, noise)]
    s_tm = torch.cat([s[0, 0] for s in srcs]).cuda()
    sp, _, _ = gb.forward_packed(LENS, mel_tm, noise_tm, None, 0, source_override=s_tm)
    ref = torch.cat([oh.decode(h, m, s)[0] for m, s in zip(mels, srcs)])
    e = rel(sp.cpu(), ref)
    print("bf16 decoder rel-L2 (oracle source)", e)
    assert e < 1e-2


def test_forward_bf16_end_to_end(dev, case):
    W, h, gm, mels, noise = case
    gb = HiFTModel(W, HiFTConfig(), decode_bf16=True)
    g = torch.Generator().manual_seed(9)
    mel = torch.randn(2, 80, 58, generator=g) * 2 - 5
    cs = torch.randn(2, 1, 3840, generator=g) * 0.01
    ri, nz = oh.hift_noise(9, [5, 6], 58 * 480)
    sp, src = gb.forward_noise(mel.cuda(), cs.cuda(), ri.cuda(), nz.cuda())
    rsp, rsrc = oh.forward_noise(h, mel, cs, ri, nz)
    e = rel(sp.cpu(), rsp)
    print("bf16 end-to-end speech rel-L2", e, "source", rel(src.cpu(), rsrc))
    assert e < 1e-2


@pytest.mark.parametrize("fusion", ["auto", "on"])
def test_forward_bf16_streaming_window(dev, case, fusion):
    """One 50-frame window with a source cache (the per-chunk call of a stream): with "auto" every decoder conv runs on
    the small-grid kernels (32 output channels per workgroup where the grid allows); "on" fuses the ResBlock dilations."""
    W, h, gm, mels, noise = case
    gb = HiFTModel(W, HiFTConfig(), decode_bf16=True, resblock_fusion=fusion)
    g = torch.Generator().manual_seed(12)
    mel = torch.randn(1, 80, 50, generator=g) * 2 - 5
    cs = torch.randn(1, 1, 3840, generator=g) * 0.01
    ri, nz = oh.hift_noise(9, [11], 50 * 480)
    sp, src = gb.forward_noise(mel.cuda(), cs.cuda(), ri.cuda(), nz.cuda())
    rsp, rsrc = oh.forward_noise(h, mel, cs, ri, nz)
    e = rel(sp.cpu(), rsp)
    print("bf16 50-frame window speech rel-L2", e, "source", rel(src.cpu(), rsrc))
    assert e < 1e-2


def test_resblock_fusion_equals_two_kernels():
    """Fused ResBlock dilations (conv1's output kept on chip) against the same dilations as two conv kernels.  On a call
    large enough for the two-kernel path's whole-slab tiles (eight rows of 150 to 220 frames; "auto" fuses stages 1 and
    2 and keeps stage 0 as two convs) both sum each output's products in the same order and round at the same points:
    equal bit for bit.  On rows of 1 to 7 frames (one partial workgroup per row) the two-kernel path's small-grid
    kernels split the sums over waves, which moves a bf16 rounding now and then (measured rel-L2 1.5e-3)."""
    W = init_hift(HiFTConfig(), seed=4)
    g = torch.Generator().manual_seed(4)
    for lens in ([150, 220, 171, 200, 163, 209, 188, 195], [1, 7, 3, 2]):
        mel_tm = torch.cat([torch.randn(t, 80, generator=g) * 2 - 5 for t in lens]).cuda()
        outs = {}
        for fusion in ("off", "auto", "on"):
            hm = HiFTModel(W, HiFTConfig(), decode_bf16=True, resblock_fusion=fusion)
            ri, nz = hm.noise([50 + i for i in range(len(lens))], max(lens) * 480)
            noise_tm = torch.cat([nz[i, : t * 480] for i, t in enumerate(lens)])
            sp, src, _ = hm.forward_packed(lens, mel_tm, noise_tm, None, 0)
            outs[fusion] = sp.cpu()
            assert torch.isfinite(outs[fusion]).all()
        e_auto, e_on = rel(outs["auto"], outs["off"]), rel(outs["on"], outs["off"])
        print("rows", lens, "fused vs two-kernel rel-L2: auto", e_auto, "on", e_on)
        if max(lens) >= 150:
            assert torch.equal(outs["auto"], outs["off"]) and torch.equal(outs["on"], outs["off"])
        else:
            assert torch.equal(outs["auto"], outs["off"]) and e_on < 5e-3


def test_hift_graphs_equal_eager():
    """Graph replays (one graph per row lengths and source-cache length) equal eager calls bit for bit, replay after
    replay with new inputs, eager work and synchronisations in between; a second key gets its own graph."""
    W = init_hift(HiFTConfig(), seed=5)
    eager = HiFTModel(W, HiFTConfig(), decode_bf16=True)
    graphed = HiFTModel(W, HiFTConfig(), decode_bf16=True, use_graphs=True)
    g = torch.Generator().manual_seed(8)
    for rep, (lens, S) in enumerate([([58, 58], 3840), ([58, 58], 3840), ([50, 20, 7], 0), ([58, 58], 3840), ([50, 20, 7], 0)]):
        mel = [torch.randn(t, 80, generator=g) * 2 - 5 for t in lens]
        mel_tm = torch.cat(mel).cuda()
        ri, nz = eager.noise([rep * 10 + i for i in range(len(lens))], max(lens) * 480)
        noise_tm = torch.cat([nz[i, : t * 480] for i, t in enumerate(lens)])
        cs = torch.randn(len(lens), S, generator=g).cuda() * 0.1 if S else None
        sp_e, src_e, _ = eager.forward_packed(lens, mel_tm, noise_tm, cs, S)
        torch.cuda.synchronize()
        sp_g, src_g, _ = graphed.forward_packed(lens, mel_tm, noise_tm, cs, S)
        torch.cuda.synchronize()
        assert torch.equal(sp_e, sp_g) and torch.equal(src_e, src_g), (rep, lens)
    assert graphed.counts["graph"] == 5 and len(graphed.graphs) == 2


def test_call_with_seeds(dev, case):
    """``HiFTModel(mel, cache_source, seeds)`` (the ``HiFTGraphs.__call__`` contract): noise drawn from each row's seed
    -- on the host generator it is the oracle's ``hift_noise`` draw (speech within the strict bound of the oracle fed the
    same seeds), on the device it is what the reference's device generators give (equal to ``forward_noise`` on that
    draw, bit for bit); a graph replay of the same call gives the same bits."""
    W, h, gm, mels, noise = case
    mel = torch.cat([m[:, :, :50] for m in mels[:3]])
    cs = torch.randn(3, 1, 480, generator=torch.Generator().manual_seed(9)) * 0.1
    seeds = [11, 12, 13]
    sp, src = gm(mel.cuda(), cs.cuda(), seeds, noise_device="cpu")
    ri, nz = oh.hift_noise(9, seeds, 50 * 480)
    rsp, rsrc = oh.forward_noise(h, mel, cs, ri, nz)
    e = rel(sp.cpu(), rsp)
    print("seeded call vs oracle rel-L2", e)
    assert e < 5e-4 and torch.equal(src.cpu()[:, :, :480], cs)
    a = gm(mel.cuda(), cs.cuda(), seeds)
    gens = [torch.Generator(device="cuda").manual_seed(s) for s in seeds]
    ri_d = torch.cat([torch.rand(1, 9, generator=g, device="cuda") for g in gens])
    nz_d = torch.cat([torch.randn(1, 9, 50 * 480, generator=g, device="cuda") for g in gens]).transpose(1, 2)
    b = gm.forward_noise(mel.cuda(), cs.cuda(), ri_d, nz_d)
    assert torch.equal(a[0], b[0])
    gg = HiFTModel(W, HiFTConfig(), use_graphs=True)
    assert torch.equal(gg(mel.cuda(), cs.cuda(), seeds)[0], a[0]) and gg.counts["graph"] == 1
