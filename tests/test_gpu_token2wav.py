"""The worker-facing Token2Wav surface on the GPU against the oracle pipeline, stream by stream.

Three streams with prompts of different lengths set up in one call, then decoded in staggered ragged calls (steady
windows, first windows with no HiFT cache, final flushes) past the trim point.  Two bounds, each measuring one part:

* every window's mel from the packed GPU solve against the oracle solving that stream alone: rel-L2 < 2e-2 (bf16);
* each stream's audio against the oracle's vocode glue (``engine/models/token2wav.py:319-332``) run on the same GPU
  mels with the same host-drawn noise: rel-L2 < 1e-4 (the reference's strict-fp32 stream bound,
  ``tests/engine/test_token2wav_stream.py:54``).

End to end (oracle mels into the oracle vocoder) the bf16 mel error is amplified by the NSF phase integration of HiFT
(f0 -> ~1e4 rad of phase per window), so that figure is printed, not bounded.
"""

import numpy as np
import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd.config import DiTConfig, HiFTConfig
from t2w_amd.dit import DiTModel, FastDiT
from t2w_amd.hift import HiFTModel
from t2w_amd.token2wav import BatchedToken2Wav, PendingAudio, prompt_features
from t2w_amd.weights import init_dit, init_hift
from oracle import dit as od
from oracle import hift as oh
from conftest import rel

pytestmark = pytest.mark.gpu

TINY = DiTConfig(hidden=256, depth=2, heads=4, ffn=512)


def test_batched_decode_matches_oracle_per_stream(dev):
    W, Wh = init_dit(TINY, seed=21), init_hift(HiFTConfig(), seed=22)
    fd = FastDiT(DiTModel(W, TINY), n_slots=8192, max_streams=8)
    bt = BatchedToken2Wav(fd, HiFTModel(Wh), noise_device="cpu")
    d = od.dims_of(W)
    h = oh.HiFT(Wh)
    g = torch.Generator().manual_seed(4)
    P = [60, 30, 45]
    feats = [(torch.randn(80, p, generator=g), torch.randn(80, generator=g), torch.randn(80, p, generator=g)) for p in P]
    prompts = bt.setup_many([prompt_features(m.cuda(), s.cuda(), c.cuda()) for m, s, c in feats])
    sts = [bt.new_stream(p, noise_seed=j, adopt=True) for j, p in enumerate(prompts)]
    # oracle streams
    rc = [od.empty_cache(d, keep=p) for p in P]
    for i, (m, s, c) in enumerate(feats):
        od.solve(W, d, W["rand_noise"], [rc[i]], [m], s[None], [c], [True])
    rh = [oh.new_hift_state(noise_seed=j) for j in range(3)]
    plans = [[50, 50, 50, 50, 22], [50, 50, 50, 8], [16, 50, 50, 50, 50, 50, 34]]
    starts = [0, 2, 1]
    windows = [[torch.randn(80, t, generator=g) for t in pl] for pl in plans]
    got, ref, e2e = [[], [], []], [[], [], []], [[], [], []]
    rh2 = [oh.new_hift_state(noise_seed=j) for j in range(3)]
    seen = []
    solve = fd.solve

    def recording_solve(*a, **k):
        out = solve(*a, **k)
        seen.extend(out)
        return out

    fd.solve = recording_solve
    mel_err = []
    for tick in range(max(s + len(p) for s, p in zip(starts, plans))):
        items, who = [], []
        for j in range(3):
            k = tick - starts[j]
            if 0 <= k < len(plans[j]):
                last = k == len(plans[j]) - 1
                items.append((sts[j], windows[j][k].cuda(), last))
                who.append((j, k, last))
        seen.clear()
        wavs = bt.decode(items)
        for (j, k, last), wav, gm in zip(who, wavs, list(seen)):
            got[j].append(wav)
            mel = od.solve(W, d, W["rand_noise"], [rc[j]], [windows[j][k]], feats[j][1][None], None, [not last])[0]
            gm = gm.float().cpu()
            mel_err.append(float((gm - mel).norm() / mel.norm()))
            ref[j].append(oh.vocode_chunk(h, rh[j], gm[None], last))
            e2e[j].append(oh.vocode_chunk(h, rh2[j], mel[None], last))
    print("window mel rel-L2 max", max(mel_err))
    assert max(mel_err) < 2e-2
    for j in range(3):
        a, b = np.concatenate(got[j]), np.concatenate(ref[j])
        assert a.shape == b.shape, (j, a.shape, b.shape)
        e = float(np.linalg.norm(a - b) / np.linalg.norm(b))
        c = np.concatenate(e2e[j])
        print("stream", j, "waveform rel-L2 (same mels)", e, "end to end", float(np.linalg.norm(a - c) / np.linalg.norm(c)))
        assert e < 1e-4
        assert sts[j].cache.length == rc[j].length
    for st in sts:
        bt.release_stream(st)
    assert fd.pool.in_use() == fd.scratch


def _stream_pair(W, Wh, cfg, P, windows, seed, graphs=False):
    """One stream through the module: a P-frame prompt setup, then the windows (the last one final); returns the module's
    audio per window, its GPU mels, and the oracle's mels and vocode glue on those GPU mels."""
    fd = FastDiT(DiTModel(W, cfg), n_slots=4096, max_streams=2, use_graphs=graphs)
    bt = BatchedToken2Wav(fd, HiFTModel(Wh, use_graphs=graphs), noise_device="cpu")
    d = od.dims_of(W)
    h = oh.HiFT(Wh)
    g = torch.Generator().manual_seed(seed)
    mu, spk, pm = torch.randn(80, P, generator=g), torch.randn(80, generator=g), torch.randn(80, P, generator=g)
    st = bt.new_stream(bt.setup(prompt_features(mu.cuda(), spk.cuda(), pm.cuda())), noise_seed=seed, adopt=True)
    rc = od.empty_cache(d, keep=P)
    od.solve(W, d, W["rand_noise"], [rc], [mu], spk[None], [pm], [True])
    rh = oh.new_hift_state(noise_seed=seed)
    seen, solve = [], fd.solve

    def recording_solve(*a, **k):
        out = solve(*a, **k)
        seen.extend(out)
        return out

    fd.solve = recording_solve
    mel_err, got, ref = [], [], []
    for k, T in enumerate(windows):
        last = k == len(windows) - 1
        w = torch.randn(80, T, generator=g)
        seen.clear()
        got.append(bt.decode([(st, w.cuda(), last)])[0])
        gm = seen[0].float().cpu()
        mel = od.solve(W, d, W["rand_noise"], [rc], [w], spk[None], None, [not last])[0]
        mel_err.append(rel(gm, mel))
        ref.append(oh.vocode_chunk(h, rh, gm[None], last))
    bt.release_stream(st)
    assert fd.pool.in_use() == fd.scratch
    return mel_err, got, ref


@pytest.mark.parametrize("graphs", [False, True])
def test_config2_chunk_full_size(dev, graphs):
    """The streaming chunk of the latency workload at full model size: a 300-frame prompt setup (600 tokens with the CFG
    pair), then a 50-frame first window and a 50-frame final window through ``decode`` (DiT + HiFT + glue).  With
    graphs the DiT solves replay bucket graphs and HiFT its own graphs, as in the latency bench, against the oracle."""
    W, Wh = init_dit(DiTConfig(), seed=1), init_hift(HiFTConfig(), seed=1)
    mel_err, got, ref = _stream_pair(W, Wh, DiTConfig(), 300, [50, 50], seed=1, graphs=graphs)
    a, b = np.concatenate(got), np.concatenate(ref)
    e = float(np.linalg.norm(a - b) / np.linalg.norm(b))
    print("config-2 window mel rel-L2", mel_err, "audio vs oracle glue on the same mels", e)
    assert max(mel_err) < 2e-2 and e < 1e-4


def test_worker_call_sequence(dev):
    """The worker's sequence of calls (``engine/runtime/t2w_worker.py:448-560, 642-665, 826-838``) with graphs on:
    startup prompt set up, ``capture_graphs``, that prompt released; stats reads; ``setup_many`` + ``new_stream(adopt)``;
    asynchronous decodes polled with ``ready()`` and collected with ``result()``; a prefetched setup (``setup_encode``)
    fused into a decode (``decode(setups=...)``) and adopted; an unused prefetched setup released; streams released.
    Asynchronous audio equals a second module's synchronous audio bit for bit (same graphs, same inputs), and every
    slot comes back."""
    W, Wh = init_dit(TINY, seed=31), init_hift(HiFTConfig(), seed=32)

    def module():
        fd = FastDiT(DiTModel(W, TINY), n_slots=8192, max_streams=8, use_graphs=True)
        return BatchedToken2Wav(fd, HiFTModel(Wh, decode_bf16=True, use_graphs=True), fuse_setup_frames=200, max_flow_streams=8)

    bt, ref = module(), module()
    g = torch.Generator().manual_seed(5)
    feat = lambda P: prompt_features(torch.randn(80, P, generator=g).cuda(), torch.randn(80, generator=g).cuda(),  # noqa: E731
                                     torch.randn(80, P, generator=g).cuda())
    stats = lambda b: (b.fast.pool.in_use() - b.fast.scratch, len(b.fast.cnn_free), b.fast.counts["graph"], b.fast.counts["eager"])  # noqa: E731
    free0 = len(bt.fast.cnn_free)
    p0 = bt.setup(feat(40))
    n = bt.capture_graphs(p0)
    bt.release_prompt(p0)
    print("captured", n, "stats", stats(bt))
    assert n["dit"] > 0 and n["hift"] > 0 and stats(bt)[:2] == (0, free0)
    feats = [feat(60), feat(35), feat(50)]
    streams = {}
    for b in (bt, ref):
        ps = b.setup_many(feats[:2])
        streams[id(b)] = [b.new_stream(p, noise_seed=10 + j, adopt=True) for j, p in enumerate(ps)]
    windows = [[torch.randn(80, T, generator=g).cuda() for T in (16, 50, 50, 30)] for _ in range(3)]
    out_async, out_sync = [[], [], []], [[], [], []]
    for k in range(4):
        last = k == 3
        if k == 1:  # prefetch the third prompt's setup while a call runs, then fuse it into this decode
            pre = bt.setup_encode([feats[2]])
            spare = bt.setup_encode([feat(20)])
            pend, prompts = bt.decode([(st, windows[j][k], last) for j, st in enumerate(streams[id(bt)])], async_result=True, setups=pre)
            streams[id(bt)].append(bt.new_stream(prompts[0], noise_seed=12, adopt=True))
            bt.release_presetup(spare[0])
            wavs, rp = ref.decode([(st, windows[j][k], last) for j, st in enumerate(streams[id(ref)])], setups=ref.setup_encode([feats[2]]))
            streams[id(ref)].append(ref.new_stream(rp[0], noise_seed=12, adopt=True))
        else:
            items = [(st, windows[j][k], last) for j, st in enumerate(streams[id(bt)])]
            pend = bt.decode(items, async_result=True)
            wavs = ref.decode([(st, windows[j][k], last) for j, st in enumerate(streams[id(ref)])])
        assert isinstance(pend, PendingAudio)
        while not pend.ready():
            pass
        res = pend.result()
        for j, (a, b) in enumerate(zip(res, wavs)):
            out_async[j].append(a)
            out_sync[j].append(b)
        print("decode", k, "stats", stats(bt))
    for j in range(3):
        a, b = np.concatenate(out_async[j]), np.concatenate(out_sync[j])
        print("stream", j, "samples", a.size, "async vs sync max-abs", float(np.abs(a - b).max()) if a.size else 0.0)
        assert a.shape == b.shape and np.array_equal(a, b)
    assert sum(x.size for x in out_async[2]) > 0
    for b in (bt, ref):
        for st in streams[id(b)]:
            b.release_stream(st)
    assert stats(bt)[:2] == (0, free0)
    assert bt.fast.counts["graph"] > 0


def test_codec_tokens_end_to_end_mels(dev):
    """Codec-token prompts and windows (the reference's ``decode(items)`` surface): the flow encoder, speaker affine
    layer, prompt-mel conditioning and the solve against the oracle pipeline (oracle encoder -> oracle solve) per
    stream; DiT at hidden 256, encoder at full width.  Mel rel-L2 < 2e-2."""
    from oracle import flow as of
    from t2w_amd.config import FlowConfig
    from t2w_amd.flow import FlowEncoder, FlowModel
    from t2w_amd.weights import init_flow

    W, Wh, Wf = init_dit(TINY, seed=31), init_hift(HiFTConfig(), seed=32), init_flow(FlowConfig(), seed=33)
    fd = FastDiT(DiTModel(W, TINY), n_slots=8192, max_streams=8)
    enc = FlowEncoder(FlowModel(Wf, FlowConfig()), n_slots1=4096, n_slots2=8192, n_cnn=64)
    bt = BatchedToken2Wav(fd, HiFTModel(Wh), flow=enc, noise_device="cpu")
    d, fdims = od.dims_of(W), of.enc_dims_of(Wf)
    g = torch.Generator().manual_seed(6)
    toks = [torch.randint(0, 6561, (1, n), generator=g) for n in (40, 25)]
    spks = [torch.randn(1, 192, generator=g) for _ in toks]
    mels = [torch.randn(1, 2 * t.shape[1], 80, generator=g) for t in toks]
    feats = [(t, torch.tensor([t.shape[1]]), s, m, torch.tensor([m.shape[1]])) for t, s, m in zip(toks, spks, mels)]
    seen = []
    solve = fd.solve

    def recording_solve(*a, **k):
        out = solve(*a, **k)
        seen.extend(out)
        return out

    fd.solve = recording_solve
    prompts = bt.setup_many(feats)
    sts = [bt.new_stream(p, noise_seed=j) for j, p in enumerate(prompts)]
    # oracle: encoder setup, speaker affine, prompt solve with the prompt mel as condition
    rf, rc, rspk = [], [], []
    for t, s, m in zip(toks, spks, mels):
        mu0, fst = of.setup(Wf, fdims, t[0].tolist())
        rf.append(fst)
        rspk.append(of.speaker(Wf, s))
        rc.append(od.empty_cache(d, keep=m.shape[1]))
        od.solve(W, d, W["rand_noise"], [rc[-1]], [mu0], rspk[-1], [m[0].t()], [True])
    errs = []
    plan = [(28, False), (28, False), (28, False), (28, False), (17, True)]
    for k, (n, last) in enumerate(plan):
        wins = [torch.randint(0, 6561, (n,), generator=g).tolist() for _ in sts]
        seen.clear()
        bt.decode([(st, w, last) for st, w in zip(sts, wins)])
        for j in range(2):
            mu = of.encode_window(Wf, fdims, rf[j], wins[j], last)
            mel = od.solve(W, d, W["rand_noise"], [rc[j]], [mu], rspk[j], None, [not last])[0]
            errs.append(rel(seen[j].float().cpu(), mel))
    print("token windows: mel rel-L2 max", max(errs))
    assert max(errs) < 2e-2
    for p in prompts:
        bt.release_prompt(p)
    for st in sts:
        bt.release_stream(st)
    assert fd.pool.in_use() == fd.scratch and enc.in_use() == (0, 0, 0)


def test_exhausted_pools_leak_nothing(dev):
    """Pool exhaustion inside a token-prompt setup (the estimator's conv-cache rows run out after the encoder ran) and
    inside an encoder call (its conv-cache slots run out after the key slots were taken) raises, and every slot the
    failed call took is back: the pools read as before the call."""
    from t2w_amd.config import FlowConfig
    from t2w_amd.flow import FlowEncoder, FlowModel
    from t2w_amd.weights import init_flow

    W, Wh, Wf = init_dit(TINY, seed=41), init_hift(HiFTConfig(), seed=42), init_flow(FlowConfig(), seed=43)
    fd = FastDiT(DiTModel(W, TINY), n_slots=4096, max_streams=1)  # 4 conv rows + 2 reserved: one stream's caches
    enc = FlowEncoder(FlowModel(Wf, FlowConfig()), n_slots1=1024, n_slots2=2048, n_cnn=3)
    bt = BatchedToken2Wav(fd, HiFTModel(Wh), flow=enc, noise_device="cpu")
    g = torch.Generator().manual_seed(8)
    toks = [torch.randint(0, 6561, (1, n), generator=g) for n in (20, 15)]
    feats = [(t, torch.tensor([t.shape[1]]), torch.randn(1, 192, generator=g), torch.randn(1, 2 * t.shape[1], 80, generator=g),
              torch.tensor([2 * t.shape[1]])) for t in toks]
    before = (enc.in_use(), fd.pool.in_use(), len(fd.cnn_free))
    with pytest.raises(RuntimeError, match="conv-cache row slots exhausted"):
        bt.setup_encode(feats)  # the encoder serves both prompts, the second estimator cache does not fit
    assert (enc.in_use(), fd.pool.in_use(), len(fd.cnn_free)) == before
    states = [enc.new_state(0) for _ in range(3)]
    with pytest.raises(RuntimeError):
        enc.encode(states, [t[0].tolist() for t in toks] + [toks[0][0].tolist()], [False] * 3)  # 3 conv slots, 2 free
    assert enc.in_use() == before[0]
    for st in states:
        enc.release(st)
    assert enc.in_use() == before[0]
