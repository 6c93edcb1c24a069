"""DiT estimator and CFG Euler solve on the GPU against the fp32 CPU oracle (same seeded random-init weights/inputs).

Tolerance: bf16 GEMM operands with fp32 accumulation, fp16 residual stream (the reference's), fp32 Euler state: mel rel-L2 <= 2e-2 against
the fp32 oracle (the reference's own fast-vs-reference FP16 bounds are 2e-2 for setups and 3e-2 for windows,
``tests/engine/test_dit_fast.py:86,103`` of the reference); measured values are printed.
"""

import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd.config import DiTConfig
from t2w_amd.dit import DiTModel, FastDiT
from t2w_amd.weights import init_dit
from oracle import dit as od
from conftest import rel

pytestmark = pytest.mark.gpu

TINY = DiTConfig(hidden=256, depth=2, heads=4, ffn=512)
TOL = 2e-2


@pytest.fixture(scope="module")
def tiny():
    W = init_dit(TINY, seed=11)
    model = DiTModel(W, TINY)
    return W, model


@pytest.fixture(scope="module")
def full():
    W = init_dit(DiTConfig(), seed=0)
    model = DiTModel(W, DiTConfig())
    return W, model


def test_estimator_forward_config1(dev, full):
    """One estimator forward at the config-1 shape: B=2 rows, T=100, t=0.5, cond zeros, seed 0."""
    W, model = full
    fd = FastDiT(model, n_slots=1024, max_streams=2)
    g = torch.Generator().manual_seed(0)
    x, mu = torch.randn(2, 80, 100, generator=g), torch.randn(2, 80, 100, generator=g)
    spk = torch.randn(2, 80, generator=g)
    cond = torch.zeros(2, 80, 100)
    ref = od.estimator_forward(W, od.dims_of(W), x, mu, torch.full((2,), 0.5), spk, cond)
    got = fd.estimator_forward(x.cuda(), mu.cuda(), 0.5, spk.cuda(), cond.cuda()).cpu()
    e = rel(got, ref)
    print("config1 estimator rel-L2", e, "max-abs", float((got - ref).abs().max()))
    assert e < TOL


def test_estimator_forward_3000_tokens(dev, full):
    """One estimator forward with 3000 tokens (B=2 rows, T=1500, t=0.3): the N = 1024 and 2048 GEMMs run on 128 x 128
    tiles (a 256 x 256 grid would fill under a fifth of the CUs), the qkv projection with its fused q/k LayerNorm and
    key/value scatter on 144 tiles of 256 x 256."""
    W, model = full
    fd = FastDiT(model, n_slots=4096, max_streams=2)
    g = torch.Generator().manual_seed(3)
    x, mu = torch.randn(2, 80, 1500, generator=g), torch.randn(2, 80, 1500, generator=g)
    spk = torch.randn(2, 80, generator=g)
    cond = torch.randn(2, 80, 1500, generator=g) * 0.5
    ref = od.estimator_forward(W, od.dims_of(W), x, mu, torch.full((2,), 0.3), spk, cond)
    got = fd.estimator_forward(x.cuda(), mu.cuda(), 0.3, spk.cuda(), cond.cuda()).cpu()
    e = rel(got, ref)
    print("3000-token estimator rel-L2", e, "max-abs", float((got - ref).abs().max()))
    assert e < TOL


def _stream_case(W, model, graphs: bool, buckets: bool = False, outs: list | None = None, stats: dict | None = None,
                 prompts=(70, 40), oracle_rope: float | None = None):
    rope = model.cfg.rope_theta if oracle_rope is None else oracle_rope
    d = od.dims_of(W, steps=TINY.steps, rope_theta=rope)
    fd = FastDiT(model, n_slots=4096, max_streams=4, use_graphs=graphs, buckets=buckets)
    g = torch.Generator().manual_seed(1)
    n = len(prompts)
    caches = [fd.new_cache(keep=p) for p in prompts]
    refc = [od.empty_cache(d, keep=p) for p in prompts]
    spks = torch.randn(n, 80, generator=g)
    mus = [torch.randn(80, p, generator=g) for p in prompts]
    conds = [torch.randn(80, p, generator=g) for p in prompts]
    errs = []
    ref = od.solve(W, d, W["rand_noise"], refc, mus, spks, conds, [True, True])
    got = fd.solve(caches, [m.cuda() for m in mus], spks.cuda(), [c.cuda() for c in conds], [True, True])
    errs.append(max(rel(a.cpu(), b) for a, b in zip(got, ref)))
    if outs is not None:
        outs += [a.cpu() for a in got]
    for w in range(5):
        Ts = [50, 16 if w == 0 else 50][:n] if n > 1 else [16 if w == 0 else 50]
        keep = [w < 4, True][:n]
        if w == 4:
            Ts[0] = 34
        mus = [torch.randn(80, t, generator=g) for t in Ts]
        ref = od.solve(W, d, W["rand_noise"], refc, mus, spks, None, keep)
        got = fd.solve(caches, [m.cuda() for m in mus], spks.cuda(), None, keep)
        errs.append(max(rel(a.cpu(), b) for a, b in zip(got, ref)))
        if outs is not None:
            outs += [a.cpu() for a in got]
        assert [c.length for c in caches] == [c.length for c in refc], w
    for c in caches:
        fd.release(c)
    assert fd.pool.in_use() == fd.scratch
    if stats is not None:
        stats.update(fd.counts, n_graphs=len(fd.graphs))
    return errs


def test_solve_streaming_tiny(dev, tiny):
    """Prompt setups (cond = prompt mel), then windows past the trim point, a 16-frame first window and a final flush
    that keeps nothing, two requests per ragged call; caches and trims must follow the oracle's."""
    W, model = tiny
    errs = _stream_case(W, model, graphs=False)
    print("stream rel-L2 per call", errs)
    assert max(errs) < TOL


def test_solve_streaming_one_request(dev, tiny):
    """One request per call (120-token setup, then 32- to 100-token windows): every call has at most 128 tokens, so the
    gated-residual and conv GEMMs split K over four workgroups per tile and the row kernels finish their epilogues."""
    W, model = tiny
    errs = _stream_case(W, model, graphs=False, prompts=(60,))
    print("one-request stream rel-L2 per call", errs)
    assert max(errs) < TOL


def test_solve_streaming_one_request_graphs_equal_eager(dev, tiny):
    """The deferred GEMM epilogues replay bit for bit under graphs."""
    W, model = tiny
    assert _stream_case(W, model, graphs=False, prompts=(60,)) == _stream_case(W, model, graphs=True, prompts=(60,))


def test_solve_streaming_full_size_window(dev, full):
    """Full model size, one stream: a 100-frame prompt setup (200 tokens), then windows of 50 and 16 frames (100 and
    32 tokens: two and four K splits of the deferred GEMMs), each against the oracle."""
    W, model = full
    d = od.dims_of(W)
    fd = FastDiT(model, n_slots=4096, max_streams=2)
    g = torch.Generator().manual_seed(5)
    cache, refc = fd.new_cache(keep=100), od.empty_cache(d, keep=100)
    spk = torch.randn(1, 80, generator=g)
    mu, cond = torch.randn(80, 100, generator=g), torch.randn(80, 100, generator=g)
    errs = []
    ref = od.solve(W, d, W["rand_noise"], [refc], [mu], spk, [cond], [True])
    got = fd.solve([cache], [mu.cuda()], spk.cuda(), [cond.cuda()], [True])
    errs.append(rel(got[0].cpu(), ref[0]))
    for T in (50, 16):
        mu = torch.randn(80, T, generator=g)
        ref = od.solve(W, d, W["rand_noise"], [refc], [mu], spk, None, [True])
        got = fd.solve([cache], [mu.cuda()], spk.cuda(), None, [True])
        errs.append(rel(got[0].cpu(), ref[0]))
    fd.release(cache)
    print("full-size window rel-L2 per call", errs)
    assert max(errs) < TOL


def test_solve_streaming_graphs_equal_eager(dev, tiny):
    """Graphs keyed by the exact call shape replay the eager launches: identical results."""
    W, model = tiny
    a = _stream_case(W, model, graphs=False)
    b = _stream_case(W, model, graphs=True)
    print("exact-shape graphs vs oracle rel-L2 per call", b)
    assert a == b and max(b) < TOL


def test_solve_streaming_bucketed_graphs(dev, tiny):
    """Calls of 220, 132, 200 and 168 tokens over 2 requests all fall in the (4 rows, 256 tokens) bucket: one graph
    serves all six calls, with padding rows beside the real ones.  Padding changes GEMM row counts (so the split-K plan
    and its summation order), so the results match the eager solve to 1e-3 rather than bit for bit, and the oracle to the
    usual tolerance."""
    W, model = tiny
    ea, ga, st = [], [], {}
    _stream_case(W, model, graphs=False, outs=ea)
    errs = _stream_case(W, model, graphs=True, buckets=True, outs=ga, stats=st)
    d = max(rel(a, b) for a, b in zip(ga, ea))
    print("bucketed graphs vs eager rel-L2", d, "vs oracle", errs, st)
    assert st["graph"] == 6 and st["n_graphs"] == 1
    assert d < 1e-3 and max(errs) < TOL


def test_captured_buckets_serve_long_caches(dev, tiny):
    """Graphs captured up front on padding-only plans (``capture``) serve prompt setups and steady windows over caches
    of 300-450 frames without a capture mid-stream, and match the eager solve."""
    from t2w_amd.dit import bucket_of

    W, model = tiny
    fdg = FastDiT(model, n_slots=8192, max_streams=4, use_graphs=True, buckets=True)
    fde = FastDiT(model, n_slots=8192, max_streams=4)
    prompts = (300, 380)
    fdg.capture(*bucket_of(4, 2 * sum(prompts)))
    fdg.capture(*bucket_of(4, 2 * 100))
    held = set(fdg.graphs)
    g = torch.Generator().manual_seed(21)
    spks = torch.randn(2, 80, generator=g).cuda()
    cg = [fdg.new_cache(keep=p) for p in prompts]
    ce = [fde.new_cache(keep=p) for p in prompts]
    calls = [([torch.randn(80, p, generator=g).cuda() for p in prompts], [torch.randn(80, p, generator=g).cuda() for p in prompts])]
    calls += [([torch.randn(80, 50, generator=g).cuda() for _ in prompts], None) for _ in range(3)]
    worst = 0.0
    for mus, conds in calls:
        a = fdg.solve(cg, mus, spks, conds, [True, True])
        b = fde.solve(ce, mus, spks, conds, [True, True])
        worst = max(worst, max(rel(x.cpu(), y.cpu()) for x, y in zip(a, b)))
    print("captured buckets vs eager rel-L2", worst, "cached frames", [c.length for c in cg], fdg.counts)
    assert min(c.length for c in cg) > 256
    assert set(fdg.graphs) == held and fdg.counts["graph"] == 4
    assert worst < 1e-3


def test_chunk_causal_many_rows(dev, tiny):
    """16 requests x 700 frames (22,400 tokens): the qkv GEMM's 264 tiles of 256 x 256 leave a mostly idle last round,
    so its last 640 rows run on 256 x 128 tiles with the q/k LayerNorm and key scatter of their own rows."""
    W, model = tiny
    d = od.dims_of(W, steps=TINY.steps)
    fd = FastDiT(model, n_slots=32768, max_streams=16)
    g = torch.Generator().manual_seed(6)
    Ts = [700] * 16
    mus = [torch.randn(80, t, generator=g) for t in Ts]
    spks = torch.randn(16, 80, generator=g)
    ref = od.solve(W, d, W["rand_noise"], [od.empty_cache(d) for _ in Ts], mus, spks, None, [False] * 16, chunk=50)
    caches = [fd.new_cache() for _ in Ts]
    got = fd.solve(caches, [m.cuda() for m in mus], spks.cuda(), None, [False] * 16, chunk=50)
    errs = [rel(a.cpu(), b) for a, b in zip(got, ref)]
    print("many-row chunk-causal rel-L2 max", max(errs))
    assert max(errs) < TOL


def test_chunk_causal_whole_sequence(dev, tiny):
    """A whole 150-frame row per request under the chunk-causal mask (chunk 50) equals the oracle's."""
    W, model = tiny
    d = od.dims_of(W, steps=TINY.steps)
    fd = FastDiT(model, n_slots=4096, max_streams=4)
    g = torch.Generator().manual_seed(2)
    Ts = [150, 120, 37]
    mus = [torch.randn(80, t, generator=g) for t in Ts]
    spks = torch.randn(3, 80, generator=g)
    ref = od.solve(W, d, W["rand_noise"], [od.empty_cache(d) for _ in Ts], mus, spks, None, [False] * 3, chunk=50)
    caches = [fd.new_cache() for _ in Ts]
    got = fd.solve(caches, [m.cuda() for m in mus], spks.cuda(), None, [False] * 3, chunk=50)
    errs = [rel(a.cpu(), b) for a, b in zip(got, ref)]
    print("chunk-causal rel-L2", errs)
    assert max(errs) < TOL


FP8_TOL = 5e-2  # fp8 (e4m3 weights, MX fp8 activations) against the bf16 result: the bound stated for config 5


def _solve_once(model, fp8: bool, Ts, seed: int, chunk: int):
    fd = FastDiT(model, n_slots=4096, max_streams=4, fp8=fp8)
    g = torch.Generator().manual_seed(seed)
    caches = [fd.new_cache() for _ in Ts]
    mus = [torch.randn(80, t, generator=g).cuda() for t in Ts]
    spks = torch.randn(len(Ts), 80, generator=g).cuda()
    out = fd.solve(caches, mus, spks, None, [False] * len(Ts), chunk=chunk)
    for c in caches:
        fd.release(c)
    return [o.cpu() for o in out]


def test_fp8_solve_vs_bf16_full_size(dev):
    """Config-5 form at the full model size: 10-step CFG solve with fp8 block GEMMs against the bf16 solve."""
    W = init_dit(DiTConfig(), seed=4)
    model = DiTModel(W, DiTConfig(), fp8=True)
    Ts = [200, 130]
    b = _solve_once(model, False, Ts, 4, 50)
    f = _solve_once(model, True, Ts, 4, 50)
    e = max(rel(x, y) for x, y in zip(f, b))
    print("fp8 vs bf16 mel rel-L2", e, "max-abs", max(float((x - y).abs().max()) for x, y in zip(f, b)))
    assert e < FP8_TOL


def test_fp8_streaming_vs_oracle(dev):
    """fp8 streaming windows with caches (small model) against the fp32 oracle, same structure as the bf16 case."""
    W = init_dit(TINY, seed=12)
    model = DiTModel(W, TINY, fp8=True)
    d = od.dims_of(W, steps=TINY.steps)
    fd = FastDiT(model, n_slots=4096, max_streams=4, fp8=True)
    g = torch.Generator().manual_seed(2)
    caches = [fd.new_cache(keep=30)]
    refc = [od.empty_cache(d, keep=30)]
    spks = torch.randn(1, 80, generator=g)
    errs = []
    for w, T in enumerate([30, 50, 50]):
        mus = [torch.randn(80, T, generator=g)]
        conds = [torch.randn(80, T, generator=g)] if w == 0 else None
        ref = od.solve(W, d, W["rand_noise"], refc, mus, spks, conds, [True])
        got = fd.solve(caches, [m.cuda() for m in mus], spks.cuda(), [c.cuda() for c in conds] if conds else None, [True])
        errs.append(rel(got[0].cpu(), ref[0]))
    print("fp8 streaming vs oracle rel-L2 per window", errs)
    assert max(errs) < FP8_TOL


ROPE = DiTConfig(hidden=256, depth=2, heads=4, ffn=512, rope_theta=10000.0)


@pytest.fixture(scope="module")
def tiny_rope():
    """Random weights whose q / k LayerNorm gains are scaled by 8: sharper attention, so that the rotary embedding
    moves the mel by ~3% (with the plain gains it moves it by 0.4%, inside the tolerance)."""
    W = init_dit(ROPE, seed=11)
    for b in range(ROPE.depth):
        for n in ("q_norm", "k_norm"):
            W[f"blocks.{b}.attn.{n}.weight"] = W[f"blocks.{b}.attn.{n}.weight"] * 8
    return W, DiTModel(W, ROPE)


def test_rope_streaming(dev, tiny_rope):
    """The optional rotary embedding (none in the reference) against the oracle's: prompt setups and windows past the
    trim point, so keys cached at earlier stream positions meet queries at later ones.  Setups and two-request windows
    (132 to 220 tokens) rotate in the split-K path's q/k kernel, one-request windows (at most 128 tokens) in the
    small-row GEMM's epilogue.  Every call is also at least 5x further from the oracle without the embedding."""
    W, model = tiny_rope
    errs = _stream_case(W, model, graphs=False) + _stream_case(W, model, graphs=False, prompts=(60,))
    plain = _stream_case(W, model, graphs=False, oracle_rope=0.0) + _stream_case(W, model, graphs=False, prompts=(60,), oracle_rope=0.0)
    print("rope stream rel-L2 per call", errs, "against the oracle without rope", plain)
    assert max(errs) < TOL
    assert all(p > 5 * e for p, e in zip(plain, errs))


def test_rope_bucketed_graphs(dev, tiny_rope):
    """Bucketed graph replays carry the stream positions (their table sits before the variable-length key lists)."""
    W, model = tiny_rope
    ea, ga = [], []
    _stream_case(W, model, graphs=False, outs=ea)
    errs = _stream_case(W, model, graphs=True, buckets=True, outs=ga)
    d = max(rel(a, b) for a, b in zip(ga, ea))
    print("rope bucketed graphs vs eager rel-L2", d, "vs oracle", errs)
    assert d < 1e-3 and max(errs) < TOL


def test_rope_tile_path(dev, tiny_rope):
    """16 requests x 700 frames (11,200 tokens): the qkv projection on 256 x 256 tiles with its fused q/k LayerNorm,
    then the separate rotation kernel over q rows and key slots.  Sampled rows against the oracle with and without
    the embedding."""
    W, model = tiny_rope
    fd = FastDiT(model, n_slots=32768, max_streams=16)
    g = torch.Generator().manual_seed(16)
    Ts = [700] * 16
    mus = [torch.randn(80, t, generator=g) for t in Ts]
    spks = torch.randn(16, 80, generator=g)
    caches = [fd.new_cache() for _ in Ts]
    got = fd.solve(caches, [m.cuda() for m in mus], spks.cuda(), None, [False] * 16, chunk=50)
    idx = (0, 7, 15)
    res = {}
    for theta in (ROPE.rope_theta, 0.0):
        d = od.dims_of(W, steps=ROPE.steps, rope_theta=theta)
        ref = od.solve(W, d, W["rand_noise"], [od.empty_cache(d) for _ in idx], [mus[i] for i in idx], spks[list(idx)], None,
                       [False] * len(idx), chunk=50)
        res[theta] = [rel(got[i].cpu(), r) for i, r in zip(idx, ref)]
    errs, plain = res[ROPE.rope_theta], res[0.0]
    print("rope tile-path rel-L2 (rows 0, 7, 15)", errs, "against the oracle without rope", plain)
    assert max(errs) < TOL
    assert all(p > 5 * e for p, e in zip(plain, errs))


@pytest.mark.parametrize("chunk", [0, 25])
def test_estimator_chunk_dense_caches(dev, tiny, chunk):
    """The estimator on dense caches as the reference module passes them (``_estimator_temb``): 2 rows of 50 new frames
    over 70 cached frames per row, against the oracle's ``estimator_chunk`` with the same caches and mask.  The cached
    keys come back as the bf16 of what went in, the new keys / values and conv frames as the oracle's to bf16 accuracy."""
    W, model = tiny
    d = od.dims_of(W, steps=TINY.steps)
    fd = FastDiT(model, n_slots=4096, max_streams=2)
    g = torch.Generator().manual_seed(17)
    B, T, L, H = 2, 50, 70, TINY.hidden
    x, mu, cond = (torch.randn(B, 80, T, generator=g) for _ in range(3))
    spk = torch.randn(B, 80, generator=g)
    att = torch.randn(d.depth, B, d.heads, L, 2 * d.head_dim, generator=g)
    cnn = torch.randn(d.depth, B, 2 * H, 2, generator=g)
    t = 0.4
    mask = torch.ones(B, T, T + L, dtype=torch.bool)
    mask[:, :, :T] = od.chunk_mask(T, chunk)
    ref, ref_cnn, ref_att = od.estimator_chunk(W, d, x, mu, od.t_embed(W, torch.full((B,), t)), spk, cond, cnn, att, mask,
                                               torch.full((B,), T))
    got, got_cnn, got_att = fd.estimator_chunk(x.cuda(), mu.cuda(), t, spk.cuda(), cond.cuda(), cnn.cuda(), att.cuda(), chunk=chunk)
    e, ec, ea = rel(got.cpu(), ref), rel(got_cnn.cpu(), ref_cnn), rel(got_att[:, :, :, :T].cpu(), ref_att[:, :, :, :T])
    print("dense-cache estimator rel-L2: dphi", e, "new conv cache", ec, "new keys / values", ea)
    assert e < TOL and ec < 1e-2 and ea < 1e-2
    assert torch.equal(got_att[:, :, :, T:].cpu(), att.bfloat16().float())
    assert fd.pool.in_use() == fd.scratch


def _dequantized_weights(W, model8, cfg):
    """The plain weights W with every block GEMM weight replaced by its e4m3 codes times their per-channel scale (fp32),
    in W's own layouts: a bf16 model of these holds exactly what the weight-only fp8 solve computes with."""
    H = cfg.hidden
    Wd = dict(W)
    for b, blk8 in enumerate(model8.blocks8):
        deq = {k: blk8[k + "_w8"].cpu().view(torch.float8_e4m3fn).float() * blk8[k + "_ws"].cpu()[:, None]
               for k in ("qkv", "proj", "c1", "c2", "fc1", "fc2")}
        p, a = f"blocks.{b}.", f"blocks.{b}.attn."
        Wd[a + "to_q.weight"], Wd[a + "to_k.weight"], Wd[a + "to_v.weight"] = deq["qkv"].split(H)
        Wd[a + "proj.weight"] = deq["proj"]
        Wd[p + "conv.block.1.weight"] = deq["c1"].reshape(H, 3, H).permute(0, 2, 1).contiguous()
        Wd[p + "conv.block.6.weight"] = deq["c2"].reshape(H, 3, H).permute(0, 2, 1).contiguous()
        Wd[p + "mlp.fc1.weight"], Wd[p + "mlp.fc2.weight"] = deq["fc1"], deq["fc2"]
    return Wd


@pytest.mark.parametrize("graphs", [False, True])
def test_fp8_weights_mode_is_bf16_on_dequantized_weights(dev, graphs):
    """fp8="weights" (e4m3 weights with per-output-channel scales, bf16 activations and MFMA): a streaming solve (setups,
    windows at 100 tokens with their deferred GEMMs, a 1,400-token call on tile GEMMs) equals, bit for bit, the bf16
    solve of a model whose weights are the dequantized ones -- the dequantization is bf16(e4m3 x scale), nothing more."""
    W = init_dit(TINY, seed=13)
    model8 = DiTModel(W, TINY, fp8=True)
    modeld = DiTModel(_dequantized_weights(W, model8, TINY), TINY)
    g = torch.Generator().manual_seed(3)
    spk = torch.randn(2, 80, generator=g).cuda()
    calls = [([torch.randn(80, 60, generator=g).cuda() for _ in range(2)], True),
             ([torch.randn(80, 50, generator=g).cuda() for _ in range(2)], False),
             ([torch.randn(80, 700, generator=g).cuda() for _ in range(2)], False)]
    outs = []
    for model, mode in ((model8, "weights"), (modeld, False)):
        fd = FastDiT(model, n_slots=8192, max_streams=2, use_graphs=graphs, fp8=mode)
        caches = [fd.new_cache(keep=60) for _ in range(2)]
        res = []
        for mus, cond in calls:
            res.append(torch.cat(fd.solve(caches, mus, spk, [m * 0.5 for m in mus] if cond else None, [True, True]), 1).cpu())
        outs.append(torch.cat(res, 1))
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("graphs", [False, True])
def test_fp8_weights_mode_large_call(dev, graphs):
    """fp8="weights" on a call of 8,400 CFG tokens (2 streams x 2,100 frames, chunk 50), where every block GEMM is a tile
    GEMM of 256-row tiles: still bit for bit the bf16 solve of the dequantized weights, and within bf16 solve error of
    the fp32 oracle on those weights."""
    W = init_dit(TINY, seed=17)
    model8 = DiTModel(W, TINY, fp8=True)
    Wd = _dequantized_weights(W, model8, TINY)
    modeld = DiTModel(Wd, TINY)
    g = torch.Generator().manual_seed(5)
    spk = torch.randn(2, 80, generator=g)
    mus = [torch.randn(80, 2100, generator=g) for _ in range(2)]
    outs = []
    for model, mode in ((model8, "weights"), (modeld, False)):
        fd = FastDiT(model, n_slots=16384, max_streams=2, use_graphs=graphs, fp8=mode)
        caches = [fd.new_cache() for _ in range(2)]
        outs.append(torch.cat(fd.solve(caches, [m.cuda() for m in mus], spk.cuda(), None, [False, False], chunk=50), 1).cpu())
    assert torch.equal(outs[0], outs[1])
    d = od.dims_of(Wd, steps=TINY.steps)
    ref = od.solve(Wd, d, Wd["rand_noise"], [od.empty_cache(d) for _ in range(2)], mus, spk, None, [False, False], chunk=50)
    assert rel(outs[0], torch.cat(ref, 1)) < TOL
