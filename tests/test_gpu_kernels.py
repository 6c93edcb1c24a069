"""Kernel-level parity on the GPU: each HIP kernel against a plain PyTorch fp32 computation of the same op."""

import ctypes as C

import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd import _lib
from conftest import rel
from oracle import fp8 as of

pytestmark = pytest.mark.gpu


def _gemm(A, W, bias, C_, epi, gate=None, a_src=None, lda=None, K=None, ws=None):
    L = _lib.lib()
    M = C_.shape[0] if a_src is None else a_src.numel()
    N = W.shape[0]
    K = K or A.shape[1]
    if ws is None:
        _lib.check(L.t2w_gemm_bf16(A.data_ptr(), lda or A.shape[1], _lib.ptr(a_src), W.data_ptr(), bias.data_ptr(), _lib.ptr(gate),
                                   C_.data_ptr(), C_.shape[1], M, N, K, epi, _lib.stream_handle()), "gemm")
    else:
        _lib.check(L.t2w_gemm_bf16_ws(A.data_ptr(), lda or A.shape[1], _lib.ptr(a_src), W.data_ptr(), bias.data_ptr(), _lib.ptr(gate),
                                      C_.data_ptr(), C_.shape[1], M, N, K, epi, ws.data_ptr(), ws.numel(), _lib.stream_handle()), "gemm")
    torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K", [(1, 256, 64), (100, 80, 1024), (333, 1024, 320), (1000, 3072, 1024), (257, 2048, 2048),
                                   (5400, 3072, 1024)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 7])
def test_gemm_dense(dev, M, N, K, epi):
    """5400 x 3072: 264 tiles of 256 x 256, so the rows of the first full round run on 256 x 256 tiles and the last
    24 rows on 256 x 128 tiles (a second round of 8 tiles would leave most CUs idle)."""
    g = torch.Generator(device=dev).manual_seed(M * 7 + N + K + epi)
    A = torch.randn(M, K, device=dev, generator=g).bfloat16()
    W = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).bfloat16()
    bias = torch.randn(N, device=dev, generator=g)
    ref = A.float() @ W.float().t() + bias
    if epi in (0, 1):
        out = torch.full((M, N), 7.0, device=dev).bfloat16()
        _gemm(A, W, bias, out, epi)
        if epi == 1:
            ref = torch.nn.functional.gelu(ref, approximate="tanh")
        assert rel(out.float(), ref) < 6e-3
    elif epi == 2:  # the fp16 residual stream: h = fp16(h + gate * (.))
        h = torch.randn(M, N, device=dev, generator=g).half()
        gate = torch.randn(N, device=dev, generator=g)
        expect = h.float() + gate * ref
        _gemm(A, W, bias, h, 2, gate=gate)
        assert rel(h.float(), expect) < 1e-3
    elif epi == 7:
        out = torch.zeros(M, N, device=dev).half()
        _gemm(A, W, bias, out, 7)
        assert rel(out.float(), ref) < 1e-3
    else:
        out = torch.zeros(M, N, device=dev)
        _gemm(A, W, bias, out, 3)
        assert rel(out, ref) < 1e-5


def test_gemm_row_split_taps(dev):
    """The row split of a mostly idle last round in taps mode: the second launch reads its frames through the frame ids
    of its own rows."""
    M, N, H = 5400, 3072, 1024
    g = torch.Generator(device=dev).manual_seed(77)
    P = torch.randn(M + 40, H, device=dev, generator=g).bfloat16()
    a_src = (torch.arange(M, device=dev) + torch.arange(M, device=dev) // 300 * 2).int()
    W = (torch.randn(N, 3 * H, device=dev, generator=g) / (3 * H) ** 0.5).bfloat16()
    bias = torch.randn(N, device=dev, generator=g)
    out = torch.full((M, N), 7.0, device=dev).bfloat16()
    _gemm(P, W, bias, out, 0, a_src=a_src, lda=H, K=3 * H)
    rows = a_src.long()
    X = torch.cat([P[rows], P[rows + 1], P[rows + 2]], 1).float()
    ref = X @ W.float().t() + bias
    assert rel(out.float(), ref) < 6e-3


@pytest.mark.parametrize("M,N,K", [(1100, 640, 1024), (2048, 3072, 1024), (1300, 1024, 3072), (300, 256, 128)])
@pytest.mark.parametrize("tile", [0, 1, 2, 3])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_gemm_tiles(dev, M, N, K, tile, epi):
    """Explicit tile configurations (0: four waves of 64 x 64; 1: eight waves of 64 x 128; 2: eight waves of 64 x 64;
    3: 208-row tiles of eight waves of 112 x 64 and 96 x 64) with ragged rows and columns against fp32."""
    L = _lib.lib()
    g = torch.Generator(device=dev).manual_seed(M + N * 3 + K * 5 + epi)
    A = torch.randn(M, K, device=dev, generator=g).bfloat16()
    W = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).bfloat16()
    bias = torch.randn(N, device=dev, generator=g)
    gate = torch.randn(N, device=dev, generator=g)
    ref = A.float() @ W.float().t() + bias
    if epi in (0, 1):
        out = torch.full((M, N), 7.0, device=dev).bfloat16()
        if epi == 1:
            ref = torch.nn.functional.gelu(ref, approximate="tanh")
    elif epi == 2:
        out = torch.randn(M, N, device=dev, generator=g).half()
        ref = out.float() + gate * ref
    else:
        out = torch.zeros(M, N, device=dev)
    _lib.check(L.t2w_gemm_bf16_tile(A.data_ptr(), K, None, W.data_ptr(), bias.data_ptr(), gate.data_ptr() if epi == 2 else None,
                                    out.data_ptr(), N, M, N, K, epi, tile, _lib.stream_handle()), "gemm tile")
    torch.cuda.synchronize()
    assert rel(out.float(), ref) < {0: 6e-3, 1: 6e-3, 2: 1e-3, 3: 1e-5}[epi]


@pytest.mark.parametrize("M,N", [(12800, 1024), (2979, 2048), (416, 256)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3, 7])
def test_gemm_208_rows_equal_256(dev, M, N, epi):
    """The 208-row tile and the 256 x 256 tile sum every output in the same K order and apply the same epilogue: equal
    bits, dense and taps mode, every epilogue of the tile entry (7: fp16 out, the DiT's in_proj) (12,800 rows: the
    DiT's proj / conv / fc shapes at 16 streams x 400 frames)."""
    L = _lib.lib()
    g = torch.Generator(device=dev).manual_seed(M + N + epi)
    H = 1024
    P = torch.randn(M + 2, H, device=dev, generator=g).bfloat16()
    W = (torch.randn(N, 3 * H, device=dev, generator=g) / (3 * H) ** 0.5).bfloat16()
    bias = torch.randn(N, device=dev, generator=g)
    gate = torch.randn(N, device=dev, generator=g)
    a_src = torch.arange(M, dtype=torch.int32, device=dev)
    h0 = torch.randn(M, N, device=dev, generator=g).half()
    for taps in (False,) if epi == 7 else (False, True):  # the fp16 epilogue has no taps form
        outs = []
        for tile in (1, 3):
            if epi == 2:
                out = h0.clone()
            elif epi == 3:
                out = torch.zeros(M, N, device=dev)
            elif epi == 7:  # fp16 out
                out = torch.full((M, N), 7.0, device=dev).half()
            else:
                out = torch.full((M, N), 7.0, device=dev).bfloat16()
            _lib.check(L.t2w_gemm_bf16_tile(P.data_ptr(), H, a_src.data_ptr() if taps else None, W.data_ptr(), bias.data_ptr(),
                                            gate.data_ptr() if epi == 2 else None, out.data_ptr(), N, M, N, 3 * H if taps else H, epi,
                                            tile, _lib.stream_handle()), "gemm tile")
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), (taps, epi)


@pytest.mark.parametrize("M,N,K", [(1, 1024, 1024), (37, 3072, 1024), (100, 1024, 2048), (100, 80, 1024), (300, 2048, 1024), (600, 1024, 320)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_gemm_splitk(dev, M, N, K, epi):
    """Calls with few rows split K over many waves (partials in the caller's workspace, fixed-order reduction):
    parity with fp32 and bit-identical repeats."""
    g = torch.Generator(device=dev).manual_seed(M + N + K + 5 * epi)
    A = torch.randn(M, K, device=dev, generator=g).bfloat16()
    W = (torch.randn(N, K, device=dev, generator=g) / K ** 0.5).bfloat16()
    bias = torch.randn(N, device=dev, generator=g)
    gate = torch.randn(N, device=dev, generator=g)
    ws = torch.empty(16 << 20, dtype=torch.uint8, device=dev)
    ref = A.float() @ W.float().t() + bias
    if epi == 1:
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    outs = []
    for _ in range(2):
        if epi in (0, 1):
            out = torch.full((M, N), 7.0, device=dev).bfloat16()
        elif epi == 2:
            out = torch.randn(M, N, device=dev, generator=torch.Generator(device=dev).manual_seed(9)).half()
            h0 = out.float()
        else:
            out = torch.zeros(M, N, device=dev)
        _gemm(A, W, bias, out, epi, gate=gate if epi == 2 else None, ws=ws)
        outs.append(out)
    if epi in (0, 1):
        assert rel(outs[0].float(), ref) < 6e-3
    elif epi == 2:
        assert rel(outs[0].float(), h0 + gate * ref) < 1e-3
    else:
        assert rel(outs[0], ref) < 1e-5
    assert torch.equal(outs[0], outs[1])


def test_gemm_splitk_taps(dev):
    """Split-K in taps mode (a streaming chunk's conv GEMM) equals the tile kernel's result for the same call."""
    H, lens = 512, [50, 50]
    g = torch.Generator(device=dev).manual_seed(3)
    R, N = len(lens), sum(lens)
    P = torch.randn(N + 2 * R, H, device=dev, generator=g).bfloat16()
    Wfm = (torch.randn(H, 3 * H, device=dev, generator=g) / (3 * H) ** 0.5).bfloat16()
    bias = torch.randn(H, device=dev, generator=g)
    tok_row = [r for r, t in enumerate(lens) for _ in range(t)]
    a_src = torch.tensor([i + 2 * r for i, r in enumerate(tok_row)], dtype=torch.int32, device=dev)
    full = torch.cat([P[a_src.long() + j] for j in range(3)], 1).float()
    ref = full @ Wfm.float().t() + bias
    out = torch.zeros(N, H, device=dev)
    _gemm(P, Wfm, bias, out, 3, a_src=a_src, lda=H, K=3 * H, ws=torch.empty(16 << 20, dtype=torch.uint8, device=dev))
    assert rel(out, ref) < 1e-5


@pytest.mark.parametrize("lens,tile", [([5, 0, 1, 2, 3, 40, 0, 17, 1, 56], -1), ([400] * 3, -1), ([400] * 3, 1), ([400] * 3, 2),
                                       ([400] * 3, 3), ([5, 0, 300, 2, 3, 400, 0, 17, 1, 560], 0)])
def test_gemm_conv_taps(dev, lens, tile):
    """Taps mode: row m reads three consecutive frames starting at a_src[m] of the padded frame buffer; equals a
    kernel-3 conv over [2 cached frames | row frames] (F.conv1d, fp32).  tile: as chosen by shape (-1) or explicit."""
    H = 256
    g = torch.Generator(device=dev).manual_seed(11)
    R, N = len(lens), sum(lens)
    P = torch.randn(N + 2 * R, H, device=dev, generator=g).bfloat16()
    w = (torch.randn(H, H, 3, device=dev, generator=g) / (3 * H) ** 0.5)
    Wfm = w.permute(0, 2, 1).reshape(H, 3 * H).bfloat16().contiguous()
    bias = torch.randn(H, device=dev, generator=g)
    tok_row = [r for r, t in enumerate(lens) for _ in range(t)]
    a_src = torch.tensor([i + 2 * r for i, r in enumerate(tok_row)], dtype=torch.int32, device=dev)
    out = torch.zeros(N, H, device=dev)
    if tile < 0:
        _gemm(P, Wfm, bias, out, 3, a_src=a_src, lda=H, K=3 * H)
    else:
        _lib.check(_lib.lib().t2w_gemm_bf16_tile(P.data_ptr(), H, a_src.data_ptr(), Wfm.data_ptr(), bias.data_ptr(), None, out.data_ptr(), H,
                                                 N, H, 3 * H, 3, tile, _lib.stream_handle()), "gemm tile")
        torch.cuda.synchronize()
    refs, o = [], 0
    for r, t in enumerate(lens):
        if t:
            frames = P[o + 2 * r: o + 2 * r + 2 + t].float().t()[None]  # [1, H, 2 + t]
            refs.append(torch.nn.functional.conv1d(frames, w.bfloat16().float(), bias)[0].t())
        o += t
    assert rel(out, torch.cat(refs)) < 1e-5


def test_ln_mod(dev):
    L = _lib.lib()
    g = torch.Generator(device=dev).manual_seed(2)
    for H in (256, 512, 1024):
        N = 77
        h = (torch.randn(N, H, device=dev, generator=g) * 3 + 1).half()  # the fp16 residual stream
        sh, sc = torch.randn(H, device=dev, generator=g), 1 + torch.randn(H, device=dev, generator=g)
        out = torch.empty(N, H, dtype=torch.bfloat16, device=dev)
        _lib.check(L.t2w_ln_mod(h.data_ptr(), sh.data_ptr(), sc.data_ptr(), 1e-6, out.data_ptr(), N, H, _lib.stream_handle()))
        torch.cuda.synchronize()
        ref = torch.nn.functional.layer_norm(h.float(), (H,), eps=1e-6) * sc + sh
        assert rel(out.float(), ref) < 4e-3


def test_qk_norm_scatter(dev):
    L = _lib.lib()
    g = torch.Generator(device=dev).manual_seed(5)
    for heads in (4, 16):
        H, N = heads * 64, 333
        qkv = (torch.randn(N, 3 * H, device=dev, generator=g) * 3 + torch.randn(3 * H, device=dev, generator=g)).bfloat16()
        qw, qb, kw, kb = (torch.randn(64, device=dev, generator=g) for _ in range(4))
        slots = torch.randperm(2048, device=dev, generator=g)[:N].int()
        q = torch.zeros(N, H, dtype=torch.bfloat16, device=dev)
        kp = torch.zeros(2048, H, dtype=torch.bfloat16, device=dev)
        vp = torch.zeros_like(kp)
        _lib.check(L.t2w_qk_norm_scatter(qkv.data_ptr(), qw.data_ptr(), qb.data_ptr(), kw.data_ptr(), kb.data_ptr(), 1e-6, q.data_ptr(),
                                         kp.data_ptr(), vp.data_ptr(), slots.data_ptr(), N, heads, _lib.stream_handle()))
        torch.cuda.synchronize()
        x = qkv.float().view(N, 3, heads, 64)
        ln = lambda t, w, b: torch.nn.functional.layer_norm(t, (64,), w, b, 1e-6)  # noqa: E731
        assert rel(q.float().view(N, heads, 64), ln(x[:, 0], qw, qb)) < 4e-3
        assert rel(kp[slots.long()].float().view(N, heads, 64), ln(x[:, 1], kw, kb)) < 4e-3
        assert torch.equal(vp[slots.long()], qkv.view(N, 3, H)[:, 2])


def _attention_case(dev, lens, cached, heads, chunk, seed, kv_max=0):
    L = _lib.lib()
    g = torch.Generator(device=dev).manual_seed(seed)
    n_slots = 2 * (sum(lens) + sum(cached)) + 64
    H = heads * 64
    N = sum(lens)
    q = torch.randn(N, H, device=dev, generator=g).bfloat16()
    kp = torch.randn(n_slots, H, device=dev, generator=g).bfloat16()
    vp = torch.randn(n_slots, H, device=dev, generator=g).bfloat16()
    perm = torch.randperm(n_slots, generator=torch.Generator().manual_seed(seed)).tolist()
    kv, row_start, row_kv_off, row_kv_len, tiles, o = [], [], [], [], [], 0
    lists = []
    for r, (t, c) in enumerate(zip(lens, cached)):
        lst = [perm.pop() for _ in range(t + c)]
        lists.append(lst)
        row_start.append(o)
        row_kv_off.append(len(kv))
        row_kv_len.append(t + c)
        kv += lst
        tiles += [v for q0 in range(0, t, 64) for v in (r, q0)]
        o += t
    it = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)  # noqa: E731
    out = torch.zeros(N, H, dtype=torch.bfloat16, device=dev)
    keep = [it(x) for x in (kv, row_start, lens, row_kv_off, row_kv_len, tiles)]  # alive until the kernel ran
    _lib.check(L.t2w_attention(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), out.data_ptr(), *[t.data_ptr() for t in keep], len(tiles) // 2,
                               heads, chunk, 0.125, len(lens), kv_max, _lib.stream_handle()))
    torch.cuda.synchronize()
    if kv_max:  # the row-resident kernel does each query's arithmetic in the tile kernel's order: the same bits
        tile_out = torch.zeros_like(out)
        _lib.check(L.t2w_attention(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), tile_out.data_ptr(), *[t.data_ptr() for t in keep],
                                   len(tiles) // 2, heads, chunk, 0.125, len(lens), 0, _lib.stream_handle()))
        torch.cuda.synchronize()
        assert torch.equal(out, tile_out)
    worst = 0.0
    for r, (t, c) in enumerate(zip(lens, cached)):
        if t == 0:
            continue
        idx = torch.tensor(lists[r], device=dev)
        qq = q[row_start[r]:row_start[r] + t].float().view(t, heads, 64).transpose(0, 1)
        kk = kp[idx].float().view(t + c, heads, 64).transpose(0, 1)
        vv = vp[idx].float().view(t + c, heads, 64).transpose(0, 1)
        s = qq @ kk.transpose(1, 2) * 0.125
        vis = torch.ones(t, t + c, dtype=torch.bool, device=dev)
        if chunk > 0:
            cid = torch.arange(t, device=dev) // chunk
            vis[:, :t] = cid[None, :] <= cid[:, None]
        s = s.masked_fill(~vis[None], float("-inf"))
        ref = (torch.softmax(s, -1) @ vv).transpose(0, 1).reshape(t, H)
        e = rel(out[row_start[r]:row_start[r] + t].float(), ref)
        worst = max(worst, e)
        assert e < 1e-2, (r, t, c, e)
    return worst


@pytest.mark.parametrize("chunk", [0, 50])
@pytest.mark.parametrize("rep", [1, 9])
def test_attention_paged_block_causal(dev, chunk, rep):
    """Rows of new frames with cached keys in scattered slots; mask: cached keys always visible, new keys by chunk.
    rep 1: 32 workgroups (the key tiles of each split over four wave groups and merged); rep 9: 288 (one group)."""
    _attention_case(dev, [50, 1, 0, 130, 64, 65] * rep, [300, 0, 7, 0, 100, 33] * rep, 4, chunk, 9 + chunk)


@pytest.mark.parametrize("chunk", [0, 50])
def test_attention_stream_chunk(dev, chunk):
    """The streaming chunk's call (a CFG pair of 50 new frames over 300 and 462 cached keys, 16 heads) with the
    planner's key bound: the bound leaves small calls on the tile kernel (the same bits) and the result matches fp32."""
    _attention_case(dev, [50, 50], [300, 462], 16, chunk, 41 + chunk, kv_max=512)


@pytest.mark.parametrize("chunk", [0, 50])
def test_attention_long_rows(dev, chunk):
    """32 rows of up to 600 new frames and up to 500 cached keys, 16 heads (the grid of the 16-stream solve): rows of
    many query tiles, cached lists that do not start on a 64-key boundary, empty and one-token rows."""
    lens = [400, 150, 0, 450, 64, 1, 33, 600, 300, 257, 400, 95, 400, 400, 170, 222] * 2
    cached = [0, 300, 7, 0, 100, 33, 500, 0, 0, 31, 129, 0, 400, 0, 0, 64] * 2
    worst = _attention_case(dev, lens, cached, 16, chunk, 21 + chunk)
    print("long-row attention worst rel-L2", worst)


@pytest.mark.parametrize("chunk", [0, 50])
@pytest.mark.parametrize("kv_max", [256, 512])
def test_attention_row_resident(dev, chunk, kv_max):
    """Key lists held in LDS per (row, head): 32 rows of the 16-head grid with new runs of 0..kv_max keys and cached
    runs that start off the 64-key grid, equal to the tile kernel bit for bit and to fp32.  kv_max 256: two
    workgroups per CU."""
    if kv_max == 512:
        lens = [400, 150, 0, 450, 64, 1, 33, 512, 300, 257, 400, 95, 400, 200, 170, 222] * 2  # 4.1 query tiles per row
        cached = [0, 300, 7, 62, 100, 33, 479, 0, 0, 31, 112, 0, 112, 312, 0, 64] * 2
    else:
        lens = [200, 193, 0, 250, 64, 1, 33, 256, 193, 129, 200, 192, 200, 200, 170, 222] * 2  # 3.1 query tiles per row
        cached = [0, 63, 7, 6, 100, 33, 223, 0, 0, 31, 56, 0, 56, 0, 0, 34] * 2
    assert max(t + c for t, c in zip(lens, cached)) == kv_max
    worst = _attention_case(dev, lens, cached, 16, chunk, 31 + chunk, kv_max=kv_max)
    print("row-resident attention worst rel-L2", worst)


def test_attention_row_bound_broken(dev):
    """A row longer than the stated bound gets NaN outputs (no reads past the LDS lists); the rows within it are
    unaffected."""
    L = _lib.lib()
    heads, H, lens, cached = 16, 1024, [192] * 16, [0] * 15 + [400]
    N, n_slots = sum(lens), 3600
    g = torch.Generator(device=dev).manual_seed(3)
    q = torch.randn(N, H, device=dev, generator=g).bfloat16()
    kp = torch.randn(n_slots, H, device=dev, generator=g).bfloat16()
    vp = torch.randn(n_slots, H, device=dev, generator=g).bfloat16()
    kv, off, kvl = [], [], []
    for t, c in zip(lens, cached):
        off.append(len(kv))
        kvl.append(t + c)
        kv += list(range(len(kv), len(kv) + t + c))
    it = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)  # noqa: E731
    keep = [it(x) for x in (kv, [192 * r for r in range(16)], lens, off, kvl, [v for r in range(16) for v in (r, 0, r, 64, r, 128)])]
    outs = []
    for kv_max in (512, 0):
        out = torch.zeros(N, H, dtype=torch.bfloat16, device=dev)
        _lib.check(L.t2w_attention(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), out.data_ptr(), *[t.data_ptr() for t in keep], 48, heads, 0,
                                   0.125, 16, kv_max, _lib.stream_handle()))
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.isnan(outs[0][15 * 192:]).all() and not torch.isnan(outs[1]).any()
    assert torch.equal(outs[0][:15 * 192], outs[1][:15 * 192])


def test_quant_mx8_matches_oracle(dev):
    """The device MX quantizer equals the restatement bit for bit (codes and block scales), zero blocks and a wide
    dynamic range included."""
    L = _lib.lib()
    g = torch.Generator().manual_seed(4)
    M, K = 77, 1024
    x = (torch.randn(M, K, generator=g) * torch.exp(torch.randn(M, K // 32, generator=g) * 4).repeat_interleave(32, dim=1)).bfloat16()
    x[3, 64:96] = 0
    x[5, :32] = 448.0
    xd = x.to(dev)
    q = torch.empty(M, K, dtype=torch.uint8, device=dev)
    s = torch.empty(M, K // 32, dtype=torch.uint8, device=dev)
    _lib.check(L.t2w_quant_mx8(xd.data_ptr(), K, M, K, q.data_ptr(), K, s.data_ptr(), _lib.stream_handle()), "quant")
    torch.cuda.synchronize()
    qo, so = of.quantize_mx(x)
    assert torch.equal(s.cpu(), so)
    assert torch.equal(q.cpu(), qo)


def _fp8_operands(dev, M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(M, K, generator=g).bfloat16()
    W = torch.randn(N, K, generator=g) / K ** 0.5
    qa, sa = of.quantize_mx(A)
    qw, sw = of.quantize_weight(W)
    return (qa.to(dev), sa.to(dev), qw.to(dev), sw.to(dev), of.dequantize_mx(qa, sa), of.dequantize_weight(qw, sw), A, W,
            torch.randn(N, generator=g).to(dev), torch.randn(N, generator=g).to(dev))


@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (100, 1024, 1024), (333, 80, 1024), (1300, 1024, 2048), (2048, 3072, 1024)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_gemm_fp8(dev, M, N, K, epi):
    """fp8 MFMA GEMM against fp32 matmul of the dequantized operands (the quantization itself is the restatement's).
    The fp8 MFMA sums its 64 products at a precision measured at ~6e-5 of the largest output on random e4m3 data, hence
    1e-4 where bf16 GEMMs are held to 1e-5."""
    L = _lib.lib()
    qa, sa, qw, sw, Ad, Wd, A, W, bias, gate = _fp8_operands(dev, M, N, K, M + N + K + epi)
    ref = Ad.to(dev) @ Wd.to(dev).t() + bias
    if epi == 1:
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    if epi in (0, 1):
        out = torch.full((M, N), 7.0, device=dev).bfloat16()
    elif epi == 2:  # the fp16 residual stream
        out = torch.randn(M, N, device=dev).half()
        h0 = out.float()
    else:
        out = torch.zeros(M, N, device=dev)
    _lib.check(L.t2w_gemm_fp8(qa.data_ptr(), K, None, sa.data_ptr(), K // 32, qw.data_ptr(), sw.data_ptr(), bias.data_ptr(),
                              gate.data_ptr() if epi == 2 else None, out.data_ptr(), N, M, N, K, epi, _lib.stream_handle()), "gemm_fp8")
    torch.cuda.synchronize()
    if epi in (0, 1):
        assert rel(out.float(), ref) < 6e-3
    elif epi == 2:
        assert rel(out.float(), h0 + gate * ref) < 1e-3
    else:
        assert rel(out, ref) < 1e-4
        # and against the unquantized bf16 product: the fp8 rounding error itself
        exact = A.float().to(dev) @ W.to(dev).t() + bias
        assert rel(out, exact) < 6e-2


@pytest.mark.parametrize("N,epi", [(3072, 0), (1024, 2), (2048, 3)])
def test_gemm_fp8_large_tiles(dev, N, epi):
    """fp8 at the 12,800-token shapes, where the grid takes 256 x 256 tiles of 64 x 128-wave sub-tiles (and, for
    N = 3072, the rows of its last partial round on 256 x 128 tiles, whose activation scale rows start past the split):
    against fp32 matmul of the dequantized operands, as test_gemm_fp8."""
    L = _lib.lib()
    M, K = 12800, 1024
    qa, sa, qw, sw, Ad, Wd, A, W, bias, gate = _fp8_operands(dev, M, N, K, 77 + N + epi)
    ref = Ad.to(dev) @ Wd.to(dev).t() + bias
    if epi == 0:
        out = torch.full((M, N), 7.0, device=dev).bfloat16()
    elif epi == 2:
        out = torch.randn(M, N, device=dev).half()
        h0 = out.float()
    else:
        out = torch.zeros(M, N, device=dev)
    _lib.check(L.t2w_gemm_fp8(qa.data_ptr(), K, None, sa.data_ptr(), K // 32, qw.data_ptr(), sw.data_ptr(), bias.data_ptr(),
                              gate.data_ptr() if epi == 2 else None, out.data_ptr(), N, M, N, K, epi, _lib.stream_handle()), "gemm_fp8")
    torch.cuda.synchronize()
    if epi == 0:
        assert rel(out.float(), ref) < 6e-3
    elif epi == 2:
        assert rel(out.float(), h0 + gate * ref) < 1e-3
    else:
        assert rel(out, ref) < 1e-4
    if N == 3072:  # the rows of the last partial round (the 256 x 128 tail) on their own
        tail = slice(M - 1536, M)
        assert rel(out[tail].float(), ref[tail]) < 6e-3


def test_gemm_fp8_taps(dev):
    """fp8 taps mode: the block scales of a row come from its three frames."""
    L = _lib.lib()
    H, lens = 256, [50, 7, 300]
    R, N = len(lens), sum(lens)
    g = torch.Generator().manual_seed(9)
    frames = torch.randn(N + 2 * R, H, generator=g).bfloat16()  # padded frame buffer [frames, H]
    qa, sa = of.quantize_mx(frames)
    Ad = of.dequantize_mx(qa, sa)
    qw, sw = of.quantize_weight(torch.randn(H, 3 * H, generator=g) / (3 * H) ** 0.5)
    Wd = of.dequantize_weight(qw, sw)
    qa, sa, qw, sw = qa.to(dev), sa.to(dev), qw.to(dev), sw.to(dev)
    bias = torch.randn(H, generator=g).to(dev)
    tok_row = [r for r, t in enumerate(lens) for _ in range(t)]
    a_src = torch.tensor([i + 2 * r for i, r in enumerate(tok_row)], dtype=torch.int32, device=dev)
    full = torch.cat([Ad.to(dev)[a_src.long() + j] for j in range(3)], 1)
    ref = full @ Wd.to(dev).t() + bias
    out = torch.zeros(N, H, device=dev)
    _lib.check(L.t2w_gemm_fp8(qa.data_ptr(), H, a_src.data_ptr(), sa.data_ptr(), H // 32, qw.data_ptr(), sw.data_ptr(), bias.data_ptr(),
                              None, out.data_ptr(), H, N, H, 3 * H, 3, _lib.stream_handle()), "gemm_fp8 taps")
    torch.cuda.synchronize()
    assert rel(out, ref) < 1e-4


@pytest.mark.parametrize("kv_max,rows", [(512, 16), (0, 16), (0, 2)])
def test_attention_list_shorter_than_row(dev, kv_max, rows):
    """A table whose row states fewer keys than the row's own new frames gets NaN outputs for that row from every
    attention form (row-resident, tile, and the small-grid tile kernel that splits key tiles over four wave groups);
    the other rows equal a well-formed call's.  The key table holds every row's full list, so no read could leave it
    even without the check."""
    L = _lib.lib()
    heads, H = 16, 1024
    T = 192 if rows == 16 else 50
    lens = [T] * rows
    N = sum(lens)
    g = torch.Generator(device=dev).manual_seed(4)
    q = torch.randn(N, H, device=dev, generator=g).bfloat16()
    kp = torch.randn(N + 64, H, device=dev, generator=g).bfloat16()
    vp = torch.randn(N + 64, H, device=dev, generator=g).bfloat16()
    kv = list(range(N))
    off = [T * r for r in range(rows)]
    tiles = [v for r in range(rows) for q0 in range(0, T, 64) for v in (r, q0)]
    it = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)  # noqa: E731
    outs = []
    for short in (False, True):
        kvl = [T] * rows
        if short:
            kvl[rows - 1] = T // 2
        keep = [it(x) for x in (kv, off, lens, off, kvl, tiles)]
        out = torch.zeros(N, H, dtype=torch.bfloat16, device=dev)
        _lib.check(L.t2w_attention(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), out.data_ptr(), *[t.data_ptr() for t in keep], len(tiles) // 2,
                                   heads, 0, 0.125, rows, kv_max, _lib.stream_handle()))
        torch.cuda.synchronize()
        outs.append(out)
    last = (rows - 1) * T
    assert not torch.isnan(outs[0]).any()
    assert torch.isnan(outs[1][last:]).all()
    assert torch.equal(outs[1][:last], outs[0][:last])
