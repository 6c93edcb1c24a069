"""Host logic of the solve (CPU): call planning tables and the per-row cache bookkeeping against the oracle's trim."""

import numpy as np
import pytest

import t2w_amd  # noqa: F401
from t2w_amd.dit import FastRow, SlotPool, advance_row, all_buckets, bucket_of, bucket_tiles, plan_call, token_buckets
from oracle import dit as od


def _rows(specs):
    return [FastRow(slots=np.asarray(s, dtype=np.int32), conv=c, cur=cur) for s, c, cur in specs]


def _L(x):
    return np.asarray(x).tolist()


def test_plan_tables_are_consistent():
    rows = _rows([([100, 101, 102], (0, 1), 0), ([], (2, 3), 1), ([200, 201, 202], (4, 5), 0), ([], (6, 7), 1)])
    for r, pos in zip(rows, (250, 9, 250, 9)):  # stream positions of the rows' next frames (rotary embedding)
        r.pos = pos
    Ts = [70, 1]
    new = [np.arange(10, 80), np.array([90]), np.arange(300, 370), np.array([390])]
    p = plan_call(rows, Ts, new, [True, False], cnn_scratch=99)
    tok_row, tok_pos, a_src, new_slot, row_start, lens, kv_off, kv_len, rd, wr, tiles, tok_abs, kv = map(_L, p["parts"])
    assert p["n_tok"] == 142 and p["half"] == 71 and p["n_rows"] == 4
    assert tok_abs == [rows[r].pos + t for r, t in zip(tok_row, tok_pos)]
    assert a_src == [i + 2 * r for i, r in enumerate(tok_row)]
    assert tok_pos == [t for T in lens for t in range(T)]
    assert lens == [70, 1, 70, 1] and row_start == [0, 70, 71, 141]
    for r in range(4):
        lst = kv[kv_off[r]:kv_off[r] + kv_len[r]]
        assert lst[:lens[r]] == _L(new[r]) and lst[lens[r]:] == rows[r].order
    assert rd == [0, 3, 4, 7] and wr == [1, 99, 5, 99]
    covered = sorted((r, q) for r, q0 in zip(tiles[::2], tiles[1::2]) for q in range(q0, min(q0 + 64, lens[r])))
    assert covered == sorted((r, q) for r in range(4) for q in range(lens[r]))
    assert set(rd).isdisjoint(set(wr))


def test_bucket_table():
    """Row buckets of 2..64 request rows, token buckets (both halves) in steps of 128 below 512 and 256 above, up to 56
    frames per row (at least 4096 tokens for up to 8 rows); calls beyond the largest bucket have none."""
    assert token_buckets(2)[:6] == [128, 256, 384, 512, 768, 1024] and token_buckets(2)[-1] == 4096
    assert token_buckets(16)[-2:] == [768, 896] and token_buckets(64)[-1] == 3584
    assert bucket_of(4, 220) == (4, 256) and bucket_of(4, 256) == (4, 256) and bucket_of(3, 257) == (4, 384)
    assert bucket_of(2, 5000) is None and bucket_of(6, 4000) == (8, 4096) and bucket_of(10, 4000) is None
    assert bucket_of(10, 900) == (32, 1024) and bucket_of(64, 3584) == (64, 3584) and bucket_of(66, 10) is None
    assert len(all_buckets()) == sum(len(token_buckets(rb)) for rb in (2, 4, 8, 16, 32, 64))


@pytest.mark.parametrize("Ts,keep", [([70, 1], [True, False]), ([64, 128, 5], [True, True, False]), ([50], [True])])
def test_padded_plan_keeps_every_real_row(Ts, keep):
    n = len(Ts)
    rows = _rows([(range(1000 * r, 1000 * r + 7 * r), (2 * r, 2 * r + 1), r % 2) for r in range(2 * n)])
    for r, row in enumerate(rows):
        row.pos = 13 * (r % n)
    new = [np.arange(100000 + 1000 * r, 100000 + 1000 * r + Ts[r % n]) for r in range(2 * n)]
    P = [_L(x) for x in plan_call(rows, Ts, new, keep, cnn_scratch=99)["parts"]]
    rb, nb = bucket_of(2 * n, 2 * sum(Ts))
    q = plan_call(rows, Ts, new, keep, cnn_scratch=99, cnn_zero=98, bucket=(rb, nb), kv_scratch=77)
    hr = rb // 2 + 1
    tok_row, tok_pos, a_src, new_slot, row_start, lens, kv_off, kv_len, rd, wr, tiles, tok_abs, kv = map(_L, q["parts"])
    assert q["n_rows"] == 2 * hr and q["n_tok"] == nb and q["half"] == nb // 2 and len(tok_row) == nb
    assert q["real_half"] == sum(Ts)
    assert sum(lens[:hr]) == sum(lens[hr:]) == nb // 2
    assert a_src == [i + 2 * r for i, r in enumerate(tok_row)]
    for h in range(2):
        for j in range(hr):
            r = h * hr + j
            s, T = row_start[r], lens[r]
            assert tok_row[s:s + T] == [r] * T and tok_pos[s:s + T] == list(range(T))
            if j < n:  # a request row: the same tables as unpadded
                o = h * n + j
                assert T == P[5][o] and new_slot[s:s + T] == P[3][P[4][o]:P[4][o] + T]
                assert kv[kv_off[r]:kv_off[r] + kv_len[r]] == P[12][P[6][o]:P[6][o] + P[7][o]]
                assert (rd[r], wr[r]) == (P[8][o], P[9][o])
                assert tok_abs[s:s + T] == P[11][P[4][o]:P[4][o] + T] == [rows[o].pos + t for t in range(T)]
            else:  # empty rows, then the padding row: scratch key slot, zero conv cache in, scratch conv cache out
                assert T == (0 if j < hr - 1 else nb // 2 - sum(Ts))
                assert new_slot[s:s + T] == [77] * T and kv[kv_off[r]:kv_off[r] + kv_len[r]] == [77] * T
                assert tok_abs[s:s + T] == list(range(T))
                assert rd[r] == 98 and wr[r] == 99
    assert q["n_tiles"] == len(tiles) // 2 == bucket_tiles(rb, nb)
    live = [(r, q0) for r, q0 in zip(tiles[::2], tiles[1::2]) if q0 < lens[r]]
    covered = sorted((r, t) for r, q0 in live for t in range(q0, min(q0 + 64, lens[r])))
    assert covered == sorted((r, t) for r in range(2 * hr) for t in range(lens[r]))
    # no row reads a conv slot that any row of the call writes
    assert set(rd).isdisjoint(set(wr))


def test_every_bucket_plans_within_its_tile_bound():
    for rb, nb in all_buckets():
        q = plan_call([], [], [], [], cnn_scratch=1, cnn_zero=0, bucket=(rb, nb), kv_scratch=5)
        assert q["n_tok"] == nb and q["n_tiles"] == bucket_tiles(rb, nb)


@pytest.mark.parametrize("keep_len", [0, 40, 300])
def test_row_bookkeeping_follows_the_oracle_trim(keep_len):
    pool = SlotPool(10000, reserved=1)
    row = FastRow(slots=pool.alloc(keep_len), conv=(0, 1))
    ref = row.order
    for w in range(7):
        nw = pool.alloc(50)
        freed = advance_row(row, nw, keep=w != 3, keep_len=keep_len)
        pool.release(freed)
        if w != 3:
            ref = od.trim_order(_L(nw) + ref, keep_len)
        assert row.order == ref
        assert pool.in_use() - 1 == len(row.order)
    assert row.cur == 0  # six kept windows swapped the conv slots six times
    assert row.pos == 6 * 50  # stream position: frames of the kept windows, trimmed ones included


def test_slot_pool_reserved_and_exhaustion():
    pool = SlotPool(8, reserved=1)
    assert pool.in_use() == 1 and pool.n_free == 7
    a = pool.alloc(5)
    assert len(set(_L(a)) | set(_L(pool.reserved))) == 6
    with pytest.raises(RuntimeError, match="exhausted"):
        pool.alloc(3)
    pool.release(a)
    assert pool.in_use() == 1
    b = pool.alloc(7)
    assert sorted(_L(b) + _L(pool.reserved)) == list(range(8))


def test_kv_max_classes():
    """The key-list bound a call states: 256 or 512 when every row's list fits (the row-resident attention's two LDS
    sizes), 0 beyond 512; it is part of the graph keys, so a replay never exceeds its capture's bound."""
    import numpy as np
    from t2w_amd.dit import ATTN_ROW_KMAX, _kv_max
    part = lambda lens: {"parts": [None] * 7 + [np.array(lens, dtype=np.int64)]}  # noqa: E731
    assert ATTN_ROW_KMAX == 512
    assert _kv_max(part([1, 256])) == 256 and _kv_max(part([257, 3])) == 512 and _kv_max(part([512])) == 512
    assert _kv_max(part([513, 10])) == 0 and _kv_max(part([])) == 256


def test_bucket_graphs_never_take_the_row_resident_attention():
    """The row-resident attention launches only for calls of at least 256 (row, head) pairs whose rows average three
    or more 64-query tiles (``attention`` in csrc/attn.hip).  With the model's 16 heads no bucket's padded plan meets
    both, so bucket plans state no key-list bound (0: the tile kernel, which every bucket call took anyway)."""
    from t2w_amd.config import DiTConfig
    from t2w_amd.dit import _kv_max

    heads = DiTConfig().heads
    for rb, nb in all_buckets():
        p = plan_call([], [], [], [], cnn_scratch=99, cnn_zero=98, bucket=(rb, nb), kv_scratch=97)
        assert p["n_rows"] * heads < 256 or p["n_tiles"] < 3 * p["n_rows"], (rb, nb)
        assert _kv_max(p) == 0


def test_steady_window_key_is_the_captured_bucket_key():
    """A steady streaming call (50 new frames per stream on 300-450 cached frames) pads to a bucket whose graph key is
    the one ``capture`` / ``capture_all`` create from padding-only plans, whatever the rows' cached lengths."""
    from t2w_amd.dit import _kv_max, bucket_graph_key

    rng = np.random.default_rng(0)
    captured = {bucket_graph_key(b, 0, 0) for b in all_buckets()}
    for n in (1, 3, 8, 16, 32):
        cached = rng.integers(300, 451, n)
        rows = _rows([(np.arange(10000 * r, 10000 * r + int(cached[r % n])), (2 * r, 2 * r + 1), 0) for r in range(2 * n)])
        Ts = [50] * n
        new = [np.arange(500000 + 100 * r, 500000 + 100 * r + 50) for r in range(2 * n)]
        bucket = bucket_of(2 * n, 2 * sum(Ts))
        p = plan_call(rows, Ts, new, [True] * n, cnn_scratch=99, cnn_zero=98, bucket=bucket, kv_scratch=97)
        assert int(p["parts"][7].max()) > 256  # the lists are long: a length-derived bound would have been 512
        assert _kv_max(p) == 0
        assert bucket_graph_key(bucket, 0, 0) in captured
        empty = plan_call([], [], [], [], cnn_scratch=99, cnn_zero=98, bucket=bucket, kv_scratch=97)
        assert _kv_max(empty) == _kv_max(p)


def test_cu_mask_spread():
    """The co-scheduling mask gives 32-CU groups equal shares as runs from each group's first CU, at least 8 CUs in
    every group it uses (the runtime refuses masks that interleave single CUs or give a group fewer)."""
    from t2w_amd.cosched import spread_mask

    ones = lambda m: [bin(x).count("1") for x in m]  # noqa: E731
    assert spread_mask(64, total=256) == [0xFF] * 8
    assert spread_mask(256, total=256) == [0xFFFFFFFF] * 8
    assert spread_mask(128, total=256) == [0xFFFF] * 8
    assert spread_mask(32, total=256) == [0xFF] * 4 + [0] * 4
    assert spread_mask(8, total=256) == [0xFF] + [0] * 7
    m = spread_mask(100, total=256)
    assert ones(m) == [13] * 4 + [12] * 4 and all(x & (x + 1) == 0 for x in m)
    assert ones(spread_mask(20, total=256)) == [10, 10] + [0] * 6
    m = spread_mask(70, total=72)  # a short last group
    assert sum(ones(m)) == 70 and all(k == 0 or k >= 8 for k in ones(m))
    for n in range(8, 257):
        m = spread_mask(n, total=256)
        assert sum(ones(m)) == n and all(k == 0 or k >= 8 for k in ones(m)) and all(x & (x + 1) == 0 for x in m)
    with pytest.raises(ValueError):
        spread_mask(4, total=256)
    with pytest.raises(ValueError):
        spread_mask(300, total=256)
