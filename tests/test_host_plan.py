"""Host logic of the solve (CPU): call planning tables and the per-row cache bookkeeping against the oracle's trim."""

import pytest

import t2w_amd  # noqa: F401
from t2w_amd.dit import FastRow, SlotPool, advance_row, plan_call
from oracle import dit as od


def test_plan_tables_are_consistent():
    rows = [FastRow(order=[100, 101, 102], cnn=(0, 1)), FastRow(order=[], cnn=(2, 3), cur=1),
            FastRow(order=[200, 201, 202], cnn=(4, 5)), FastRow(order=[], cnn=(6, 7), cur=1)]
    Ts = [70, 1]
    new = [list(range(10, 80)), [90], list(range(300, 370)), [390]]
    p = plan_call(rows, Ts, new, [True, False], cnn_scratch=99)
    tok_row, tok_pos, a_src, new_slot, row_start, lens, kv_off, kv_len, rd, wr, tiles, kv = p["parts"]
    assert p["n_tok"] == 142 and p["half"] == 71 and p["n_rows"] == 4
    assert a_src == [i + 2 * r for i, r in enumerate(tok_row)]
    assert lens == [70, 1, 70, 1] and row_start == [0, 70, 71, 141]
    for r in range(4):
        lst = kv[kv_off[r]:kv_off[r] + kv_len[r]]
        assert lst[:lens[r]] == new[r] and lst[lens[r]:] == rows[r].order
    assert rd == [0, 3, 4, 7] and wr == [1, 99, 5, 99]
    covered = sorted((r, q) for r, q0 in zip(tiles[::2], tiles[1::2]) for q in range(q0, min(q0 + 64, lens[r])))
    assert covered == sorted((r, q) for r in range(4) for q in range(lens[r]))
    assert set(rd).isdisjoint(set(wr))


@pytest.mark.parametrize("keep_len", [0, 40, 300])
def test_row_bookkeeping_follows_the_oracle_trim(keep_len):
    pool = SlotPool(10000)
    row = FastRow(order=pool.alloc(keep_len), cnn=(0, 1))
    ref = list(row.order)
    for w in range(7):
        nw = pool.alloc(50)
        freed = advance_row(row, nw, keep=w != 3, keep_len=keep_len)
        pool.release(freed)
        if w != 3:
            ref = od.trim_order(nw + ref, keep_len)
        assert row.order == ref
        assert pool.in_use() == len(row.order)
    assert row.cur == 0  # six kept windows swapped the conv slots six times
