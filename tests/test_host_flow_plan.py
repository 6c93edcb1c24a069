"""Host logic of the flow encoder (CPU, no kernel runs): the per-call index tables stay inside the buffers the kernels
index, the key lists follow the reference's packed-cache rule (first stack: first half of ``trim(list + list)``; second
stack: ``trim(list)``), and slot reference counts return to zero.

The C call is replaced by a checker that reads the tables the host uploaded (CPU tensors, so their addresses are host
memory) and asserts every index each kernel and GEMM would form is in bounds.
"""

import ctypes

import numpy as np
import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd import _lib
from t2w_amd import flow as fl
from t2w_amd.config import FlowConfig

CFG = FlowConfig()


class _FakeModel:
    def __init__(self):
        self.cfg, self.device, self.handle = CFG, torch.device("cpu"), None


def _arr(ptr, n):
    return np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_int32)), shape=(max(n, 1),))[:n].copy()


class _Checker:
    """Stands in for the library: workspace size 0, and t2w_flow_encode checks the call's tables."""

    def __init__(self, enc):
        self.enc, self.calls = enc, []

    def t2w_flow_workspace_bytes(self, *a):
        return 0

    def t2w_flow_encode(self, handle, aref, stream):
        a = aref._obj
        R, n_in, n_gap, n1, n_up, n2 = a.n_rows, a.n_in, a.n_gap, a.n1, a.n_up, a.n2
        look, s = CFG.look, CFG.stride
        assert n_in == n1 + look * R and n_gap == n1 + 2 * R and n2 == s * n1 and n_up == n2 + 2 * s * R
        t = {k: _arr(getattr(a, k), n) for k, n in (("tok", n_in), ("res", n_in), ("c1_src", n_gap), ("gofs", R), ("t1", R),
                                                  ("c2_src", n1), ("up_dst", n1), ("uofs", R), ("o1", R), ("up_src", n2), ("o2", R),
                                                  ("t2", R), ("cnn_rd", R), ("cnn_wr", R), ("new1", n1), ("new2", n2),
                                                  ("kv1_off", R), ("kv1_len", R), ("kv2_off", R), ("kv2_len", R),
                                                  ("tiles1", 2 * a.n_tiles1), ("tiles2", 2 * a.n_tiles2))}
        kv1 = _arr(a.kv1_idx, int((t["kv1_off"] + t["kv1_len"]).max()))
        kv2 = _arr(a.kv2_idx, int((t["kv2_off"] + t["kv2_len"]).max()))
        assert ((t["tok"] >= -1) & (t["tok"] < CFG.vocab)).all()
        assert ((t["res"] >= -1) & (t["res"] < n1)).all() and np.array_equal(np.sort(t["res"][t["res"] >= 0]), np.arange(n1))
        assert (t["c1_src"] >= 0).all() and (t["c1_src"] + look < n_in).all()           # conv1 taps rows
        assert (t["c2_src"] >= 0).all() and (t["c2_src"] + 2 < n_gap).all()             # conv2 taps rows
        assert (t["up_dst"] >= 0).all() and (t["up_dst"] + 1 < n_up).all()
        assert (t["up_src"] >= 0).all() and (t["up_src"] + 2 * s < n_up).all()          # upsampling taps rows
        assert (t["gofs"] + t["t1"] + 2 <= n_gap).all() and (t["uofs"] + 2 * s + s * t["t1"] <= n_up).all()
        assert (t["o1"] + t["t1"] <= n1).all() and (t["o2"] + t["t2"] <= n2).all()
        # conv caches: written slots are fresh and never read in this call
        assert len(set(t["cnn_wr"])) == R and not set(t["cnn_wr"]) & set(t["cnn_rd"])
        n_c = self.enc.cnn_pool.shape[0]
        assert ((t["cnn_rd"] >= 0) & (t["cnn_rd"] < n_c)).all() and ((t["cnn_wr"] > 0) & (t["cnn_wr"] < n_c)).all()
        for kv, new, nslots, key in ((kv1, t["new1"], self.enc.pool1.shape[1], "1"), (kv2, t["new2"], self.enc.pool2.shape[1], "2")):
            assert ((kv >= 0) & (kv < nslots)).all() and ((new >= 0) & (new < nslots)).all()
            assert len(set(new)) == new.size
            L, T = t["kv" + key + "_len"], t["t" + key]
            assert (L >= T).all() and (L <= CFG.rmax).all()
            tiles = t["tiles" + key].reshape(-1, 2)
            assert ((tiles[:, 0] >= 0) & (tiles[:, 0] < R)).all() and (tiles[:, 1] < T[tiles[:, 0]]).all()
            for r in range(R):  # each stream's list ends with its own new rows' slots, and every query has a tile
                o, rs = t["kv" + key + "_off"][r], t["o" + key][r]
                assert np.array_equal(kv[o + L[r] - T[r]:o + L[r]], new[rs:rs + T[r]])
                assert sorted(tiles[tiles[:, 0] == r, 1].tolist()) == list(range(0, int(T[r]), 32))
        self.calls.append(t)
        return 0


@pytest.fixture()
def enc(monkeypatch):
    e = fl.FlowEncoder(_FakeModel(), n_slots1=4096, n_slots2=8192, n_cnn=32)
    chk = _Checker(e)
    monkeypatch.setattr(_lib, "lib", lambda: chk)
    monkeypatch.setattr(_lib, "stream_handle", lambda stream=None: 0)
    return e


def _sim_lists(k1, k2, T1, keep, last):
    """The reference's packed cache on frame ids."""
    n1 = list(range(1000000 + len(k1), 1000000 + len(k1) + T1))
    c1, c2 = k1 + n1, k2 + ["x"] * (2 * T1)
    if last:
        return [], []
    p1 = c1 + c1
    if len(p1) > keep + 100:
        p1 = p1[:keep] + p1[-100:]
        c2 = c2[:keep] + c2[-100:]
    return p1[: len(p1) // 2], c2


def test_plan_bounds_lists_and_refcounts(enc):
    rng = np.random.default_rng(0)
    states, mu, rows, frames = enc.setup([rng.integers(0, CFG.vocab, n).tolist() for n in (30, 57, 8, 120)])
    assert frames == [60, 114, 16, 240] and [st.keep for st in states] == frames
    assert [st.k1.size for st in states] == [30, 57, 8, 120] and [st.k2.size for st in states] == frames
    streams = [enc.clone(s) for s in states]
    for s in states:
        enc.release(s)
    live = list(range(4))
    for call in range(12):
        wins, lasts = [], []
        for i in live:
            last = call == 11 or (i == 2 and call == 5)
            n = int(rng.integers(4, 30)) if last else (11 if call == 0 else 28)
            wins.append(rng.integers(0, CFG.vocab, n).tolist())
            lasts.append(last)
        before = [(enc_state.k1.size, enc_state.k2.size) for enc_state in (streams[i] for i in live)]
        mu, rows, frames = enc.encode([streams[i] for i in live], wins, lasts)
        assert frames == [2 * (len(w) - (0 if l else CFG.look)) for w, l in zip(wins, lasts)]
        for k, i in enumerate(live):
            T1 = len(wins[k]) - (0 if lasts[k] else CFG.look)
            e1, e2 = _sim_lists(list(range(before[k][0])), list(range(before[k][1])), T1, streams[i].keep, lasts[k])
            assert streams[i].k1.size == len(e1) and streams[i].k2.size == len(e2)
            assert 2 * streams[i].k1.size == streams[i].k2.size or lasts[k]
        live = [i for i, l in zip(live, lasts) if not l]
        if not live:
            break
    assert not live
    assert enc.in_use() == (0, 0, 0)


def test_list_contents_follow_the_trim(enc):
    """Slot ids in the lists: the second stack keeps the prompt's frames and the newest 100; the first stack (prompt of
    60 tokens, keep 120 >= 100) freezes at the prompt and the first windows."""
    rng = np.random.default_rng(1)
    [st], _, _, _ = enc.setup([rng.integers(0, CFG.vocab, 60).tolist()])
    prompt1, prompt2 = st.k1.copy(), st.k2.copy()
    news1, news2 = [], []
    for call in range(6):
        enc.encode([st], [rng.integers(0, CFG.vocab, 28).tolist()], [False])
        news1.append(enc_new(enc, 1))
        news2.append(enc_new(enc, 2))
    all1 = np.concatenate([prompt1] + news1)
    all2 = np.concatenate([prompt2] + news2)
    assert np.array_equal(st.k1, all1[:(120 + 100) // 2])
    assert np.array_equal(st.k2, np.concatenate([all2[:120], all2[-100:]]))
    enc.release(st)
    assert enc.in_use() == (0, 0, 0)


def enc_new(enc, stack):
    return lib_calls(enc)[-1]["new" + str(stack)]


def lib_calls(enc):
    return _lib.lib().calls
