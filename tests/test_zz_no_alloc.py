"""The no-allocation solve (``t2w_dit_solve_noalloc``: the workspace is the library's static device scratch) against
``t2w_dit_solve`` with a caller workspace, through the C ABI, at full model size: two calls in a row on the same tables
and inputs, the second smaller (a 500-token call on the tile / split-K GEMMs, then an 80-token streaming call on the
small-row GEMMs whose K-split sums the next row kernel finishes).  Same kernels, same plan: outputs equal bit for bit.
A call needing more than the scratch holds is refused with a message and launches nothing."""

import ctypes as C

import numpy as np
import pytest
import torch

import t2w_amd  # noqa: F401
from t2w_amd import _lib
from t2w_amd.config import DiTConfig
from t2w_amd.dit import DiTModel, FastDiT, _Upload, plan_call
from t2w_amd.weights import init_dit

pytestmark = pytest.mark.gpu


def _args(fd, Ts, seed, workspace: bool):
    g = torch.Generator().manual_seed(seed)
    n = len(Ts)
    mus = [torch.randn(80, t, generator=g).cuda() for t in Ts]
    spks = torch.randn(n, 80, generator=g).cuda()
    caches = [fd.new_cache() for _ in Ts]
    x0, stat = fd._inputs(caches, mus, spks, None, Ts)
    rows = [c.rows[0] for c in caches] + [c.rows[1] for c in caches]
    new = [fd.pool.alloc(t) for t in Ts + Ts]
    p = plan_call(rows, Ts, new, [False] * n, fd.cnn_scratch, fd.cnn_zero)
    tables = _Upload.new(fd._flat(p), fd.device)
    out = torch.full((p["half"], 80), float("nan"), device="cuda")
    ws = fd._workspace(p["n_tok"], p["n_rows"]) if workspace else None
    if ws is None:
        ws = torch.empty(0, dtype=torch.uint8, device="cuda")
    a = fd._args(p, tables, x0, stat, out, ws, chunk=0)
    if not workspace:
        a.workspace, a.workspace_bytes = None, 0
    keep = (tables, x0, stat, ws, caches, new)
    return a, out, keep


def _release(fd, keep):
    tables, x0, stat, ws, caches, new = keep
    for ids in new:
        fd.pool.release(ids)
    for c in caches:
        fd.release(c)


def test_noalloc_solve_equals_workspace_solve(dev):
    W = init_dit(DiTConfig(), seed=9)
    model = DiTModel(W, DiTConfig())
    fd = FastDiT(model, n_slots=8192, max_streams=4)
    L, st = _lib.lib(), _lib.stream_handle()
    for k, Ts in enumerate(([150, 100], [40])):
        a, out_ws, keep_a = _args(fd, Ts, seed=10 + k, workspace=True)
        b, out_na, keep_b = _args(fd, Ts, seed=10 + k, workspace=False)
        print(f"call {k}: {2 * sum(Ts)} tokens", flush=True)
        _lib.check(L.t2w_dit_solve(model.handle, C.byref(a), st), "dit_solve")
        _lib.check(L.t2w_dit_solve_noalloc(model.handle, C.byref(b), st), "dit_solve_noalloc")
        torch.cuda.synchronize()
        assert torch.isfinite(out_ws).all()
        assert torch.equal(out_ws, out_na), float((out_ws - out_na).abs().max())
        _release(fd, keep_a)
        _release(fd, keep_b)
    # beyond the scratch: refused before any launch
    big, out_big, keep_big = _args(fd, [1000, 1000], seed=20, workspace=False)
    rc = L.t2w_dit_solve_noalloc(model.handle, C.byref(big), st)
    msg = L.t2w_last_error().decode()
    print("refused:", msg)
    assert rc != 0 and "static scratch" in msg
    torch.cuda.synchronize()
    assert torch.isnan(out_big).all()
    _release(fd, keep_big)
    assert fd.pool.in_use() == fd.scratch and np.isfinite(float(out_na.sum()))
