"""Flow encoder on the GPU (C-ABI ``t2w_flow_encode``) against the fp32 CPU oracle at the real width (512, 8 heads, FFN
2048, 6 + 4 layers, vocabulary 6561): prompt setups in one ragged call, then streams with steady, ramped and final
windows riding one call each, long enough for the trim to engage.

Tolerance: bf16 MFMA GEMM inputs and fp16 keys / values / residual stream (the reference's activation dtype) against
fp32: rel-L2 of each window's ``mu`` <= 6e-3 (measured 3.4e-3 .. 3.8e-3).
"""

import numpy as np
import pytest
import torch

from oracle import flow as of

import t2w_amd  # noqa: F401
from t2w_amd.config import FlowConfig
from t2w_amd.flow import FlowEncoder, FlowModel
from t2w_amd.weights import init_flow

from conftest import rel

pytestmark = pytest.mark.gpu

TOL = 6e-3


@pytest.fixture(scope="module")
def flow(dev):
    W = init_flow(FlowConfig(), seed=11)
    model = FlowModel(W, FlowConfig(), device=dev)
    return W, of.enc_dims_of(W), FlowEncoder(model, n_slots1=4096, n_slots2=8192, n_cnn=64)


def test_speaker_affine(flow):
    W, _, enc = flow
    spk = torch.randn(3, 192, generator=torch.Generator().manual_seed(0)) * 2
    out = enc.model.speaker(spk.cuda()).cpu()
    assert rel(out, of.speaker(W, spk)) < 1e-5


def test_setup_and_streams_match_oracle(flow):
    W, d, enc = flow
    g = torch.Generator().manual_seed(3)
    tok = lambda n: torch.randint(0, d.vocab, (n,), generator=g).tolist()  # noqa: E731
    prompts = [tok(30), tok(57), tok(8)]
    states, mu, rows, frames = enc.setup(prompts)
    assert frames == [2 * len(p) for p in prompts]
    ref_states = []
    for i, p in enumerate(prompts):
        ref_mu, st = of.setup(W, d, p)
        ref_states.append(st)
        got = mu[rows[i]:rows[i] + frames[i]].t().cpu()
        err = rel(got, ref_mu)
        print(f"setup prompt {i} ({len(p)} tokens): rel {err:.2e}", flush=True)
        assert err < TOL
    # streams from the prompts (shared slots), a second stream of prompt 0 that gets a ramped first window
    streams = [enc.clone(s) for s in states] + [enc.clone(states[0])]
    refs = [of.EncState(s.att.clone(), s.cnn.clone(), s.keep) for s in ref_states] + \
           [of.EncState(ref_states[0].att.clone(), ref_states[0].cnn.clone(), ref_states[0].keep)]
    for s in states:
        enc.release(s)
    plan = [  # per call: (tokens, last) for streams 0..3 (None: not in the call)
        [(28, False), (28, False), (28, False), (11, False)],
        [(28, False), (28, False), None, (28, False)],
        [(28, False), (28, False), (28, False), (28, False)],
        [(28, False), (13, True), (28, False), (28, False)],
        [(28, False), None, (9, True), (28, False)],
        [(5, True), None, None, (28, False)],
    ]
    live = [True] * 4
    for c, call in enumerate(plan):
        idx = [i for i, w in enumerate(call) if w is not None]
        assert all(live[i] for i in idx)
        wins = {i: tok(call[i][0]) for i in idx}
        mu, rows, frames = enc.encode([streams[i] for i in idx], [wins[i] for i in idx], [call[i][1] for i in idx])
        for k, i in enumerate(idx):
            ref_mu = of.encode_window(W, d, refs[i], wins[i], call[i][1])
            got = mu[rows[k]:rows[k] + frames[k]].t().cpu()
            assert got.shape == ref_mu.shape
            err = rel(got, ref_mu)
            print(f"call {c} stream {i} ({call[i][0]} tokens, last={call[i][1]}, cache {refs[i].att.shape[2]}): rel {err:.2e}", flush=True)
            assert err < TOL
            if not call[i][1]:
                assert streams[i].k2.size == refs[i].att.shape[2] and 2 * streams[i].k1.size == refs[i].att.shape[2]
            else:
                live[i] = False
    for i, s in enumerate(streams):
        enc.release(s)
    assert enc.in_use() == (0, 0, 0)


def test_batched_equals_single(flow):
    """Streams are independent: one call over three streams gives each what it gets alone (up to the GEMMs' summation
    order, which follows the call's row count)."""
    W, d, enc = flow
    g = torch.Generator().manual_seed(5)
    tok = lambda n: torch.randint(0, d.vocab, (n,), generator=g).tolist()  # noqa: E731
    prompts = [tok(20), tok(44), tok(33)]
    wins = [tok(28), tok(11), tok(17)]
    lasts = [False, False, True]
    sa, _, _, _ = enc.setup(prompts)
    sb = [enc.clone(s) for s in sa]
    mu, rows, frames = enc.encode(sa, wins, lasts)
    for i in range(3):
        m1, r1, f1 = enc.encode([sb[i]], [wins[i]], [lasts[i]])
        assert rel(m1[:f1[0]], mu[rows[i]:rows[i] + frames[i]]) < 2e-3
    for s in sa + sb:
        enc.release(s)
    assert enc.in_use() == (0, 0, 0)


def test_window_errors(flow):
    _, d, enc = flow
    st = enc.new_state(10)
    with pytest.raises(ValueError):
        enc.encode([st], [[1, 2, 3]], [False])  # no frame left after the lookahead
    with pytest.raises(ValueError):
        enc.encode([st], [[d.vocab] * 5], [True])
    assert enc.in_use() == (0, 0, 0)


def test_window_graphs_equal_eager(dev):
    """Window calls replayed from captured graphs (one per call shape; the key lists' lengths are not part of it)
    equal the eager calls bit for bit, through steady, ramped and final windows past the trim; prompt setups stay
    eager."""
    W = init_flow(FlowConfig(), seed=11)
    model = FlowModel(W, FlowConfig(), device=dev)
    encs = [FlowEncoder(model, n_slots1=4096, n_slots2=8192, n_cnn=64, use_graphs=gr) for gr in (False, True)]
    g = torch.Generator().manual_seed(4)
    tok = lambda n: torch.randint(0, 6561, (n,), generator=g).tolist()  # noqa: E731
    prompts = [tok(40), tok(23)]
    sts = [e.setup(prompts)[0] for e in encs]
    plan = [([28, 28], [False, False])] * 6 + [([13, 28], [False, False]), ([28, 9], [False, True])]
    for sizes, lasts in plan:
        wins = [tok(n) for n in sizes]
        live = [i for i in range(2) if sts[0][i] is not None]
        outs = [e.encode([st[i] for i in live], [wins[i] for i in live], [lasts[i] for i in live])[0] for e, st in zip(encs, sts)]
        assert torch.equal(outs[0], outs[1])
        for st in sts:
            for i in live:
                if lasts[i]:
                    st[i] = None
    assert encs[1].counts["graph"] == len(plan) and encs[1].counts["eager"] == 1  # the setup
    assert len(encs[1].graphs) < len(plan)  # steady windows share one graph
    for e, st in zip(encs, sts):
        for x in st:
            if x is not None:
                e.release(x)
    assert all(e.in_use() == (0, 0, 0) for e in encs)
