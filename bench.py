"""Token2Wav hot-path benchmark on one MI355X: 10-step CFG Euler DiT solve + HiFT, B=32 CFG rows (16 streams x 400
mel frames, chunk-causal attention with chunk 50), random-init weights, synthetic inputs resident in HBM.

Prints one JSON line: mel frames/s of the 16 streams' output (value), audio-seconds/s, per-chunk p50 latency of a
streaming chunk (300-frame cached prompt + 50 new frames, one stream, CFG pair, 10 steps, + HiFT), the ragged variant
of the 16-stream workload (lengths uniform 150-450), HiFT alone (16 rows, 50-400 frames, fp32 and bf16 decoder), the
roofline of the dominant kernel (the DiT's conv1 GEMM, timed with HIP events on its own stream) and the fp32 CPU
oracle baseline timed on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 (AMD public spec)


def dit_flops_per_solve(cfg, rows_T: list[int], chunk: int) -> tuple[float, float]:
    """Algorithmic FLOPs of one 10-step CFG solve over real tokens: GEMMs 28 H^2 D + 2*320 H + 2 H mel per token per
    step (both CFG rows counted) and attention 4 H per visible (query, key) pair per block."""
    H, D, mel = cfg.hidden, cfg.depth, cfg.mel
    per_tok = 28 * H * H * D + 2 * 4 * mel * H + 2 * H * mel
    toks = 2 * sum(rows_T)
    pairs = 0
    for T in rows_T:
        c = np.arange(T) // chunk if chunk > 0 else np.zeros(T, dtype=int)
        lim = np.minimum(T, (c + 1) * chunk) if chunk > 0 else np.full(T, T)
        pairs += 2 * int(lim.sum())
    return float(per_tok * toks * cfg.steps), float(4 * H * pairs * D * cfg.steps)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--streams", type=int, default=16)
    ap.add_argument("--frames", type=int, default=400)
    ap.add_argument("--chunk", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-hift", action="store_true")
    ap.add_argument("--latency-reps", type=int, default=20)
    ap.add_argument("--hift-fp32", action="store_true", help="HiFT decoder in strict fp32 (default: bf16 MFMA decoder)")
    ap.add_argument("--no-extra", action="store_true", help="skip the ragged-length and HiFT-alone measurements")
    ap.add_argument("--no-fp8", action="store_true", help="skip the fp8 (e4m3 weights, MX fp8 activations) measurement")
    ap.add_argument("--latency-only", action="store_true",
                    help="only the per-chunk latency case (one stream, 300 cached + 50 new frames, + HiFT of the window)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the conv1 GEMM launches, after three 256 MiB calibration copies (for rocprofv3 --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (no sharding or collectives); use --gpus 1", file=sys.stderr)
        return 2

    import t2w_amd  # noqa: F401
    from t2w_amd import _lib
    from t2w_amd.config import DiTConfig, HiFTConfig

    if args.roofline_only:
        k_ms, k_tf, k_fl = conv1_roofline(DiTConfig(), args.streams, args.frames, calibrate=True)
        print(json.dumps({"kernel": "gemm_kernel<256,256,4,2,EPI_BF16,taps> (DiT conv1)", "launch_ms": k_ms, "tflops": k_tf,
                          "calibration_copy_bytes": 2 * (256 << 20)}))
        return 0
    from t2w_amd.dit import DiTModel, FastDiT
    from t2w_amd.weights import init_dit, init_hift

    dev = "cuda"
    cfg = DiTConfig()
    W = init_dit(cfg, seed=2)
    model = DiTModel(W, cfg, fp8=not args.no_fp8)
    model.drop_table_weights()
    n, T = args.streams, args.frames
    fd = FastDiT(model, n_slots=max(8192, 4 * n * 450 + 4096), max_streams=2 * n + 2, use_graphs=True)
    g = torch.Generator().manual_seed(2)
    mus = [torch.randn(cfg.mel, T, generator=g).to(dev) for _ in range(n)]
    spks = torch.randn(n, cfg.mel, generator=g).to(dev)
    caches = [fd.new_cache() for _ in range(n)]

    hift = None
    if not args.no_hift:
        from t2w_amd.hift import HiFTModel

        Wh = init_hift(HiFTConfig(), seed=3)
        hift = HiFTModel(Wh, HiFTConfig(), decode_bf16=not args.hift_fp32, use_graphs=True)
        hsrc = torch.zeros(n, 1, 0, device=dev)
        hnoise = hift.noise([1000 + i for i in range(n)], T * hift.cfg.upsample_scale)

    def chunk_latency():
        # one stream, 300-frame prompt cached, 50 new frames, CFG pair, 10 steps, + HiFT of the window: medians of the
        # whole call and of its DiT solve and HiFT parts
        fl = FastDiT(model, n_slots=4096, max_streams=2, use_graphs=True)
        c = fl.new_cache(keep=300)
        pm = torch.randn(cfg.mel, 300, generator=g).to(dev)
        fl.solve([c], [pm], spks[:1], [torch.randn(cfg.mel, 300, generator=g).to(dev)], [True])
        wm = torch.randn(cfg.mel, 50, generator=g).to(dev)
        hs = None
        if hift is not None:
            hs = (torch.zeros(1, 1, 0, device=dev), *hift.noise([7], 50 * hift.cfg.upsample_scale))
        ts, td, th = [], [], []
        for i in range(args.latency_reps + 3):
            torch.cuda.synchronize()
            a = time.perf_counter()
            m = fl.solve([c], [wm], spks[:1], None, [False])
            torch.cuda.synchronize()
            b = time.perf_counter()
            if hift is not None:
                hift.forward_noise(m[0][None], *hs)
            torch.cuda.synchronize()
            e = time.perf_counter()
            if i >= 3:
                ts.append(e - a)
                td.append(b - a)
                th.append(e - b)
        return float(np.median(ts) * 1e3), float(np.median(td) * 1e3), float(np.median(th) * 1e3)

    if args.latency_only:
        lat, lat_dit, lat_hift = chunk_latency()
        print(json.dumps({"p50_chunk_latency_ms": lat, "p50_chunk_dit_ms": lat_dit, "p50_chunk_hift_ms": lat_hift,
                          "reps": args.latency_reps}))
        return 0

    def step():
        mels = fd.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
        if hift is not None:
            mel = torch.stack(mels)
            hift.forward_noise(mel, hsrc, *hnoise)
        return mels

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    frames = n * T
    gemm_f, attn_f = dit_flops_per_solve(cfg, [T] * n, args.chunk)

    # DiT solve alone (for the MFMA fraction of the whole solve)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(max(1, args.steps // 2)):
        fd.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
    torch.cuda.synchronize()
    dit_dt = (time.perf_counter() - t1) / max(1, args.steps // 2)

    k_ms, k_tflops, k_flops = conv1_roofline(cfg, n, T)

    lat = lat_dit = lat_hift = None
    if args.latency_reps > 0:
        lat, lat_dit, lat_hift = chunk_latency()

    extra = {}
    if not args.no_fp8:
        extra["fp8"] = fp8_workload(args, cfg, model, mus, spks, hift, hsrc if hift is not None else None,
                                    hnoise if hift is not None else None, step)
    if not args.no_extra:
        extra.update(extra_workloads(args, cfg, fd, spks, hift, Wh if hift is not None else None))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(W, T, args.chunk, hift_weights=Wh if hift is not None else None)

    res = {
        "metric": "Token2Wav mel frames/s (10-step CFG DiT+HiFT, B=32) + per-chunk p50 latency",
        "value": frames / dt,
        "unit": "mel frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, seeded N(0,1) inputs)",
        "config": {"workload": f"{n} streams x {T} mel frames, CFG B={2 * n}, chunk-causal {args.chunk}, 10-step Euler DiT"
                               + ("" if hift is None else (" + HiFT fp32" if args.hift_fp32 else " + HiFT (bf16-MFMA decoder, fp32 f0/source)")),
                   "global_batch": 2 * n, "seq_len": T, "parallelism": "single GPU"},
        "audio_seconds_per_s": frames / 50.0 / dt,
        "p50_chunk_latency_ms": lat,
        "p50_chunk_dit_ms": lat_dit,
        "p50_chunk_hift_ms": lat_hift,
        "dit_solve_ms": dit_dt * 1e3,
        "dit_mfma_frac": (gemm_f + attn_f) / dit_dt / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "roofline": {"bound": "mfma", "kernel": "gemm_kernel<256,256,4,2,EPI_BF16,taps> (DiT conv1)", "achieved": k_tflops,
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": k_tflops / MFMA_BF16_PEAK_TFLOPS, "traffic": pmc_traffic(),
                     "launch_ms": k_ms, "flops_per_launch": k_flops},
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(res))
    return 0


def conv1_roofline(cfg, n: int, T: int, calibrate: bool = False) -> tuple[float, float, float]:
    """The dominant kernel alone: the DiT's conv1 GEMM (taps mode, bf16 out) at the workload's shape, 20 launches timed
    with HIP events on its own stream.  calibrate: first three plain 256 MiB device copies (torch copy_), the known-size
    reference for the HBM byte counters of a rocprofv3 --pmc run of this same command."""
    from t2w_amd import _lib

    dev = "cuda"
    if calibrate:
        src = torch.ones(64 << 20, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    H, N = cfg.hidden, 2 * n * T
    R = 2 * n
    P = torch.randn(N + 2 * R, H, device=dev).bfloat16()
    Wc = (torch.randn(H, 3 * H, device=dev) * 0.02).bfloat16()
    bc = torch.zeros(H, device=dev)
    tok_row = np.repeat(np.arange(R), T)
    a_src = torch.from_numpy((np.arange(N) + 2 * tok_row).astype(np.int32)).to(dev)
    out = torch.empty(N, H, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())  # operands were written on the default stream
    L = _lib.lib()
    with torch.cuda.stream(s):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        for _ in range(3):
            _lib.check(L.t2w_gemm_bf16(P.data_ptr(), H, a_src.data_ptr(), Wc.data_ptr(), bc.data_ptr(), None, out.data_ptr(), H, N, H, 3 * H, 0, s.cuda_stream))
        e0.record(s)
        for _ in range(reps):
            _lib.check(L.t2w_gemm_bf16(P.data_ptr(), H, a_src.data_ptr(), Wc.data_ptr(), bc.data_ptr(), None, out.data_ptr(), H, N, H, 3 * H, 0, s.cuda_stream))
        e1.record(s)
    s.synchronize()
    k_ms = e0.elapsed_time(e1) / reps
    flops = 2.0 * N * H * 3 * H
    return k_ms, flops / (k_ms * 1e-3) / 1e12, flops


def pmc_traffic() -> float | None:
    """HBM bytes per launch of the conv1 GEMM as measured by the committed rocprofv3 --pmc summary (FETCH_SIZE +
    WRITE_SIZE of the GEMM dispatches, each scaled by the same counter's reading on a plain copy of known size), or
    None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "gemm_conv1_b32x400_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def fp8_workload(args, cfg, model, mus, spks, hift, hsrc, hnoise, bf16_step) -> dict:
    """The same 16 x 400 workload with the block GEMMs on fp8 MFMA (e4m3 weights with per-output-channel scales, MX
    fp8 activations); error of its mels against the bf16 solve's on identical inputs and weights."""
    from t2w_amd.dit import FastDiT

    n = len(mus)
    T = int(mus[0].shape[1])
    f8 = FastDiT(model, n_slots=max(8192, 2 * n * T + 4096), max_streams=n + 2, use_graphs=True, fp8=True)
    caches = [f8.new_cache() for _ in range(n)]

    def step():
        mels = f8.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
        if hift is not None:
            hift.forward_noise(torch.stack(mels), hsrc, *hnoise)
        return mels

    ref = bf16_step()
    got = step()
    torch.cuda.synchronize()
    d = torch.cat([(a - b).flatten() for a, b in zip(got, ref)])
    r = torch.cat([b.flatten() for b in ref])
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    t1 = time.perf_counter()
    for _ in range(max(1, args.steps // 2)):
        f8.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
    torch.cuda.synchronize()
    dit_dt = (time.perf_counter() - t1) / max(1, args.steps // 2)
    for c in caches:
        f8.release(c)
    del f8
    return {"mel_frames_per_s": n * T / dt, "ms_per_step": dt * 1e3, "dit_solve_ms": dit_dt * 1e3,
            "mel_rel_l2_vs_bf16": float(d.norm() / r.norm()), "mel_max_abs_vs_bf16": float(d.abs().max()),
            "config": f"{n} streams x {T} frames, CFG B={2 * n}, chunk {args.chunk}, block GEMMs fp8 e4m3 / MX fp8, "
                      "in_proj / final linear / attention bf16" + ("" if hift is None else " + HiFT")}


def extra_workloads(args, cfg, fd, spks, hift, Wh) -> dict:
    """The ragged 16-stream workload (lengths uniform 150-450, seed 2; DiT solve + HiFT of the ragged mels) and HiFT
    alone (16 rows of mel ~ N(-5, 2), lengths uniform 50-400, seed 3), each timed over args.steps calls after a
    warm-up call."""
    from t2w_amd.config import HiFTConfig
    from t2w_amd.hift import HiFTModel

    dev = "cuda"
    n = args.streams
    rng = np.random.default_rng(2)
    lens = [int(x) for x in rng.integers(150, 451, size=n)]
    g = torch.Generator().manual_seed(2)
    mus = [torch.randn(cfg.mel, t, generator=g).to(dev) for t in lens]
    caches = [fd.new_cache() for _ in range(n)]
    hnz = None
    if hift is not None:
        ri, nz = hift.noise([2000 + i for i in range(n)], max(lens) * 480)
        hnz = torch.cat([nz[i, : t * 480] for i, t in enumerate(lens)])

    def ragged():
        mels = fd.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
        if hift is not None:
            hift.forward_packed(lens, torch.cat([m.t() for m in mels]), hnz, None, 0)

    ragged()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ragged()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    for c in caches:
        fd.release(c)
    out = {"ragged_b32": {"mel_frames_per_s": sum(lens) / dt, "ms_per_step": dt * 1e3, "frames": sum(lens),
                          "lengths": "uniform 150-450 (numpy default_rng(2))", "hift": hift is not None}}
    if Wh is None:
        return out
    rng = np.random.default_rng(3)
    hl = [int(x) for x in rng.integers(50, 401, size=16)]
    g = torch.Generator().manual_seed(3)
    mel_tm = torch.cat([torch.randn(t, cfg.mel, generator=g) * 2 - 5 for t in hl]).to(dev)
    res = {"rows": 16, "lengths": "uniform 50-400 (numpy default_rng(3))", "frames": sum(hl)}
    for tag, bf in (("fp32", False), ("bf16", True)):
        hm = HiFTModel(Wh, HiFTConfig(), decode_bf16=bf, use_graphs=True)
        ri, nz = hm.noise([3000 + i for i in range(16)], max(hl) * 480)
        ntm = torch.cat([nz[i, : t * 480] for i, t in enumerate(hl)])
        hm.forward_packed(hl, mel_tm, ntm, None, 0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            hm.forward_packed(hl, mel_tm, ntm, None, 0)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / args.steps
        res[f"{tag}_samples_per_s"] = sum(hl) * 480 / dt
        res[f"{tag}_ms_per_call"] = dt * 1e3
        del hm
    out["hift_alone"] = res
    return out


def cpu_baseline(W, T: int, chunk: int, hift_weights=None) -> dict:
    """fp32 CPU oracle on this host's cores: one estimator forward of one stream's CFG pair (2 rows x T frames,
    chunk-causal) x 10 steps, plus HiFT of the stream's T-frame mel; mel frames/s of that one stream."""
    from oracle import dit as od
    from oracle import hift as oh

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    d = od.dims_of(W)
    g = torch.Generator().manual_seed(5)
    x, mu = torch.randn(2, 80, T, generator=g), torch.randn(2, 80, T, generator=g)
    spk = torch.randn(2, 80, generator=g)
    cnn = torch.zeros(d.depth, 2, 2 * d.hidden, 2)
    att = torch.zeros(d.depth, 2, d.heads, 0, 2 * d.head_dim)
    mask = od.chunk_mask(T, chunk)[None].expand(2, T, T)
    tr = torch.full((2,), T, dtype=torch.int64)
    with torch.no_grad():
        temb = od.t_embed(W, torch.full((2,), 0.5))
        t0 = time.perf_counter()
        od.estimator_chunk(W, d, x, mu, temb, spk, torch.zeros_like(mu), cnn, att, mask, tr)
        fwd = time.perf_counter() - t0
        hift_s = 0.0
        if hift_weights is not None:
            h = oh.HiFT(hift_weights)
            mel = torch.randn(1, 80, T, generator=g) * 2 - 5
            ri, nz = oh.hift_noise(9, [1], T * 480)
            t0 = time.perf_counter()
            oh.forward_noise(h, mel, torch.zeros(1, 1, 0), ri, nz)
            hift_s = time.perf_counter() - t0
    total = 10 * fwd + hift_s
    return {"value": T / total, "unit": "mel frames/s", "cores": cores, "kind": "port",
            "sample": f"fp32 oracle: 1 estimator forward of a CFG pair (2 x {T} frames, chunk {chunk}) timed and x10 steps, "
                      f"+ HiFT of one {T}-frame mel ({'timed' if hift_weights is not None else 'not run'}); forward {fwd:.2f} s, HiFT {hift_s:.2f} s"}


if __name__ == "__main__":
    sys.exit(main())
