"""Token2Wav hot-path benchmark on one MI355X: 10-step CFG Euler DiT solve + HiFT, B=32 CFG rows (16 streams x 400
mel frames, chunk-causal attention with chunk 50), random-init weights, synthetic inputs resident in HBM.

Prints one JSON line: mel frames/s of the 16 streams' output (value), audio-seconds/s, per-chunk p50 latency of a
streaming chunk through ``BatchedToken2Wav.decode`` (300-frame cached prompt, steady 50-frame windows, one stream, CFG
pair, 10 steps, HiFT with its 8 cached mel frames and source cache, cross-fade, device-to-host copy), the roofline of
the dominant kernel (the gated-residual GEMM instantiation that runs proj and fc2, timed with HIP events on its own
stream), every DiT GEMM of the workload next to hipBLASLt on the same shape, the ragged variant (lengths uniform
150-450), fp8 block GEMMs, HiFT alone, and the fp32 CPU oracle baseline timed on a bounded sample on this host.
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
HBM_PEAK_GBS = 8000.0


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


def hift_model(Wh, mode: str, use_graphs: bool = True):
    """HiFT in one of three precisions: "reference" (the reference's split: f0 predictor, source, conv_pre, stage 0's
    transposed conv and conv_post fp32, the other decoder convs on bf16 MFMA where the reference allows TF32), "bf16"
    (every decoder conv on bf16 MFMA), "fp32" (strict fp32)."""
    from t2w_amd.config import HiFTConfig
    from t2w_amd.hift import REFERENCE_FP32_CONVS, HiFTModel

    return HiFTModel(Wh, HiFTConfig(), decode_bf16=mode != "fp32", use_graphs=use_graphs,
                     fp32_convs=REFERENCE_FP32_CONVS if mode == "reference" else ())


HIFT_DESC = {"reference": "HiFT in the reference's precision split (fp32 f0/source/conv_pre/ups.0/conv_post, bf16-MFMA elsewhere)",
             "bf16": "HiFT with every decoder conv on bf16 MFMA (fp32 f0/source)", "fp32": "HiFT strict fp32"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--streams", type=int, default=16)
    ap.add_argument("--frames", type=int, default=400)
    ap.add_argument("--chunk", type=int, default=50)
    ap.add_argument("--hift-mode", choices=("reference", "bf16", "fp32"), default="reference")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-hift", action="store_true")
    ap.add_argument("--latency-reps", type=int, default=20)
    ap.add_argument("--no-extra", action="store_true", help="skip the ragged-length and HiFT-alone measurements")
    ap.add_argument("--no-fp8", action="store_true", help="skip the fp8 (e4m3 weights, MX fp8 activations) measurement")
    ap.add_argument("--no-gemms", action="store_true", help="skip the per-GEMM timings and their hipBLASLt comparison")
    ap.add_argument("--latency-only", action="store_true", help="only the per-chunk latency case")
    ap.add_argument("--no-flow", action="store_true", help="skip the flow encoder (codec-token chunk latency, encoder workload)")
    ap.add_argument("--flow-only", action="store_true", help="only the flow encoder workload (16 streams, 28-token windows)")
    ap.add_argument("--hift-kernels-only", action="store_true",
                    help="only HiFT's elementwise kernels on the workload's shape (for a rocprofv3 run of just those launches)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the dominant kernel's launches, after three 256 MiB calibration copies (for rocprofv3 --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (no sharding or collectives); use --gpus 1", file=sys.stderr)
        return 2

    import t2w_amd  # noqa: F401
    from t2w_amd.config import DiTConfig, HiFTConfig

    cfg = DiTConfig()
    if args.roofline_only:
        r = resid_gemm_roofline(cfg, args.streams, args.frames, calibrate=True)
        print(json.dumps({"kernel": r["kernel"], "launch_ms": r["launch_ms"], "tflops": r["achieved"], "calibration_copy_bytes": 2 * (256 << 20)}))
        return 0
    if args.hift_kernels_only:
        from t2w_amd.weights import init_hift

        print(json.dumps(hift_kernel_table(init_hift(HiFTConfig(), seed=3), args.streams, args.frames, args.hift_mode)))
        return 0
    if args.flow_only:
        print(json.dumps(flow_workload(args, flow_encoder())))
        return 0
    from t2w_amd.dit import DiTModel, FastDiT
    from t2w_amd.weights import init_dit, init_hift

    dev = "cuda"
    W = init_dit(cfg, seed=2)
    model = DiTModel(W, cfg, fp8=not args.no_fp8)
    model.drop_table_weights()
    n, T = args.streams, args.frames
    fd = FastDiT(model, n_slots=max(8192, 4 * n * 450 + 4096), max_streams=2 * n + 2, use_graphs=True)
    g = torch.Generator().manual_seed(2)
    mus = [torch.randn(cfg.mel, T, generator=g).to(dev) for _ in range(n)]
    spks = torch.randn(n, cfg.mel, generator=g).to(dev)
    caches = [fd.new_cache() for _ in range(n)]

    hift = Wh = None
    if not args.no_hift:
        Wh = init_hift(HiFTConfig(), seed=3)
        hift = hift_model(Wh, args.hift_mode)
        hsrc = torch.zeros(n, 1, 0, device=dev)
        hnoise = hift.noise([1000 + i for i in range(n)], T * hift.cfg.upsample_scale)

    if args.latency_only:
        print(json.dumps(chunk_latency(model, Wh, args, None if args.no_flow else flow_encoder())))
        return 0

    def step():
        mels = fd.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
        if hift is not None:
            hift.forward_noise(torch.stack(mels), hsrc, *hnoise)
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

    roof = in_solve_roofline(cfg, fd, caches, mus, spks, args.chunk, resid_gemm_roofline(cfg, n, T))
    roof["traffic"] = pmc_traffic()
    hk = None if (hift is None or args.no_extra) else hift_kernel_table(Wh, n, T, args.hift_mode)
    gemms = None if args.no_gemms else dit_gemm_table(cfg, n, T)

    enc = flow_encoder() if not args.no_flow else None
    lat = chunk_latency(model, Wh, args, enc) if args.latency_reps > 0 else {}

    extra = {}
    if not args.no_fp8:
        extra["fp8"] = fp8_workload(args, cfg, model, mus, spks, hift, hsrc if hift is not None else None,
                                    hnoise if hift is not None else None, step)
        extra["fp8_weights"] = fp8_workload(args, cfg, model, mus, spks, hift, hsrc if hift is not None else None,
                                            hnoise if hift is not None else None, step, mode="weights")
    if not args.no_extra:
        extra.update(extra_workloads(args, cfg, fd, spks, hift, Wh))
    if enc is not None:
        extra["flow_encoder"] = flow_workload(args, enc)
    if not args.no_extra:
        extra["co_scheduling"] = cu_share_workload(args, model, fd, caches, mus, spks, Wh)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(W, T, args.chunk, hift_weights=Wh)

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
                               + ("" if hift is None else " + " + HIFT_DESC[args.hift_mode]),
                   "global_batch": 2 * n, "seq_len": T, "parallelism": "single GPU"},
        "audio_seconds_per_s": frames / 50.0 / dt,
        **lat,
        "dit_solve_ms": dit_dt * 1e3,
        "dit_mfma_frac": (gemm_f + attn_f) / dit_dt / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "roofline": roof,
        "dit_gemms": gemms,
        "hift_kernels": hk,
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(res))
    return 0


def _timed(launch, reps: int = 20, warm: int = 3) -> float:
    """Mean duration (ms) of ``launch(stream)`` over ``reps`` launches on a side stream, HIP events on that stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())  # operands were written on the current stream
    with torch.cuda.stream(s):
        for _ in range(warm):
            launch(s.cuda_stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            launch(s.cuda_stream)
        e1.record(s)
    s.synchronize()
    return e0.elapsed_time(e1) / reps


def resid_gemm_roofline(cfg, n: int, T: int, calibrate: bool = False) -> dict:
    """The dominant kernel of the DiT solve by total time: the gated fp16-residual GEMM instantiation (208 x 256
    tiles, dense A) that runs the attention output projection (K = H) and fc2 (K = F) of every block.  Its launches
    are timed as the solve issues them, proj and fc2 alternating at the workload's 2 n T tokens, 20 launches with HIP
    events on their own stream; achieved = the mean algorithmic FLOPs per launch / the mean launch time.  calibrate:
    first three plain 256 MiB device copies, the known-size reference for the HBM byte counters of a rocprofv3 --pmc
    run of this same command."""
    from t2w_amd import _lib

    dev = "cuda"
    if calibrate:
        src = torch.ones(64 << 20, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    H, F, N = cfg.hidden, cfg.ffn, 2 * n * T
    g = torch.Generator(device=dev).manual_seed(7)
    ao = torch.randn(N, H, device=dev, generator=g).bfloat16()
    big = torch.randn(N, F, device=dev, generator=g).bfloat16()
    Wp = (torch.randn(H, H, device=dev, generator=g) / H ** 0.5).bfloat16()
    W2 = (torch.randn(H, F, device=dev, generator=g) / F ** 0.5).bfloat16()
    b, gate = torch.zeros(H, device=dev), torch.full((H,), 1e-3, device=dev)
    h = torch.randn(N, H, device=dev, generator=g).half()
    L = _lib.lib()
    state = {"i": 0}

    def launch(st):
        A, Wt, K = (ao, Wp, H) if state["i"] % 2 == 0 else (big, W2, F)
        state["i"] += 1
        _lib.check(L.t2w_gemm_bf16(A.data_ptr(), K, None, Wt.data_ptr(), b.data_ptr(), gate.data_ptr(), h.data_ptr(), H, N, H, K, 2, st))

    ms = _timed(launch, reps=20, warm=4)
    flops = 2.0 * N * H * (H + F) / 2
    ach = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": "gemm_kernel<208,256,2,4,EPI_RESID_F16,dense> (DiT proj and fc2, alternating)",
            "achieved": ach, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": ach / MFMA_BF16_PEAK_TFLOPS, "traffic": None,
            "launch_ms": ms, "flops_per_launch": flops}


def event_bracket_ms(reps: int = 200) -> float:
    """Median elapsed time of a pair of HIP events recorded back to back right after a small kernel: the part of an
    event-bracketed launch time that is not the kernel's."""
    x = torch.zeros(1 << 16, device="cuda")
    pairs = []
    for _ in range(reps):
        x.add_(1.0)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        e1.record()
        pairs.append((e0, e1))
    torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in pairs]))


def in_solve_roofline(cfg, fd, caches, mus, spks, chunk: int, isolated: dict) -> dict:
    """The dominant kernel's roofline as it runs inside the solve: one eager solve of the workload under the library's
    launch timer (HIP events around each of its 440 proj / fc2 launches, on the solve's stream); achieved = the mean
    algorithmic FLOPs per launch (proj and fc2 alternate) / the mean launch time, which is the bracketed time less the
    time two events recorded back to back take (``event_bracket_ms``: the bracket's own part).  The isolated launches'
    figures (``resid_gemm_roofline``) are kept under "isolated"."""
    n = len(mus)
    _, launches = fd.solve_timed(caches, mus, spks, None, [False] * n, chunk=chunk)
    ms = [m for k, m, _ in launches if k == "resid_gemm"]
    if not ms:
        return isolated
    N, H, F = 2 * sum(int(m.shape[1]) for m in mus), cfg.hidden, cfg.ffn
    flops = 2.0 * N * H * (H + F) / 2
    raw = float(np.mean(ms))
    bracket = event_bracket_ms()
    mean = raw - bracket  # the kernel's own time: rocprofv3's durations of the same launches agree with it
    ach = flops / (mean * 1e-3) / 1e12
    iso = {k: isolated[k] for k in ("achieved", "frac", "launch_ms")}
    proj, fc2 = ms[0::2], ms[1::2]
    return {"bound": "mfma", "kernel": isolated["kernel"], "achieved": ach, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": ach / MFMA_BF16_PEAK_TFLOPS, "traffic": None, "launch_ms": mean, "launches": len(ms),
            "launch_ms_bracketed": raw, "event_bracket_ms": bracket, "proj_ms": float(np.mean(proj)) - bracket,
            "fc2_ms": float(np.mean(fc2)) - bracket, "flops_per_launch": flops,
            "measured": "in-solve: HIP events around every proj / fc2 launch of one eager solve, less the bracket of two "
                        "back-to-back events",
            "isolated": iso}


def hift_kernel_table(Wh, n: int, T: int, mode: str) -> dict:
    """HiFT's elementwise kernels on the workload's shape (n rows x T mel frames, no source cache) and the Snake of the
    strict-fp32 decoder, each launch timed by the library's launch timer (HIP events on the call's stream) after a
    warm-up call: mean duration, algorithmic HBM bytes per launch (least bytes its operands make it move), GB/s and
    the fraction of the 8 TB/s HBM peak.  A launch's duration is its bracketed time less the time two events recorded
    back to back take (``event_bracket_ms``), as for the in-solve roofline; the bracketed mean is kept as "us_bracketed"."""
    from t2w_amd import _lib

    bracket = event_bracket_ms()
    out = {"event_bracket_us": bracket * 1e3}
    for tag in (mode, "fp32"):
        hm = hift_model(Wh, tag, use_graphs=False)
        ri, nz = hm.noise([4000 + i for i in range(n)], T * hm.cfg.upsample_scale)
        mel = torch.randn(n, hm.cfg.mel, T, generator=torch.Generator().manual_seed(8)).cuda() * 2 - 5
        src = torch.zeros(n, 1, 0, device="cuda")
        hm.forward_noise(mel, src, ri, nz)
        with _lib.LaunchTimer(4096) as t:
            hm.forward_noise(mel, src, ri, nz)
        agg: dict[str, list] = {}
        for kind, ms, by in t.launches:
            agg.setdefault(kind.replace("hift_", ""), []).append((ms, by))
        for k, v in agg.items():
            if k in out:
                continue
            braw = float(np.mean([a for a, _ in v]))
            ms = max(braw - bracket, 1e-4)
            by = float(np.mean([b for _, b in v]))
            out[k] = {"us": ms * 1e3, "us_bracketed": braw * 1e3, "bytes": by, "GB/s": by / ms / 1e6,
                      "frac": by / ms / 1e6 / HBM_PEAK_GBS, "launches": len(v), "mode": tag}
        del hm
    out["shape"] = f"{n} rows x {T} mel frames ({n * T * 480} samples), no source cache"
    return out


def dit_gemm_table(cfg, n: int, T: int) -> dict:
    """Every block GEMM of the workload (2 n T tokens) alone, with the solve's epilogue where the kernel-level entry
    point has it (qkv without its fused q/k LayerNorm and key scatter), next to hipBLASLt (torch.matmul, bf16 out) on
    the same shape: TFLOP/s and the fraction of bf16 peak of each, 20 launches each with HIP events."""
    from t2w_amd import _lib

    dev, L = "cuda", _lib.lib()
    H, F, N = cfg.hidden, cfg.ffn, 2 * n * T
    R = 2 * n
    g = torch.Generator(device=dev).manual_seed(9)
    a_src = torch.from_numpy((np.arange(N) + 2 * np.repeat(np.arange(R), T)).astype(np.int32)).to(dev)
    P = torch.randn(N + 2 * R, H, device=dev, generator=g).bfloat16()
    X = {H: torch.randn(N, H, device=dev, generator=g).bfloat16(), F: torch.randn(N, F, device=dev, generator=g).bfloat16()}
    h = torch.randn(N, H, device=dev, generator=g).half()
    gate = torch.full((max(3 * H, F),), 1e-3, device=dev)
    bias = torch.zeros(max(3 * H, F), device=dev)
    out = torch.empty(N, max(3 * H, F), dtype=torch.bfloat16, device=dev)
    # name: (N_out, K, epilogue, taps)
    shapes = {"qkv": (3 * H, H, 0, False), "proj": (H, H, 2, False), "conv1": (H, 3 * H, 0, True), "conv2": (H, 3 * H, 2, True),
              "fc1": (F, H, 1, False), "fc2": (H, F, 2, False)}
    res = {}
    for name, (No, K, epi, taps) in shapes.items():
        Wt = (torch.randn(No, K, device=dev, generator=g) / K ** 0.5).bfloat16()
        A = P if taps else X[K]
        C, ldc = (h, H) if epi == 2 else (out, No)

        def launch(st, A=A, Wt=Wt, C=C, ldc=ldc, No=No, K=K, epi=epi, taps=taps):
            _lib.check(L.t2w_gemm_bf16(A.data_ptr(), H if taps else K, a_src.data_ptr() if taps else None, Wt.data_ptr(), bias.data_ptr(),
                                       gate.data_ptr() if epi == 2 else None, C.data_ptr(), ldc, N, No, K, epi, st))

        ms = _timed(launch)
        Al = torch.cat([P[a_src.long() + j] for j in range(3)], 1) if taps else A
        Wc = Wt.t()
        lib_ms = _timed(lambda st, Al=Al, Wc=Wc: torch.matmul(Al, Wc))
        fl = 2.0 * N * No * K
        res[name] = {"us": ms * 1e3, "tflops": fl / ms / 1e9, "frac": fl / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS,
                     "hipblaslt_us": lib_ms * 1e3, "hipblaslt_frac": fl / lib_ms / 1e9 / MFMA_BF16_PEAK_TFLOPS}
        del Al
    tot = sum(2.0 * N * No * K for No, K, _, _ in shapes.values())
    ours = sum(v["us"] for v in res.values()) * 1e-6
    lib = sum(v["hipblaslt_us"] for v in res.values()) * 1e-6
    return {"tokens": N, "per_gemm": res, "block_frac": tot / ours / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "block_frac_hipblaslt": tot / lib / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "note": "isolated launches; hipBLASLt without fused epilogues (taps as an explicit im2col)"}


def pmc_traffic() -> float | None:
    """HBM bytes per launch of the dominant kernel as measured by the committed rocprofv3 --pmc summary (FETCH_SIZE +
    WRITE_SIZE of its dispatches, each scaled by the same counter's reading on a plain copy of known size), or None
    when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "gemm_resid_f16_b32x400_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def flow_encoder(seed: int = 5):
    """The flow encoder (CosyVoice2-style conformer, width 512) with random-init weights and pools for the workloads;
    window calls replay captured graphs."""
    from t2w_amd.config import FlowConfig
    from t2w_amd.flow import FlowEncoder, FlowModel
    from t2w_amd.weights import init_flow

    return FlowEncoder(FlowModel(init_flow(FlowConfig(), seed), FlowConfig()), n_slots1=16384, n_slots2=32768, n_cnn=1024,
                       use_graphs=True)


def _latency(bt, st, wins, reps: int) -> tuple[float, dict]:
    ts = []
    for i in range(reps + 3):
        torch.cuda.synchronize()
        a = time.perf_counter()
        bt.decode([(st, wins[i], False)])
        b = time.perf_counter()
        if i >= 3:
            ts.append(b - a)
    bt.profile = {}
    for i in range(reps):
        bt.decode([(st, wins[reps + 3 + i], False)])
    prof = {k: v[1] / v[0] * 1e3 for k, v in bt.profile.items()}
    bt.profile = None
    return float(np.median(ts) * 1e3), prof


def chunk_latency(model, Wh, args, enc=None) -> dict:
    """One stream through ``BatchedToken2Wav.decode`` as the worker calls it: a 150-token prompt (300 mel frames) set
    up, then steady windows of 28 codec tokens (25 + 3 lookahead: 50 mel frames; kept, so the caches grow and trim),
    each through the flow encoder, the solve and HiFT over 8 cached + 50 new mel frames with a 3840-sample source
    cache, the cross-fade and the device-to-host copy; graphs on.  p50 of the whole call over ``latency_reps`` windows
    after three, then the mean of its encoder, solve and vocode stages (the module's profile hook).  The same with the
    encoder bypassed (50-frame ``mu`` windows) for the DiT + HiFT part alone."""
    from t2w_amd.dit import FastDiT
    from t2w_amd.token2wav import BatchedToken2Wav, prompt_features

    dev, mel = "cuda", model.cfg.mel
    if Wh is None:
        return {}
    fl = FastDiT(model, n_slots=8192, max_streams=4, use_graphs=True)
    hm = hift_model(Wh, args.hift_mode)
    g = torch.Generator().manual_seed(11)
    mk = lambda *s: torch.randn(*s, generator=g).to(dev)  # noqa: E731
    reps = args.latency_reps
    out = {}
    if enc is not None:
        bt = BatchedToken2Wav(fl, hm, flow=enc)
        tok = lambda n: torch.randint(0, 6561, (n,), generator=g)  # noqa: E731
        feats = (tok(150)[None], torch.tensor([150]), torch.randn(1, 192, generator=g), torch.randn(1, 300, mel, generator=g), torch.tensor([300]))
        st = bt.new_stream(bt.setup(feats), noise_seed=7, adopt=True)
        p50, prof = _latency(bt, st, [tok(28).tolist() for _ in range(2 * reps + 6)], reps)
        bt.release_stream(st)
        out.update({"p50_chunk_latency_ms": p50, "p50_chunk_encoder_ms": prof.get("encoder"), "p50_chunk_dit_ms": prof.get("solve"),
                    "p50_chunk_hift_ms": prof.get("vocode")})
    bt = BatchedToken2Wav(fl, hm)
    st = bt.new_stream(bt.setup(prompt_features(mk(mel, 300), mk(mel), mk(mel, 300))), noise_seed=7, adopt=True)
    p50, prof = _latency(bt, st, [mk(mel, 50) for _ in range(2 * reps + 6)], reps)
    bt.release_stream(st)
    out.update({"p50_chunk_latency_no_encoder_ms": p50, "p50_chunk_dit_no_encoder_ms": prof.get("solve"),
                "p50_chunk_hift_no_encoder_ms": prof.get("vocode")})
    out["chunk_case"] = ("BatchedToken2Wav.decode of one stream: 150-token / 300-frame prompt cached, steady windows of 28 codec "
                         "tokens (50 mel frames) through the flow encoder, the solve, HiFT on 58 frames, glue and the "
                         "device-to-host copy; the no_encoder figures pass 50-frame mu windows; stage times are means of "
                         "profiled calls")
    return out


def cu_share_workload(args, model, fd, caches, mus, spks, Wh) -> dict:
    """The module on a CU-masked stream (co-scheduling with other work of the same process, without MPS): the
    16 x 400 solve (its graph replayed on the masked stream) and the per-chunk latency of the DiT + HiFT decode path
    (50-frame windows on a 300-frame prompt, graphs), at shares of the device's CUs evenly spread over its XCDs."""
    from t2w_amd.cosched import CUStream, device_cus
    from t2w_amd.dit import FastDiT
    from t2w_amd.token2wav import BatchedToken2Wav, prompt_features

    total = device_cus()
    n = len(mus)
    fl = FastDiT(model, n_slots=8192, max_streams=4, use_graphs=True)
    bt = BatchedToken2Wav(fl, hift_model(Wh, args.hift_mode)) if Wh is not None else None
    g = torch.Generator().manual_seed(13)
    mel = model.cfg.mel
    mk = lambda *s: torch.randn(*s, generator=g).cuda()  # noqa: E731
    res = {}
    for share in (total, 3 * total // 4, total // 2, total // 4):
        cs = CUStream(share)
        with cs:
            fd.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
            cs.stream.synchronize()
            t0 = time.perf_counter()
            for _ in range(3):
                fd.solve(caches, mus, spks, None, [False] * n, chunk=args.chunk)
            cs.stream.synchronize()
            solve_ms = (time.perf_counter() - t0) / 3 * 1e3
            p50 = None
            if bt is not None:
                st = bt.new_stream(bt.setup(prompt_features(mk(mel, 300), mk(mel), mk(mel, 300))), noise_seed=5, adopt=True)
                ts = []
                for i in range(13):
                    w = mk(mel, 50)
                    cs.stream.synchronize()
                    a = time.perf_counter()
                    bt.decode([(st, w, False)])
                    if i >= 3:
                        ts.append(time.perf_counter() - a)
                bt.release_stream(st)
                p50 = float(np.median(ts) * 1e3)
        cs.close()
        res[str(share)] = {"solve_16x400_ms": solve_ms, "p50_chunk_no_encoder_ms": p50}
    return {"device_cus": total, "by_cus": res,
            "case": "CU-masked stream (t2w_stream_create_cu_mask), CUs evenly spread over the XCDs; solve: the 16 x 400 "
                    "workload's graph; chunk: BatchedToken2Wav.decode of 50-frame mu windows, 300-frame prompt"}


def flow_workload(args, enc) -> dict:
    """The flow encoder alone on the B=32 workload's streams: 16 prompts of uniform 75-225 tokens (150-450 mel frames,
    numpy default_rng(2)) set up in one call, advanced through four steady windows (so the caches are trimmed), then
    one call of 16 windows of 28 tokens (25 + 3 lookahead -> 50 mel frames each) timed on clones of that state (HIP
    events around the call, host planning included in the wall time)."""
    n = args.streams
    rng = np.random.default_rng(2)
    plen = [int(x) for x in rng.integers(75, 226, size=n)]
    prompts = [rng.integers(0, 6561, p).tolist() for p in plen]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    states, _, _, _ = enc.setup(prompts)
    torch.cuda.synchronize()
    setup_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(4):
        enc.encode(states, [rng.integers(0, 6561, 28).tolist() for _ in range(n)], [False] * n)
    wins = [rng.integers(0, 6561, 28).tolist() for _ in range(n)]
    walls, gpu = [], []
    for i in range(args.latency_reps + 3):
        cl = [enc.clone(s) for s in states]
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a = time.perf_counter()
        e0.record()
        enc.encode(cl, wins, [False] * n)
        e1.record()
        torch.cuda.synchronize()
        b = time.perf_counter()
        for c in cl:
            enc.release(c)
        if i >= 3:
            walls.append(b - a)
            gpu.append(e0.elapsed_time(e1))
    keys1 = [s.k1.size + 25 for s in states]
    keys2 = [s.k2.size + 50 for s in states]
    for s in states:
        enc.release(s)
    return {"streams": n, "prompt_tokens": "uniform 75-225", "setup_ms": setup_ms, "p50_call_ms": float(np.median(walls) * 1e3),
            "p50_call_gpu_ms": float(np.median(gpu)), "mel_frames_per_s": n * 50 / float(np.median(walls)),
            "keys_per_stream_stack1": f"{min(keys1)}-{max(keys1)}", "keys_per_stream_stack2": f"{min(keys2)}-{max(keys2)}",
            "case": "16 windows of 28 codec tokens in one encoder call, caches after 4 windows (trimmed)"}


def fp8_workload(args, cfg, model, mus, spks, hift, hsrc, hnoise, bf16_step, mode="mx") -> dict:
    """The same 16 x 400 workload with fp8 block GEMMs; error of its mels against the bf16 solve's on identical inputs
    and weights.  mode "mx": fp8 MFMA (e4m3 weights with per-output-channel scales, MX fp8 activations); "weights":
    the same e4m3 weights dequantized to bf16 before each GEMM, bf16 activations and MFMA (config 5 as written)."""
    from t2w_amd.dit import FastDiT

    n = len(mus)
    T = int(mus[0].shape[1])
    f8 = FastDiT(model, n_slots=max(8192, 2 * n * T + 4096), max_streams=n + 2, use_graphs=True, fp8=True if mode == "mx" else mode)
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
            "config": f"{n} streams x {T} frames, CFG B={2 * n}, chunk {args.chunk}, block GEMMs "
                      + ("fp8 e4m3 / MX fp8 on fp8 MFMA" if mode == "mx" else "e4m3 weights (per-channel scales) dequantized "
                         "to bf16, bf16 activations and MFMA")
                      + ", in_proj / final linear / attention bf16" + ("" if hift is None else " + HiFT")}


def extra_workloads(args, cfg, fd, spks, hift, Wh) -> dict:
    """The ragged 16-stream workload (lengths uniform 150-450, seed 2; DiT solve + HiFT of the ragged mels) and HiFT
    alone (16 rows of mel ~ N(-5, 2), lengths uniform 50-400, seed 3) in each precision, timed over args.steps calls
    after a warm-up call."""
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
    for tag in ("fp32", "reference", "bf16"):
        hm = hift_model(Wh, tag)
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
    def median_of(fn, runs: int = 5) -> float:  # one warm-up, then the median of `runs` timed calls
        fn()
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    with torch.no_grad():
        temb = od.t_embed(W, torch.full((2,), 0.5))
        fwd = median_of(lambda: od.estimator_chunk(W, d, x, mu, temb, spk, torch.zeros_like(mu), cnn, att, mask, tr))
        hift_s = 0.0
        if hift_weights is not None:
            h = oh.HiFT(hift_weights)
            mel = torch.randn(1, 80, T, generator=g) * 2 - 5
            ri, nz = oh.hift_noise(9, [1], T * 480)
            hift_s = median_of(lambda: oh.forward_noise(h, mel, torch.zeros(1, 1, 0), ri, nz))
    total = 10 * fwd + hift_s
    return {"value": T / total, "unit": "mel frames/s", "cores": cores, "kind": "port",
            "sample": f"fp32 oracle: estimator forward of a CFG pair (2 x {T} frames, chunk {chunk}) x 10 steps + HiFT of one "
                      f"{T}-frame mel ({'timed' if hift_weights is not None else 'not run'}); each the median of 5 runs after one "
                      f"warm-up: forward {fwd:.2f} s, HiFT {hift_s:.2f} s"}


if __name__ == "__main__":
    sys.exit(main())
