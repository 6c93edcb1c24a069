"""ctypes binding of ``libt2w_hip.so`` (the C ABI declared in ``include/t2w.h``).

The library is loaded from the package directory; a missing library is an error (there is no CPU fallback).  Device
pointers are passed as integers from ``torch.Tensor.data_ptr()`` and the stream as the raw ``hipStream_t`` of torch's
current stream.
"""

from __future__ import annotations

import ctypes as C
import pathlib

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libt2w_hip.so"

P = C.c_void_p
I = C.c_int
F = C.c_float
FP = C.POINTER(C.c_float)


class DitDims(C.Structure):
    _fields_ = [(n, I) for n in ("mel", "hidden", "depth", "heads", "head_dim", "ffn", "freq", "steps")] + \
               [(n, F) for n in ("eps_block", "eps_qk", "eps_conv", "eps_final", "cfg_rate")]


class DitBlock(C.Structure):
    _fields_ = [(n, P) for n in ("qkv_w", "qkv_b", "qn_w", "qn_b", "kn_w", "kn_b", "proj_w", "proj_b", "c1_w", "c1_b",
                                 "cln_w", "cln_b", "c2_w", "c2_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b")]


class DitGlobals(C.Structure):
    _fields_ = [(n, P) for n in ("in_w", "in_b", "out_w", "out_b", "mods", "final_mods")] + [("dts", FP), ("rope_freq", P)]


class ModWeights(C.Structure):
    _fields_ = [(n, P) for n in ("freqs", "te0_w", "te0_b", "te2_w", "te2_b", "ada_w", "ada_b", "fin_w", "fin_b")]


class SolveArgs(C.Structure):
    _fields_ = [(n, I) for n in ("n_tok", "n_rows", "half", "n_tiles", "chunk")] + \
               [(n, P) for n in ("x0", "stat", "in_rows", "out", "tok_row", "tok_pos", "a_src", "new_slot", "row_start", "row_len",
                                 "row_kv_off", "row_kv_len", "conv_rd", "conv_wr", "kv_idx", "tiles", "k_pool", "v_pool")] + \
               [("pool_layer_stride", C.c_longlong), ("conv_pool", P), ("workspace", P), ("workspace_bytes", C.c_size_t), ("fp8", I),
                ("tok_abs", P), ("kv_max", I)]


class DitBlockFp8(C.Structure):
    _fields_ = [(n, P) for n in ("qkv_w8", "qkv_ws", "proj_w8", "proj_ws", "c1_w8", "c1_ws", "c2_w8", "c2_ws", "fc1_w8", "fc1_ws",
                                 "fc2_w8", "fc2_ws")]


class HiftDims(C.Structure):
    _fields_ = [(n, I) for n in ("mel", "base", "n_up", "harmonics", "f0_channels", "f0_layers", "sr", "n_fft", "hop")] + \
               [(n, I * 3) for n in ("up_rates", "up_kernels", "res_kernels", "res_dilations", "src_kernels")] + \
               [(n, F) for n in ("sine_amp", "noise_std", "voiced_threshold", "lrelu_slope", "audio_limit")]


class Conv(C.Structure):
    _fields_ = [("w", P), ("b", P), ("wbf", P)]


class ResBlock(C.Structure):
    _fields_ = [("c1", Conv * 3), ("c2", Conv * 3)] + [(n, P * 3) for n in ("a1", "inv1", "a2", "inv2")]


class HiftWeights(C.Structure):
    _fields_ = [("f0", Conv * 5), ("f0_head_w", P), ("f0_head_b", P), ("src_w", P), ("src_b", P), ("conv_pre", Conv), ("ups", Conv * 3),
                ("src_down", Conv * 3), ("conv_post", Conv), ("src_res", ResBlock * 3), ("res", ResBlock * 9), ("window", P)]


class FlowDims(C.Structure):
    _fields_ = [(n, I) for n in ("vocab", "dim", "heads", "ffn", "depth1", "depth2", "look", "stride", "mel", "spk", "rmax")] + \
               [(n, F) for n in ("eps_layer", "eps_embed", "eps_after")]


class FlowLayer(C.Structure):
    _fields_ = [(n, P) for n in ("qkv_w", "qkv_b", "pos_u", "pos_v", "ptab", "out_w", "out_b", "ln1_w", "ln1_b", "ln2_w", "ln2_b",
                                 "w1", "b1", "w2", "b2")]


class FlowGlobals(C.Structure):
    _fields_ = [(n, P) for n in ("embed_table", "embed_ln_w", "embed_ln_b", "conv1_w", "conv1_b", "conv2_w", "conv2_b", "up_w", "up_b",
                                 "up_ln_w", "up_ln_b", "after_w", "after_b", "proj_w", "proj_b", "spk_w", "spk_b", "ones")]


class FlowArgs(C.Structure):
    _fields_ = [(n, I) for n in ("n_rows", "n_in", "n_gap", "n1", "n_up", "n2", "n_tiles1", "n_tiles2")] + \
               [(n, P) for n in ("tok", "res", "c1_src", "gofs", "t1", "c2_src", "up_dst", "uofs", "o1", "up_src", "o2", "t2", "cnn_rd",
                                 "cnn_wr", "new1", "new2", "kv1_idx", "kv1_off", "kv1_len", "tiles1", "kv2_idx", "kv2_off", "kv2_len",
                                 "tiles2")] + \
               [("pool1", P), ("pool1_layer_stride", C.c_longlong), ("pool2", P), ("pool2_layer_stride", C.c_longlong), ("cnn_pool", P),
                ("mu_out", P), ("workspace", P), ("workspace_bytes", C.c_size_t)]


_SIGS = {
    "t2w_abi_version": (I, []),
    "t2w_last_error": (C.c_char_p, []),
    "t2w_dit_create": (I, [C.POINTER(DitDims), C.POINTER(P)]),
    "t2w_dit_set_block": (I, [P, I, C.POINTER(DitBlock)]),
    "t2w_dit_set_globals": (I, [P, C.POINTER(DitGlobals)]),
    "t2w_dit_destroy": (None, [P]),
    "t2w_dit_mods_workspace_bytes": (C.c_size_t, [P, I]),
    "t2w_dit_build_mods": (I, [P, C.POINTER(ModWeights), P, I, P, P, P, P]),
    "t2w_dit_workspace_bytes": (C.c_size_t, [P, I, I]),
    "t2w_dit_solve": (I, [P, C.POINTER(SolveArgs), P]),
    "t2w_dit_forward": (I, [P, C.POINTER(SolveArgs), I, P, P, P]),
    "t2w_timer_arm": (I, [I]),
    "t2w_timer_read": (I, [P, C.POINTER(I), FP, C.POINTER(C.c_double), I, C.POINTER(I)]),
    "t2w_dit_solve_noalloc": (I, [P, C.POINTER(SolveArgs), P]),
    "t2w_gemm_bf16": (I, [P, I, P, P, P, P, P, I, I, I, I, I, P]),
    "t2w_gemm_bf16_tile": (I, [P, I, P, P, P, P, P, I, I, I, I, I, I, P]),
    "t2w_gemm_bf16_ws": (I, [P, I, P, P, P, P, P, I, I, I, I, I, P, C.c_size_t, P]),
    "t2w_quant_mx8": (I, [P, I, I, I, P, I, P, P]),
    "t2w_dit_set_block_fp8": (I, [P, I, P]),
    "t2w_gemm_fp8": (I, [P, I, P, P, I, P, P, P, P, P, I, I, I, I, I, P]),
    "t2w_ln_mod": (I, [P, P, P, F, P, I, I, P]),
    "t2w_qk_norm_scatter": (I, [P, P, P, P, P, F, P, P, P, P, I, I, P]),
    "t2w_attention": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, F, I, I, P]),
    "t2w_hift_create": (I, [C.POINTER(HiftDims), C.POINTER(HiftWeights), C.POINTER(P)]),
    "t2w_hift_destroy": (None, [P]),
    "t2w_hift_plan_ints": (I, [I]),
    "t2w_hift_plan": (I, [P, I, P, P]),
    "t2w_hift_workspace_bytes": (C.c_size_t, [P, I, P]),
    "t2w_hift_forward": (I, [P, I, P, P, P, P, P, I, P, P, P, P, P, P, C.c_size_t, I, P]),
    "t2w_flow_create": (I, [C.POINTER(FlowDims), C.POINTER(P)]),
    "t2w_flow_set_layer": (I, [P, I, C.POINTER(FlowLayer)]),
    "t2w_flow_set_globals": (I, [P, C.POINTER(FlowGlobals)]),
    "t2w_flow_destroy": (None, [P]),
    "t2w_flow_workspace_bytes": (C.c_size_t, [P, I, I, I, I, I]),
    "t2w_flow_encode": (I, [P, C.POINTER(FlowArgs), P]),
    "t2w_flow_speaker": (I, [P, P, P, I, P]),
    "t2w_device_cus": (I, [C.POINTER(I)]),
    "t2w_stream_create_cu_mask": (I, [C.POINTER(C.c_uint32), I, C.POINTER(P)]),
    "t2w_stream_destroy": (I, [P]),
    "t2w_graph_begin": (I, [P]),
    "t2w_graph_end": (I, [P, C.POINTER(P)]),
    "t2w_graph_launch": (I, [P, P]),
    "t2w_graph_destroy": (None, [P]),
}

_lib = None


def lib():
    """The loaded library (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built: run __graft_entry__.build() (hipcc, gfx950)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise RuntimeError(f"t2w {what}: {lib().t2w_last_error().decode()}")


TIMER_KINDS = {1: "resid_gemm", 2: "hift_phase", 3: "hift_source", 4: "hift_stft", 5: "hift_istft", 6: "hift_reflect",
               7: "hift_snake", 8: "hift_f0_head"}  # the T2W_TIMER_* codes of t2w.h


class LaunchTimer:
    """``with LaunchTimer(cap) as t: <eager library calls>`` -> ``t.launches``: (kind name, ms, algorithmic bytes) of
    every instrumented launch, in launch order (``t2w_timer_arm`` / ``t2w_timer_read``; waits for the current stream)."""

    def __init__(self, cap: int = 8192):
        self.cap = int(cap)
        self.launches: list[tuple[str, float, float]] = []

    def __enter__(self):
        check(lib().t2w_timer_arm(self.cap), "timer_arm")
        return self

    def __exit__(self, *exc):
        kinds, ms, by, n = (C.c_int * self.cap)(), (C.c_float * self.cap)(), (C.c_double * self.cap)(), C.c_int()
        rc = lib().t2w_timer_read(stream_handle(), kinds, ms, by, self.cap, C.byref(n))
        if exc[0] is None:
            check(rc, "timer_read")
        self.launches = [(TIMER_KINDS.get(kinds[i], str(kinds[i])), float(ms[i]), float(by[i])) for i in range(n.value)]
        return False


def exported_symbols() -> list[str]:
    return list(_SIGS)


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(stream=None) -> int:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream
