// Per-token row kernels of the DiT block and the Euler/CFG update.
//
// One wave64 per token row: each lane holds H / 64 consecutive values (64 contiguous bytes of fp32 for H = 1024), so a
// row is read with fully coalesced 16-byte loads and the LayerNorm statistics are two wave reductions.  Norm statistics
// and modulation are fp32 (the reference's ``dit_kernels.py`` keeps norm math in fp32); outputs that feed an MFMA GEMM
// are rounded once to bf16.
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

template <int VPL>
__device__ __forceinline__ void load_f32(const float* p, float (&v)[VPL]) {
#pragma unroll
  for (int i = 0; i < VPL / 4; ++i) {
    float4 x = *(const float4*)(p + 4 * i);
    v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
  }
}

template <int VPL>
__device__ __forceinline__ void load_bf(const bf16_t* p, float (&v)[VPL]) {
#pragma unroll
  for (int i = 0; i < VPL / 8; ++i) {
    uint4 x = *(const uint4*)(p + 8 * i);
    uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[8 * i + 2 * j] = lo2f(w[j]); v[8 * i + 2 * j + 1] = hi2f(w[j]); }
  }
  if (VPL == 4) {
    uint2 x = *(const uint2*)p;
    v[0] = lo2f(x.x); v[1] = hi2f(x.x); v[2] = lo2f(x.y); v[3] = hi2f(x.y);
  }
}

template <int VPL>
__device__ __forceinline__ void pack_bf(const float (&v)[VPL], uint32_t (&o)[VPL / 2]) {
#pragma unroll
  for (int j = 0; j < VPL / 2; ++j) o[j] = pack2(v[2 * j], v[2 * j + 1]);
}

template <int VPL>
__device__ __forceinline__ void store_packed(bf16_t* p, const uint32_t (&o)[VPL / 2]) {
  if (VPL >= 8) {
#pragma unroll
    for (int i = 0; i < VPL / 8; ++i) *(uint4*)(p + 8 * i) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  } else {
    *(uint2*)p = make_uint2(o[0], o[1]);
  }
}

// MX fp8 store of a row chunk: this lane's VPL values at c0 of a row; the 32-value block's maximum is reduced over its
// 32 / VPL lanes, and the block's first lane writes the E8M0 scale byte
template <int VPL>
__device__ __forceinline__ void store_mx8(const float (&v)[VPL], uint8_t* qrow, uint8_t* srow, int c0) {
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) a = fmaxf(a, fabsf(v[i]));
#pragma unroll
  for (int o = 1; o < 32 / VPL; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
  const int se = mx_exp(a);
  uint32_t w[VPL / 4];
#pragma unroll
  for (int i = 0; i < VPL / 4; ++i) w[i] = mx_pack4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3], se);
  if (VPL == 16) *(uint4*)(qrow + c0) = make_uint4(w[0], w[1], w[2], w[3]);
  else if (VPL == 8) *(uint2*)(qrow + c0) = make_uint2(w[0], w[1]);
  else *(uint32_t*)(qrow + c0) = w[0];
  if ((c0 & 31) == 0) srow[c0 >> 5] = (uint8_t)(se + 127);
}

// LayerNorm statistics over a row spread across the wave: v -> (v - mean) * rstd
template <int VPL>
__device__ __forceinline__ void normalize(float (&v)[VPL], int H, float eps) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) s += v[i];
  const float mean = wave_sum(s) / (float)H;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    v[i] -= mean;
    q += v[i] * v[i];
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)H + eps);
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] *= rstd;
}

// out: bf16 [N, H]; or, with q non-null, MX fp8 codes q [N, H] and block scales qs [N, H / 32]
template <int VPL>
__global__ void __launch_bounds__(256) ln_mod_kernel(const float* h, const float* shift, const float* scale1, float eps,
                                                     bf16_t* out, uint8_t* q, uint8_t* qs, int N, int H) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int c0 = lane * VPL;
  float v[VPL], sc[VPL], sh[VPL];
  load_f32<VPL>(h + (size_t)n * H + c0, v);
  normalize<VPL>(v, H, eps);
  load_f32<VPL>(scale1 + c0, sc);
  load_f32<VPL>(shift + c0, sh);
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] = v[i] * sc[i] + sh[i];
  if (q) {
    store_mx8<VPL>(v, q + (size_t)n * H, qs + (size_t)n * (H / 32), c0);
    return;
  }
  uint32_t o[VPL / 2];
  pack_bf<VPL>(v, o);
  store_packed<VPL>(out + (size_t)n * H + c0, o);
}

// Frame f of token n (position t of row r, T frames) in the padded buffer is n + 2 r + 2; it is also the row's new
// cache frame t - T + 2 when t >= T - 2.  Row programs copy the two cached frames in front of the row's frames and,
// for rows of fewer than two tokens, produce the new cache from the old one (the reference's _conv_place and
// _conv_row_cache, engine/runtime/dit_kernels.py:217-248).
template <int VPL>
__device__ __forceinline__ void place_token(const ConvPlace& cp, int n, int H, int c0, const float (&v)[VPL], const uint32_t (&o)[VPL / 2]) {
  const int r = cp.tok_row[n], t = cp.tok_pos[n], T = cp.row_len[r];
  const size_t f = (size_t)(n + 2 * r + 2);
  if (cp.P8) store_mx8<VPL>(v, cp.P8 + f * H, cp.P8s + f * (H / 32), c0);
  else store_packed<VPL>(cp.P + f * H + c0, o);
  if (t >= T - 2) store_packed<VPL>(cp.cache_out_base + (size_t)cp.wr[r] * cp.cache_stride + (size_t)(t - T + 2) * H + c0, o);
}

template <int VPL>
__device__ __forceinline__ void place_row(const ConvPlace& cp, int r, int H, int c0) {
  const int s = cp.row_start[r], T = cp.row_len[r];
  const bf16_t* ci = cp.cache_base + (size_t)cp.rd[r] * cp.cache_stride + c0;
  bf16_t* co = cp.cache_out_base + (size_t)cp.wr[r] * cp.cache_stride + c0;
  bf16_t* p = cp.P + (size_t)(s + 2 * r) * H + c0;
  const size_t f = (size_t)(s + 2 * r);
#pragma unroll
  for (int i = 0; i < VPL / 4; ++i) {
    uint2 a = *(const uint2*)(ci + 4 * i), b = *(const uint2*)(ci + H + 4 * i);
    if (!cp.P8) {
      *(uint2*)(p + 4 * i) = a;
      *(uint2*)(p + H + 4 * i) = b;
    }
    if (T == 1) *(uint2*)(co + 4 * i) = b;
    if (T == 0) { *(uint2*)(co + 4 * i) = a; *(uint2*)(co + H + 4 * i) = b; }
  }
  if (cp.P8) {  // the cached frames (kept bf16) enter the fp8 frame buffer quantized like the new ones
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float v[VPL];
      load_bf<VPL>(ci + (size_t)j * H, v);
      store_mx8<VPL>(v, cp.P8 + (f + j) * H, cp.P8s + (f + j) * (H / 32), c0);
    }
  }
}

template <int VPL>
__global__ void __launch_bounds__(256) ln_mod_conv_kernel(const float* h, const float* shift, const float* scale1, float eps,
                                                          ConvPlace cp, int H) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int c0 = lane * VPL;
  if (w < cp.N) {
    float v[VPL], sc[VPL], sh[VPL];
    load_f32<VPL>(h + (size_t)w * H + c0, v);
    normalize<VPL>(v, H, eps);
    load_f32<VPL>(scale1 + c0, sc);
    load_f32<VPL>(shift + c0, sh);
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = v[i] * sc[i] + sh[i];
    uint32_t o[VPL / 2];
    pack_bf<VPL>(v, o);
    place_token<VPL>(cp, w, H, c0, v, o);
  } else if (w < cp.N + cp.R) {
    place_row<VPL>(cp, w - cp.N, H, c0);
  }
}

template <int VPL>
__global__ void __launch_bounds__(256) ln_mish_conv_kernel(const bf16_t* y, const float* lw, const float* lb, float eps,
                                                           ConvPlace cp, int H) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int c0 = lane * VPL;
  if (w < cp.N) {
    float v[VPL], a[VPL], b[VPL];
    load_bf<VPL>(y + (size_t)w * H + c0, v);
    normalize<VPL>(v, H, eps);
    load_f32<VPL>(lw + c0, a);
    load_f32<VPL>(lb + c0, b);
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = mish(v[i] * a[i] + b[i]);
    uint32_t o[VPL / 2];
    pack_bf<VPL>(v, o);
    place_token<VPL>(cp, w, H, c0, v, o);
  } else if (w < cp.N + cp.R) {
    place_row<VPL>(cp, w - cp.N, H, c0);
  }
}

// Per-head affine LayerNorm of q and k (64 values per head, LPH = 64 / VPL lanes per head), q to its token row, k and
// v to the token's key slot (the reference's _qk_norm_scatter_kernel, engine/runtime/dit_kernels.py:103-142).
template <int VPL>
__global__ void __launch_bounds__(256) qk_norm_kernel(const bf16_t* qkv, const float* qw, const float* qb, const float* kw,
                                                      const float* kb, float eps, bf16_t* q_out, bf16_t* k_pool,
                                                      bf16_t* v_pool, const int* slots, int N, int H) {
  constexpr int LPH = 64 / VPL;
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int c0 = lane * VPL, d0 = c0 & 63;
  const size_t slot = (size_t)slots[n];
  const bf16_t* src = qkv + (size_t)n * 3 * H + c0;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    float v[VPL];
    load_bf<VPL>(src + which * H, v);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) s += v[i];
#pragma unroll
    for (int o = 1; o < LPH; o <<= 1) s += __shfl_xor(s, o, 64);
    const float mean = s * (1.0f / 64.0f);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      v[i] -= mean;
      q += v[i] * v[i];
    }
#pragma unroll
    for (int o = 1; o < LPH; o <<= 1) q += __shfl_xor(q, o, 64);
    const float rstd = rsqrtf(q * (1.0f / 64.0f) + eps);
    const float* w = which ? kw : qw;
    const float* b = which ? kb : qb;
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = v[i] * rstd * w[d0 + i] + b[d0 + i];
    uint32_t o[VPL / 2];
    pack_bf<VPL>(v, o);
    store_packed<VPL>(which ? k_pool + slot * H + c0 : q_out + (size_t)n * H + c0, o);
  }
  if (VPL >= 8) {
#pragma unroll
    for (int i = 0; i < VPL / 8; ++i) *(uint4*)(v_pool + slot * H + c0 + 8 * i) = *(const uint4*)(src + 2 * H + 8 * i);
  } else {
    *(uint2*)(v_pool + slot * H + c0) = *(const uint2*)(src + 2 * H);
  }
}

__global__ void pack_inputs_kernel(const float* x0, const float* stat, bf16_t* a_in, float* x, int half, int mel) {
  const int in = 4 * mel;
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2LL * half * in) return;
  const int row = (int)(i / in), c = (int)(i % in);
  const int r = row < half ? row : row - half;
  float v;
  if (c < mel) {
    v = x0[(size_t)r * mel + c];
    if (row < half) x[(size_t)r * mel + c] = v;
  } else {
    v = row < half ? stat[(size_t)r * 3 * mel + (c - mel)] : 0.0f;
  }
  a_in[i] = f2bf(v);
}

// x += dt ((1 + cfg) dphi_cond - cfg dphi_uncond); x rounded to bf16 into both CFG halves of the next in_proj input
// (engine/runtime/dit_fast.py:302).
__global__ void euler_kernel(float* x, const float* dphi, bf16_t* a_in, float* out, int half, int mel, float dt, float c1,
                             float cfg) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= half * mel) return;
  const int r = i / mel, c = i % mel;
  const float d = dphi[(size_t)r * mel + c], u = dphi[(size_t)(half + r) * mel + c];
  const float comb = __fsub_rn(__fmul_rn(c1, d), __fmul_rn(cfg, u));
  const float xv = __fadd_rn(x[i], __fmul_rn(dt, comb));
  x[i] = xv;
  const bf16_t b = f2bf(xv);
  a_in[(size_t)r * 4 * mel + c] = b;
  a_in[(size_t)(half + r) * 4 * mel + c] = b;
  if (out) out[i] = xv;
}

__global__ void temb_sinusoid_kernel(const float* ts, const float* freqs, float* out, int S, int half) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S * half) return;
  const int s = i / half, j = i % half;
  const float a = __fmul_rn(__fmul_rn(ts[s], 1000.0f), freqs[j]);
  out[(size_t)s * 2 * half + j] = cosf(a);
  out[(size_t)s * 2 * half + half + j] = sinf(a);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// out[s, o] = act(sum_k W[o, k] act_in(in[s, k]) + b[o]) for S <= 16 rows; one wave per output feature.
__global__ void __launch_bounds__(256) gemv_rows_kernel(const float* in, int ld_in, int in_act, const float* W,
                                                        const float* b, float* out, int ld_out, int S, int O, int K,
                                                        int out_act) {
  const int lane = threadIdx.x & 63;
  const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= O) return;
  float acc[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) acc[s] = 0.f;
  for (int k = lane; k < K; k += 64) {
    const float w = W[(size_t)o * K + k];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      if (s < S) {
        float x = in[(size_t)s * ld_in + k];
        if (in_act) x = silu(x);
        acc[s] += w * x;
      }
    }
  }
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    if (s < S) {
      float v = wave_sum(acc[s]) + b[o];
      if (out_act) v = silu(v);
      if (lane == 0) out[(size_t)s * ld_out + o] = v;
    }
  }
}

__global__ void add_one_kernel(float* tab, int rows, int stride, int offset, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * n) return;
  tab[(size_t)(i / n) * stride + offset + i % n] += 1.0f;
}

__global__ void copy_rows_kernel(const bf16_t* src, bf16_t* dst, const int* src_row, const int* dst_row, long long row_elems) {
  const int r = blockIdx.y;
  const bf16_t* s = src + (size_t)src_row[r] * row_elems;
  bf16_t* d = dst + (size_t)dst_row[r] * row_elems;
  for (long long i = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < row_elems; i += (long long)gridDim.x * blockDim.x * 8)
    *(uint4*)(d + i) = *(const uint4*)(s + i);
}

__global__ void convert_kernel(const float* src, bf16_t* dst, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = f2bf(src[i]);
}

inline unsigned blocks_for(long long n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

#define T2W_VPL_DISPATCH(H, CALL)          \
  switch ((H) / 64) {                      \
    case 4: { constexpr int V = 4; CALL; } break;   \
    case 8: { constexpr int V = 8; CALL; } break;   \
    case 16: { constexpr int V = 16; CALL; } break; \
    default: return hipErrorInvalidValue;  \
  }

hipError_t ln_mod(const float* h, const float* shift, const float* scale1, float eps, bf16_t* out, int N, int H, hipStream_t st) {
  if (N <= 0) return hipSuccess;
  T2W_VPL_DISPATCH(H, hipLaunchKernelGGL(ln_mod_kernel<V>, dim3(blocks_for(N, 4)), dim3(256), 0, st, h, shift, scale1, eps, out, nullptr, nullptr, N, H));
  return hipGetLastError();
}

hipError_t ln_mod_mx8(const float* h, const float* shift, const float* scale1, float eps, uint8_t* q, uint8_t* qs, int N,
                      int H, hipStream_t st) {
  if (N <= 0) return hipSuccess;
  T2W_VPL_DISPATCH(H, hipLaunchKernelGGL(ln_mod_kernel<V>, dim3(blocks_for(N, 4)), dim3(256), 0, st, h, shift, scale1, eps, nullptr, q, qs, N, H));
  return hipGetLastError();
}

hipError_t ln_mod_conv(const float* h, const float* shift, const float* scale1, float eps, const ConvPlace& cp, int H, hipStream_t st) {
  if (cp.N + cp.R <= 0) return hipSuccess;
  T2W_VPL_DISPATCH(H, hipLaunchKernelGGL(ln_mod_conv_kernel<V>, dim3(blocks_for(cp.N + cp.R, 4)), dim3(256), 0, st, h, shift, scale1, eps, cp, H));
  return hipGetLastError();
}

hipError_t ln_mish_conv(const bf16_t* y, const float* w, const float* b, float eps, const ConvPlace& cp, int H, hipStream_t st) {
  if (cp.N + cp.R <= 0) return hipSuccess;
  T2W_VPL_DISPATCH(H, hipLaunchKernelGGL(ln_mish_conv_kernel<V>, dim3(blocks_for(cp.N + cp.R, 4)), dim3(256), 0, st, y, w, b, eps, cp, H));
  return hipGetLastError();
}

hipError_t qk_norm_scatter(const bf16_t* qkv, const float* qw, const float* qb, const float* kw, const float* kb, float eps,
                           bf16_t* q_out, bf16_t* k_pool, bf16_t* v_pool, const int* slots, int N, int heads, hipStream_t st) {
  if (N <= 0) return hipSuccess;
  const int H = heads * 64;
  T2W_VPL_DISPATCH(H, hipLaunchKernelGGL(qk_norm_kernel<V>, dim3(blocks_for(N, 4)), dim3(256), 0, st, qkv, qw, qb, kw, kb, eps, q_out, k_pool, v_pool, slots, N, H));
  return hipGetLastError();
}

hipError_t pack_inputs(const float* x0, const float* stat, bf16_t* a_in, float* x, int half, int mel, hipStream_t st) {
  const long long n = 2LL * half * 4 * mel;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(pack_inputs_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x0, stat, a_in, x, half, mel);
  return hipGetLastError();
}

hipError_t euler_update(float* x, const float* dphi, bf16_t* a_in, float* out, int half, int mel, float dt, float cfg, hipStream_t st) {
  const int n = half * mel;
  if (n <= 0) return hipSuccess;
  const float c1 = (float)(1.0 + (double)cfg);
  hipLaunchKernelGGL(euler_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, x, dphi, a_in, out, half, mel, dt, c1, cfg);
  return hipGetLastError();
}

hipError_t temb_sinusoid(const float* ts, const float* freqs, float* out, int S, int half, hipStream_t st) {
  hipLaunchKernelGGL(temb_sinusoid_kernel, dim3(blocks_for((long long)S * half, 256)), dim3(256), 0, st, ts, freqs, out, S, half);
  return hipGetLastError();
}

hipError_t gemv_rows_f32(const float* in, int ld_in, int in_act, const float* W, const float* b, float* out, int ld_out, int S,
                         int O, int K, int out_act, hipStream_t st) {
  if (S > 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gemv_rows_kernel, dim3(blocks_for(O, 4)), dim3(256), 0, st, in, ld_in, in_act, W, b, out, ld_out, S, O, K, out_act);
  return hipGetLastError();
}

hipError_t add_one_cols(float* tab, int rows, int stride, int offset, int n, hipStream_t st) {
  hipLaunchKernelGGL(add_one_kernel, dim3(blocks_for((long long)rows * n, 256)), dim3(256), 0, st, tab, rows, stride, offset, n);
  return hipGetLastError();
}

hipError_t convert_rows_bf16(const float* src, bf16_t* dst, long long n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(convert_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, st, src, dst, n);
  return hipGetLastError();
}

hipError_t copy_rows_bf16(const bf16_t* src, bf16_t* dst, const int* src_row, const int* dst_row, int n_rows, long long row_elems,
                          hipStream_t st) {
  if (n_rows <= 0) return hipSuccess;
  if (row_elems % 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(copy_rows_kernel, dim3(64, n_rows), dim3(256), 0, st, src, dst, src_row, dst_row, row_elems);
  return hipGetLastError();
}

}  // namespace t2w
