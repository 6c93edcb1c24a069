// Per-token row kernels of the DiT block and the Euler/CFG update.
//
// One wave64 per token row: each lane holds H / 64 values of the row, four consecutive ones per 256 columns, so every
// access instruction covers a contiguous run of the row and the LayerNorm statistics are two wave reductions.  Norm
// statistics and modulation are fp32 (the reference's ``dit_kernels.py`` keeps norm math in fp32); outputs that feed an
// MFMA GEMM are rounded once to bf16.
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

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

// Whole-row access of the LayerNorm kernels: a lane holds groups of G consecutive values, value i at column
// (i / G) * 64 G + lane * G + i % G, so every load or store instruction of the wave covers one contiguous run of the
// row.  G = 4 suits rows read as fp32 (1 KB per instruction), G = 8 rows read as bf16 (16 bytes per lane).
template <int G>
__device__ __forceinline__ int row_col(int k, int lane) { return k * 64 * G + lane * G; }

template <int VPL, int G>
__device__ __forceinline__ void row_load_f32(const float* row, int lane, float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / G; ++k)
#pragma unroll
    for (int j = 0; j < G / 4; ++j) {
      const float4 x = *(const float4*)(row + row_col<G>(k, lane) + 4 * j);
      float* d = v + k * G + 4 * j;
      d[0] = x.x; d[1] = x.y; d[2] = x.z; d[3] = x.w;
    }
}

template <int VPL, int G>
__device__ __forceinline__ void row_store_f32(float* row, int lane, const float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / G; ++k)
#pragma unroll
    for (int j = 0; j < G / 4; ++j) {
      const float* x = v + k * G + 4 * j;
      *(float4*)(row + row_col<G>(k, lane) + 4 * j) = make_float4(x[0], x[1], x[2], x[3]);
    }
}

// fp16 rows (the residual stream), G-grouped like row_load_f32: 2 G bytes per lane and group
template <int VPL, int G>
__device__ __forceinline__ void row_load_f16(const f16_t* row, int lane, float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / G; ++k) {
    const f16_t* p = row + row_col<G>(k, lane);
    float* d = v + k * G;
    if (G == 8) {
      const uint4 x = *(const uint4*)p;
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) { d[2 * j] = lo2h(w[j]); d[2 * j + 1] = hi2h(w[j]); }
    } else {
      const uint2 x = *(const uint2*)p;
      d[0] = lo2h(x.x); d[1] = hi2h(x.x); d[2] = lo2h(x.y); d[3] = hi2h(x.y);
    }
  }
}

template <int VPL, int G>
__device__ __forceinline__ void row_store_f16(f16_t* row, int lane, const float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / G; ++k) {
    f16_t* p = row + row_col<G>(k, lane);
    const float* x = v + k * G;
    if (G == 8) *(uint4*)p = make_uint4(pack2h(x[0], x[1]), pack2h(x[2], x[3]), pack2h(x[4], x[5]), pack2h(x[6], x[7]));
    else *(uint2*)p = make_uint2(pack2h(x[0], x[1]), pack2h(x[2], x[3]));
  }
}

// The pending GEMM's value of row n (sum of its K splits in split order, then + bias), G-grouped like row_load_f32;
// all splits' loads are issued before the first add (at most 4 splits).
template <int VPL, int G>
__device__ __forceinline__ void pend_value(const Pend& pd, int n, int lane, float (&p)[VPL]) {
  float t[3][VPL], b[VPL];
  const float* r = pd.part + (size_t)n * pd.ld;
  row_load_f32<VPL, G>(r, lane, p);
#pragma unroll
  for (int s = 1; s < 4; ++s)
    if (s < pd.S) row_load_f32<VPL, G>(r + s * pd.stride, lane, t[s - 1]);
  row_load_f32<VPL, G>(pd.bias, lane, b);
#pragma unroll
  for (int s = 1; s < 4; ++s)
    if (s < pd.S) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) p[i] += t[s - 1][i];
    }
#pragma unroll
  for (int i = 0; i < VPL; ++i) p[i] += b[i];
}

// h row n (in v) += gate * pending value, rounded to fp16 and stored back to h (the gated residual epilogue of the
// GEMM, in its order); v keeps the rounded values the next norm reads
template <int VPL, int G>
__device__ __forceinline__ void pend_resid(const Pend& pd, f16_t* hrow, int n, int lane, float (&v)[VPL]) {
  float p[VPL], gt[VPL];
  pend_value<VPL, G>(pd, n, lane, p);
  row_load_f32<VPL, G>(pd.gate, lane, gt);
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] = h2f(f2h(v[i] + gt[i] * p[i]));
  row_store_f16<VPL, G>(hrow, lane, v);
}

// raw bf16 words of a row (G / 2 per group)
template <int VPL, int G>
__device__ __forceinline__ void row_load_words(const bf16_t* row, int lane, uint32_t (&w)[VPL / 2]) {
#pragma unroll
  for (int k = 0; k < VPL / G; ++k) {
    const bf16_t* p = row + row_col<G>(k, lane);
    if (G == 8) {
      const uint4 x = *(const uint4*)p;
      w[4 * k] = x.x; w[4 * k + 1] = x.y; w[4 * k + 2] = x.z; w[4 * k + 3] = x.w;
    } else {
      const uint2 x = *(const uint2*)p;
      w[2 * k] = x.x; w[2 * k + 1] = x.y;
    }
  }
}

template <int VPL>
__device__ __forceinline__ void words_to_f32(const uint32_t (&w)[VPL / 2], float (&v)[VPL]) {
#pragma unroll
  for (int j = 0; j < VPL / 2; ++j) { v[2 * j] = lo2f(w[j]); v[2 * j + 1] = hi2f(w[j]); }
}

template <int VPL, int G>
__device__ __forceinline__ void row_store_bf(bf16_t* row, int lane, const uint32_t (&o)[VPL / 2]) {
#pragma unroll
  for (int k = 0; k < VPL / G; ++k) {
    bf16_t* p = row + row_col<G>(k, lane);
    if (G == 8) *(uint4*)p = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
    else *(uint2*)p = make_uint2(o[2 * k], o[2 * k + 1]);
  }
}

// MX fp8 store of a whole row: a 32-value block is 32 / G consecutive lanes' groups; its maximum is reduced over them
// and the block's first lane writes the E8M0 scale byte
template <int VPL, int G>
__device__ __forceinline__ void row_store_mx8(const float (&v)[VPL], uint8_t* qrow, uint8_t* srow, int lane) {
#pragma unroll
  for (int k = 0; k < VPL / G; ++k) {
    const float* x = v + k * G;
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) a = fmaxf(a, fabsf(x[j]));
    a = 32 / G == 4 ? quad_max(a) : max8(a);  // the block's 32 / G lanes (DPP, no LDS)
    const int se = mx_exp(a);
    const int c = row_col<G>(k, lane);
    const uint32_t w0 = mx_pack4(x[0], x[1], x[2], x[3], se);
    if (G == 8) *(uint2*)(qrow + c) = make_uint2(w0, mx_pack4(x[4], x[5], x[6], x[7], se));
    else *(uint32_t*)(qrow + c) = w0;
    if ((lane & (32 / G - 1)) == 0) srow[c >> 5] = (uint8_t)(se + 127);
  }
}

// Workgroup `b` of a row kernel's prefetch workgroups: reads its PF_UNITS 16-byte units of the two ranges (taken as
// one sequence; PF_UNITS / blockDim per thread) and discards them (an empty asm keeps the loads)
constexpr int PF_UNITS = 1024;
__device__ __forceinline__ void prefetch_part(const Prefetch& pf, unsigned b) {
  const long n0 = (long)(pf.bytes[0] / 16), n1 = (long)(pf.bytes[1] / 16);
  long i = (long)b * PF_UNITS + threadIdx.x;
  uint32_t acc = 0;
  const int per = PF_UNITS / blockDim.x;
  for (int u = 0; u < per; ++u, i += blockDim.x) {
    if (i < n0) {
      const uint4 v = ((const uint4*)pf.p[0])[i];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    } else if (i < n0 + n1) {
      const uint4 v = ((const uint4*)pf.p[1])[i - n0];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  asm volatile("" ::"v"(acc));
}

// LayerNorm statistics over a row spread across the wave: v -> (v - mean) * rstd (the two sums through DPP rows and
// lane reads: no LDS round trips on the row's latency chain)
template <int VPL>
__device__ __forceinline__ void normalize(float (&v)[VPL], int H, float eps) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) s += v[i];
  const float mean = wave_sum_rows(s) / (float)H;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    v[i] -= mean;
    q += v[i] * v[i];
  }
  const float rstd = rsqrtf(wave_sum_rows(q) / (float)H + eps);
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] *= rstd;
}

// out: bf16 [N, H]; or, with q non-null, MX fp8 codes q [N, H] and block scales qs [N, H / 32]
// PEND: a pending GEMM result is finished first (a separate instantiation, so that the large calls, which never defer,
// keep the registers and occupancy of the plain kernel)
template <int VPL, bool PEND>
__global__ void __launch_bounds__(256) ln_mod_kernel(f16_t* h, const float* shift, const float* scale1, float eps,
                                                     bf16_t* out, uint8_t* q, uint8_t* qs, int N, int H, Pend pd, Prefetch pf,
                                                     unsigned row_blocks) {
  constexpr int G = VPL >= 8 ? 8 : 4;  // fp16 rows: 16 bytes per lane and instruction
  // the prefetch workgroups come first, so the weight reads start with the rows' instead of trailing them (16 x 400
  // solve 98.5 -> 98.0 ms, same bits); the row blocks follow
  const unsigned pfb = gridDim.x - row_blocks;
  if (blockIdx.x < pfb) {
    prefetch_part(pf, blockIdx.x);
    return;
  }
  const unsigned rblk = blockIdx.x - pfb;
  const int lane = threadIdx.x & 63;
  const int n = rblk * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (n >= N) return;
  float v[VPL], sc[VPL], sh[VPL];
  // the modulation (the same for every row, cache hits) is loaded with the row, not after its statistics
  row_load_f32<VPL, G>(scale1, lane, sc);
  row_load_f32<VPL, G>(shift, lane, sh);
  row_load_f16<VPL, G>(h + (size_t)n * H, lane, v);
  if (PEND) pend_resid<VPL, G>(pd, h + (size_t)n * H, n, lane, v);
  normalize<VPL>(v, H, eps);
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] = v[i] * sc[i] + sh[i];
  if (q) {
    row_store_mx8<VPL, G>(v, q + (size_t)n * H, qs + (size_t)n * (H / 32), lane);
    return;
  }
  uint32_t o[VPL / 2];
  pack_bf<VPL>(v, o);
  row_store_bf<VPL, G>(out + (size_t)n * H, lane, o);
}

// Frame f of token n (position t of row r, T frames) in the padded buffer is n + 2 r + 2; it is also the row's new
// cache frame t - T + 2 when t >= T - 2.  Row programs copy the two cached frames in front of the row's frames and,
// for rows of fewer than two tokens, produce the new cache from the old one (the reference's _conv_place and
// _conv_row_cache, engine/runtime/dit_kernels.py:217-248).
// where token n's frame goes: its row r, position t, the row's length T and cache slot wr (loaded before the token's
// row, so that this chain of index loads is not on the path after its statistics)
struct TokPlace {
  int r, t, T, wr;
};
__device__ __forceinline__ TokPlace tok_place(const ConvPlace& cp, int n) {
  TokPlace p;
  p.r = cp.tok_row[n];
  p.t = cp.tok_pos[n];
  p.T = cp.row_len[p.r];
  p.wr = cp.wr[p.r];
  return p;
}

template <int VPL, int G>
__device__ __forceinline__ void place_token(const ConvPlace& cp, const TokPlace& tp, int n, int H, int lane, const float (&v)[VPL],
                                            const uint32_t (&o)[VPL / 2]) {
  const size_t f = (size_t)(n + 2 * tp.r + 2);
  if (cp.P8) row_store_mx8<VPL, G>(v, cp.P8 + f * H, cp.P8s + f * (H / 32), lane);
  else row_store_bf<VPL, G>(cp.P + f * H, lane, o);
  if (tp.t >= tp.T - 2) row_store_bf<VPL, G>(cp.cache_out_base + (size_t)tp.wr * cp.cache_stride + (size_t)(tp.t - tp.T + 2) * H, lane, o);
}

// both cached frames are loaded before the first store (the frame buffer and the caches are distinct memory)
template <int VPL, int G>
__device__ __forceinline__ void place_row(const ConvPlace& cp, int r, int H, int lane) {
  const int s = cp.row_start[r], T = cp.row_len[r];
  const bf16_t* ci = cp.cache_base + (size_t)cp.rd[r] * cp.cache_stride;
  bf16_t* co = cp.cache_out_base + (size_t)cp.wr[r] * cp.cache_stride;
  const size_t f = (size_t)(s + 2 * r);
  uint32_t a[VPL / 2], b[VPL / 2];
  row_load_words<VPL, G>(ci, lane, a);
  row_load_words<VPL, G>(ci + H, lane, b);
  if (cp.P8) {  // the cached frames (kept bf16) enter the fp8 frame buffer quantized like the new ones
    float v[VPL];
    words_to_f32<VPL>(a, v);
    row_store_mx8<VPL, G>(v, cp.P8 + f * H, cp.P8s + f * (H / 32), lane);
    words_to_f32<VPL>(b, v);
    row_store_mx8<VPL, G>(v, cp.P8 + (f + 1) * H, cp.P8s + (f + 1) * (H / 32), lane);
  } else {
    row_store_bf<VPL, G>(cp.P + f * H, lane, a);
    row_store_bf<VPL, G>(cp.P + (f + 1) * H, lane, b);
  }
  if (T == 1) row_store_bf<VPL, G>(co, lane, b);
  if (T == 0) {
    row_store_bf<VPL, G>(co, lane, a);
    row_store_bf<VPL, G>(co + H, lane, b);
  }
}

template <int VPL, bool PEND>
__global__ void __launch_bounds__(256) ln_mod_conv_kernel(f16_t* h, const float* shift, const float* scale1, float eps,
                                                          ConvPlace cp, int H, Pend pd, Prefetch pf, unsigned row_blocks) {
  constexpr int G = VPL >= 8 ? 8 : 4;
  const unsigned pfb = gridDim.x - row_blocks;
  if (blockIdx.x < pfb) {
    prefetch_part(pf, blockIdx.x);
    return;
  }
  const unsigned rblk = blockIdx.x - pfb;
  const int lane = threadIdx.x & 63;
  const int w = rblk * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w < cp.N) {
    float v[VPL], sc[VPL], sh[VPL];
    const TokPlace tp = tok_place(cp, w);
    row_load_f32<VPL, G>(scale1, lane, sc);
    row_load_f32<VPL, G>(shift, lane, sh);
    row_load_f16<VPL, G>(h + (size_t)w * H, lane, v);
    if (PEND) pend_resid<VPL, G>(pd, h + (size_t)w * H, w, lane, v);
    normalize<VPL>(v, H, eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = v[i] * sc[i] + sh[i];
    uint32_t o[VPL / 2];
    pack_bf<VPL>(v, o);
    place_token<VPL, G>(cp, tp, w, H, lane, v, o);
  } else if (w < cp.N + cp.R) {
    place_row<VPL, G>(cp, w - cp.N, H, lane);
  }
}

template <int VPL, bool PEND>
__global__ void __launch_bounds__(256) ln_mish_conv_kernel(const bf16_t* y, const float* lw, const float* lb, float eps,
                                                           ConvPlace cp, int H, Pend pd, Prefetch pf, unsigned row_blocks) {
  const unsigned pfb = gridDim.x - row_blocks;
  if (blockIdx.x < pfb) {
    prefetch_part(pf, blockIdx.x);
    return;
  }
  const unsigned rblk = blockIdx.x - pfb;
  const int lane = threadIdx.x & 63;
  const int w = rblk * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (w < cp.N) {
    constexpr int G = VPL >= 8 ? 8 : 4;  // the row comes in as bf16
    float v[VPL], a[VPL], b[VPL];
    const TokPlace tp = tok_place(cp, w);
    row_load_f32<VPL, G>(lw, lane, a);
    row_load_f32<VPL, G>(lb, lane, b);
    if (PEND) {  // the pending conv GEMM's value, rounded to bf16 as its own epilogue would
      pend_value<VPL, G>(pd, w, lane, v);
#pragma unroll
      for (int i = 0; i < VPL; ++i) v[i] = bf2f(f2bf(v[i]));
    } else {
      uint32_t wv[VPL / 2];
      row_load_words<VPL, G>(y + (size_t)w * H, lane, wv);
      words_to_f32<VPL>(wv, v);
    }
    normalize<VPL>(v, H, eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = mish(v[i] * a[i] + b[i]);
    uint32_t o[VPL / 2];
    pack_bf<VPL>(v, o);
    place_token<VPL, G>(cp, tp, w, H, lane, v, o);
  } else if (w < cp.N + cp.R) {
    place_row<VPL, VPL >= 8 ? 8 : 4>(cp, w - cp.N, H, lane);
  }
}

// Per-head affine LayerNorm of q and k (64 values per head, LPH = 64 / VPL lanes per head), q to its token row, k and
// v to the token's key slot (the reference's _qk_norm_scatter_kernel, engine/runtime/dit_kernels.py:103-142).  With
// rfreq, q and k are then rotated at the token's stream position pos[n] (rotary embedding, no reference counterpart).
template <int VPL>
__global__ void __launch_bounds__(256) qk_norm_kernel(const bf16_t* qkv, const float* qw, const float* qb, const float* kw,
                                                      const float* kb, float eps, bf16_t* q_out, bf16_t* k_pool,
                                                      bf16_t* v_pool, const int* slots, int N, int H, const float* rfreq,
                                                      const int* pos) {
  constexpr int LPH = 64 / VPL;
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (n >= N) return;
  const int c0 = lane * VPL, d0 = c0 & 63;
  const size_t slot = (size_t)slots[n];
  const int tpos = rfreq ? pos[n] : 0;
  const bf16_t* src = qkv + (size_t)n * 3 * H + c0;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    float v[VPL];
    load_bf<VPL>(src + which * H, v);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) s += v[i];
    s = group_sum<LPH>(s);
    const float mean = s * (1.0f / 64.0f);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      v[i] -= mean;
      q += v[i] * v[i];
    }
    q = group_sum<LPH>(q);
    const float rstd = rsqrtf(q * (1.0f / 64.0f) + eps);
    const float* w = which ? kw : qw;
    const float* b = which ? kb : qb;
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = v[i] * rstd * w[d0 + i] + b[d0 + i];
    if (rfreq) rope_rotate<VPL>(v, tpos, rfreq + (d0 >> 1));
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

// Rotary embedding after the tile GEMM's q / k epilogue: 8 values (4 channel pairs) of one q row or one key slot per
// thread, q rows first; the token's stream position pos[n]
__global__ void __launch_bounds__(256) rope_qk_kernel(bf16_t* q, bf16_t* k_pool, const int* slots, const int* pos,
                                                      const float* rfreq, int N, int H) {
  const long long per = H / 8, t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 2 * (long long)N * per) return;
  const int which = t >= (long long)N * per ? 1 : 0;
  const long long r = t - (long long)which * N * per;
  const int n = (int)(r / per), c = (int)(r - (long long)n * per) * 8;
  bf16_t* p = which ? k_pool + (size_t)slots[n] * H + c : q + (size_t)n * H + c;
  const uint4 u = *(const uint4*)p;
  float y[8] = {lo2f(u.x), hi2f(u.x), lo2f(u.y), hi2f(u.y), lo2f(u.z), hi2f(u.z), lo2f(u.w), hi2f(u.w)};
  rope_rotate<8>(y, pos[n], rfreq + ((c & 63) >> 1));
  *(uint4*)p = make_uint4(pack2(y[0], y[1]), pack2(y[2], y[3]), pack2(y[4], y[5]), pack2(y[6], y[7]));
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

// Rows per block of the row kernels: calls of few rows (a streaming chunk) spread one row per CU, since a CU's load
// throughput bounds them (a LayerNorm row with pending K-split sums reads ~20 KB); large calls take four rows per block.
inline int row_waves(long long rows) { return rows <= 1024 ? 1 : 4; }

#define T2W_VPL_DISPATCH(H, CALL)          \
  switch ((H) / 64) {                      \
    case 4: { constexpr int V = 4; CALL; } break;   \
    case 8: { constexpr int V = 8; CALL; } break;   \
    case 16: { constexpr int V = 16; CALL; } break; \
    default: return hipErrorInvalidValue;  \
  }

// workgroups that read a prefetch's ranges, PF_UNITS 16-byte units each (none without ranges or when unaligned)
inline unsigned prefetch_blocks(const Prefetch& pf) {
  if ((pf.bytes[0] && ((size_t)pf.p[0] & 15)) || (pf.bytes[1] && ((size_t)pf.p[1] & 15))) return 0;
  const size_t units = pf.bytes[0] / 16 + pf.bytes[1] / 16;
  return (unsigned)((units + PF_UNITS - 1) / PF_UNITS);
}

hipError_t ln_mod(f16_t* h, const float* shift, const float* scale1, float eps, bf16_t* out, int N, int H, hipStream_t st,
                  const Pend& pd, const Prefetch& pf) {
  if (N <= 0) return hipSuccess;
  if (pd.part && (pd.S < 1 || pd.S > 4)) return hipErrorInvalidValue;
  const int w = row_waves(N);
  const unsigned rb = blocks_for(N, w);
  if (pd.part) {
    T2W_VPL_DISPATCH(H, hipLaunchKernelGGL((ln_mod_kernel<V, true>), dim3(rb + prefetch_blocks(pf)), dim3(64 * w), 0, st, h, shift, scale1, eps, out, nullptr, nullptr, N, H, pd, pf, rb));
  } else {
    T2W_VPL_DISPATCH(H, hipLaunchKernelGGL((ln_mod_kernel<V, false>), dim3(rb + prefetch_blocks(pf)), dim3(64 * w), 0, st, h, shift, scale1, eps, out, nullptr, nullptr, N, H, pd, pf, rb));
  }
  return hipGetLastError();
}

hipError_t ln_mod_mx8(const f16_t* h, const float* shift, const float* scale1, float eps, uint8_t* q, uint8_t* qs, int N,
                      int H, hipStream_t st, const Prefetch& pf) {
  if (N <= 0) return hipSuccess;
  // nothing pending: h is only read
  const int w = row_waves(N);
  const unsigned rb = blocks_for(N, w);
  T2W_VPL_DISPATCH(H, hipLaunchKernelGGL((ln_mod_kernel<V, false>), dim3(rb + prefetch_blocks(pf)), dim3(64 * w), 0, st, const_cast<f16_t*>(h), shift, scale1, eps, nullptr, q, qs, N, H, Pend(), pf, rb));
  return hipGetLastError();
}

hipError_t ln_mod_conv(f16_t* h, const float* shift, const float* scale1, float eps, const ConvPlace& cp, int H, hipStream_t st,
                       const Pend& pd, const Prefetch& pf) {
  if (cp.N + cp.R <= 0) return hipSuccess;
  if (pd.part && (pd.S < 1 || pd.S > 4)) return hipErrorInvalidValue;
  const int w = row_waves(cp.N + cp.R);
  const unsigned rb = blocks_for(cp.N + cp.R, w);
  if (pd.part) {
    T2W_VPL_DISPATCH(H, hipLaunchKernelGGL((ln_mod_conv_kernel<V, true>), dim3(rb + prefetch_blocks(pf)), dim3(64 * w), 0, st, h, shift, scale1, eps, cp, H, pd, pf, rb));
  } else {
    T2W_VPL_DISPATCH(H, hipLaunchKernelGGL((ln_mod_conv_kernel<V, false>), dim3(rb + prefetch_blocks(pf)), dim3(64 * w), 0, st, h, shift, scale1, eps, cp, H, pd, pf, rb));
  }
  return hipGetLastError();
}

hipError_t ln_mish_conv(const bf16_t* y, const float* w, const float* b, float eps, const ConvPlace& cp, int H, hipStream_t st,
                        const Pend& pd, const Prefetch& pf) {
  if (cp.N + cp.R <= 0) return hipSuccess;
  if (pd.part && (pd.S < 1 || pd.S > 4)) return hipErrorInvalidValue;
  const int wv = row_waves(cp.N + cp.R);
  const unsigned rb = blocks_for(cp.N + cp.R, wv);
  if (pd.part) {
    T2W_VPL_DISPATCH(H, hipLaunchKernelGGL((ln_mish_conv_kernel<V, true>), dim3(rb + prefetch_blocks(pf)), dim3(64 * wv), 0, st, y, w, b, eps, cp, H, pd, pf, rb));
  } else {
    T2W_VPL_DISPATCH(H, hipLaunchKernelGGL((ln_mish_conv_kernel<V, false>), dim3(rb + prefetch_blocks(pf)), dim3(64 * wv), 0, st, y, w, b, eps, cp, H, pd, pf, rb));
  }
  return hipGetLastError();
}

hipError_t qk_norm_scatter(const bf16_t* qkv, const float* qw, const float* qb, const float* kw, const float* kb, float eps,
                           bf16_t* q_out, bf16_t* k_pool, bf16_t* v_pool, const int* slots, int N, int heads, hipStream_t st,
                           const float* rfreq, const int* pos) {
  if (N <= 0) return hipSuccess;
  const int H = heads * 64;
  T2W_VPL_DISPATCH(H, hipLaunchKernelGGL(qk_norm_kernel<V>, dim3(blocks_for(N, row_waves(N))), dim3(64 * row_waves(N)), 0, st, qkv, qw, qb, kw, kb, eps, q_out, k_pool, v_pool, slots, N, H, rfreq, pos));
  return hipGetLastError();
}

hipError_t rope_qk(bf16_t* q, bf16_t* k_pool, const int* slots, const int* pos, const float* rfreq, int N, int H, hipStream_t st) {
  if (N <= 0) return hipSuccess;
  if (H % 64 || !pos || !rfreq) return hipErrorInvalidValue;
  const long long threads = 2LL * N * (H / 8);
  hipLaunchKernelGGL(rope_qk_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, q, k_pool, slots, pos, rfreq, N, H);
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
