// Flow encoder kernels (codec tokens -> mu) of the CosyVoice2-style upsampling conformer encoder
// (engine/runtime/token2wav_batch.py:42-79, 402-444; the modules themselves live in stepaudio2).
//
// Row kernels hold one token row per wave64: a lane owns groups of 8 consecutive values (column (i / 8) * 512 +
// lane * 8 + i % 8), so each access instruction of the wave covers 1 KB of bf16 / fp16 or 2 KB of fp32, and LayerNorm
// statistics are two wave reductions in fp32.
//
// The attention is the ESPnet relative-position form with per-head biases u, v:
//   score(i, j) = ((q_i + u) . k_j + (q_i + v) . P[(L - T + i) - j]) / sqrt(64)
// over a stream's L keys (cached frames, then its T new ones) for its T queries, where P[r] = linear_pos(sinusoid(r))
// does not depend on the stream: it is tabulated once per layer (fp16), and the reference's [T, 2L - 1] positional
// scores and their rel_shift become, per tile of 32 queries x 32 keys, one 32 x 64 MFMA product over the 63 relative
// positions the tile spans, read back skewed from LDS.
#include "flow_internal.h"

namespace t2w {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ half8 as_half8(uint4 v) {
  union { uint4 u; half8 h; } c;
  c.u = v;
  return c.h;
}

constexpr float NEG = -1.0e30f;

template <int VPL>
__device__ __forceinline__ void load_f32(const float* row, int lane, float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / 8; ++k) {
    const float4 a = *(const float4*)(row + k * 512 + lane * 8), b = *(const float4*)(row + k * 512 + lane * 8 + 4);
    float* d = v + 8 * k;
    d[0] = a.x; d[1] = a.y; d[2] = a.z; d[3] = a.w; d[4] = b.x; d[5] = b.y; d[6] = b.z; d[7] = b.w;
  }
}

template <int VPL>
__device__ __forceinline__ void load_f16(const f16_t* row, int lane, float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / 8; ++k) {
    const uint4 x = *(const uint4*)(row + k * 512 + lane * 8);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[8 * k + 2 * j] = lo2h(w[j]); v[8 * k + 2 * j + 1] = hi2h(w[j]); }
  }
}

template <int VPL>
__device__ __forceinline__ void store_bf16(bf16_t* row, int lane, const float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / 8; ++k) {
    const float* s = v + 8 * k;
    *(uint4*)(row + k * 512 + lane * 8) = make_uint4(pack2(s[0], s[1]), pack2(s[2], s[3]), pack2(s[4], s[5]), pack2(s[6], s[7]));
  }
}

template <int VPL>
__device__ __forceinline__ void store_f16(f16_t* row, int lane, const float (&v)[VPL]) {
#pragma unroll
  for (int k = 0; k < VPL / 8; ++k) {
    const float* s = v + 8 * k;
    *(uint4*)(row + k * 512 + lane * 8) = make_uint4(pack2h(s[0], s[1]), pack2h(s[2], s[3]), pack2h(s[4], s[5]), pack2h(s[6], s[7]));
  }
}

// LayerNorm (biased variance, fp32) with affine w, b, then times `scale`
template <int VPL>
__device__ __forceinline__ void layer_norm(float (&v)[VPL], const float* w, const float* b, float eps, float scale, int C, int lane) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) s += v[i];
  const float mean = wave_sum(s) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const float d = v[i] - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)C + eps);
#pragma unroll
  for (int k = 0; k < VPL / 8; ++k) {
    const int c0 = k * 512 + lane * 8;
    const float4 w0 = *(const float4*)(w + c0), w1 = *(const float4*)(w + c0 + 4);
    const float4 b0 = *(const float4*)(b + c0), b1 = *(const float4*)(b + c0 + 4);
    const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[8 * k + j] = ((v[8 * k + j] - mean) * rstd * ww[j] + bb[j]) * scale;
  }
}

template <int VPL>
__global__ void __launch_bounds__(256) flow_embed_kernel(const float* table, const int* tok, const int* res, const float* w,
                                                         const float* b, float eps, float xscale, bf16_t* x0, f16_t* h, int n, int C) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const int t = tok[row];
  float v[VPL];
  if (t < 0) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = 0.f;
  } else {
    load_f32<VPL>(table + (size_t)t * C, lane, v);
    layer_norm<VPL>(v, w, b, eps, xscale, C, lane);
  }
  store_bf16<VPL>(x0 + (size_t)row * C, lane, v);
  const int r = res[row];
  if (r >= 0) store_f16<VPL>(h + (size_t)r * C, lane, v);
}

__global__ void __launch_bounds__(64) flow_look_place_kernel(bf16_t* G, bf16_t* cache, const int* g, const int* t1, const int* rd,
                                                             const int* wr, int C, long long cstride) {
  const int s = blockIdx.x, lane = threadIdx.x;
  const int g0 = g[s], T = t1[s];
  const bf16_t* src = cache + (size_t)rd[s] * cstride;
  bf16_t* dst = cache + (size_t)wr[s] * cstride;
  for (int c = lane * 8; c < C; c += 512) {
#pragma unroll
    for (int f = 0; f < 2; ++f) *(uint4*)(G + (size_t)(g0 + f) * C + c) = *(const uint4*)(src + f * C + c);
#pragma unroll
    for (int f = 0; f < 2; ++f) {  // frame q of [cache | conv1 outputs]
      const int q = T + f;
      const bf16_t* p = q < 2 ? src + q * C : G + (size_t)(g0 + q) * C;
      *(uint4*)(dst + f * C + c) = *(const uint4*)(p + c);
    }
  }
}

__device__ __forceinline__ uint4 f16x8_to_bf16x8(uint4 x) {
  return make_uint4(pack2(lo2h(x.x), hi2h(x.x)), pack2(lo2h(x.y), hi2h(x.y)), pack2(lo2h(x.z), hi2h(x.z)), pack2(lo2h(x.w), hi2h(x.w)));
}

__global__ void __launch_bounds__(256) flow_up_place_kernel(const f16_t* h, bf16_t* U, const int* up_dst, int n1, int nbr, const int* u,
                                                            const int* o1, const int* t1, bf16_t* cache, const int* rd, const int* wr,
                                                            int C, long long cstride) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if ((int)blockIdx.x < nbr) {
    const int m = blockIdx.x * 4 + wave;
    if (m >= n1) return;
    bf16_t* d0 = U + (size_t)up_dst[m] * C;
    for (int c = lane * 8; c < C; c += 512) {
      const uint4 v = f16x8_to_bf16x8(*(const uint4*)(h + (size_t)m * C + c));
      *(uint4*)(d0 + c) = v;
      *(uint4*)(d0 + C + c) = v;
    }
    return;
  }
  const int s = blockIdx.x - nbr, f = wave;  // four waves: the stream's four cached frames
  const bf16_t* src = cache + (size_t)rd[s] * cstride + 2 * C;
  bf16_t* dst = cache + (size_t)wr[s] * cstride + 2 * C;
  const int q = 2 * t1[s] + f;  // frame q of [cache (4) | upsampled frames]
  for (int c = lane * 8; c < C; c += 512) {
    *(uint4*)(U + (size_t)(u[s] + f) * C + c) = *(const uint4*)(src + f * C + c);
    uint4 v;
    if (q < 4) v = *(const uint4*)(src + q * C + c);
    else v = f16x8_to_bf16x8(*(const uint4*)(h + (size_t)(o1[s] + (q - 4) / 2) * C + c));
    *(uint4*)(dst + f * C + c) = v;
  }
}

template <int VPL>
__global__ void __launch_bounds__(256) flow_ln_scale_ln_kernel(const float* y, const float* w1, const float* b1, float eps1, float xscale,
                                                               f16_t* h, const float* w2, const float* b2, float eps2, bf16_t* a, int n, int C) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  float v[VPL];
  load_f32<VPL>(y + (size_t)row * C, lane, v);
  layer_norm<VPL>(v, w1, b1, eps1, xscale, C, lane);
#pragma unroll
  for (int i = 0; i < VPL; ++i) v[i] = h2f(f2h(v[i]));  // the stored residual value
  store_f16<VPL>(h + (size_t)row * C, lane, v);
  layer_norm<VPL>(v, w2, b2, eps2, 1.0f, C, lane);
  store_bf16<VPL>(a + (size_t)row * C, lane, v);
}

__global__ void __launch_bounds__(256) flow_kv_store_kernel(const f16_t* qkv, int ldq, f16_t* pool, const int* slot, int n, int C) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const f16_t* src = qkv + (size_t)row * ldq + C;
  f16_t* dst = pool + (size_t)slot[row] * 2 * C;
  for (int c = lane * 8; c < 2 * C; c += 512) *(uint4*)(dst + c) = *(const uint4*)(src + c);
}

// One wave per (32-query tile, head).  MFMA v_mfma_f32_32x32x16_f16 with the scores transposed, S^T = K . Q^T, so a
// lane holds 16 keys of its own query (column lane % 32; key rows (r / 4) * 8 + (lane / 32) * 4 + r % 4 of register r)
// and its partner lane (lane ^ 32) the other 16; O^T += V^T . P^T keeps the output in the same per-query lanes.
// Positional scores: G^T = Pband . Qv^T over the 64 table rows rb .. rb + 63, rb = L - T + i0 - j0 - 31, the 63
// relative positions (i - j) + 31 of the tile pair; (key jj, query ii) takes G^T[ii - jj + 31][ii].
__global__ void __launch_bounds__(64) flow_rel_attn_kernel(RelAttnArgs a) {
  constexpr int GS = 40;                 // row stride of G^T in LDS: conflict-free for the writes and the skewed reads
  __shared__ float gsh[64 * GS];
  __shared__ uint4 vsh[32 * 9];          // V tile: 32 key rows of 64 fp16 (8 chunks), row stride 9 chunks
  const int tile = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
  const int s = a.tiles[2 * tile], i0 = a.tiles[2 * tile + 1];
  const int T = a.row_len[s], L = a.kv_len[s], start = a.row_start[s];
  const int* kv = a.kv_idx + a.kv_off[s];
  const int C = a.heads * 64, C2 = 2 * C;
  const int col = lane & 31, half = lane >> 5;
  const int qi = i0 + col, qc = qi < T ? qi : T - 1;

  half8 qu[4], qv[4];
  {
    const f16_t* qp = a.qkv + (size_t)(start + qc) * a.ldq + head * 64 + half * 8;
    const float* bu = a.bias_u + head * 64 + half * 8;
    const float* bv = a.bias_v + head * 64 + half * 8;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const half8 q = as_half8(*(const uint4*)(qp + kk * 16));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (float)q[e];
        qu[kk][e] = (_Float16)(x + bu[kk * 16 + e]);
        qv[kk][e] = (_Float16)(x + bv[kk * 16 + e]);
      }
    }
  }
  f32x16 o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) { o0[r] = 0.f; o1[r] = 0.f; }
  float m = NEG, l = 0.f;
  const float sl2 = a.scale * 1.4426950408889634f;
  const int zero_row = a.rmax - 1, last_row = 2 * a.rmax - 2;

  for (int j0 = 0; j0 < L; j0 += 32) {
    // keys (A operand rows): key j0 + col
    half8 kf[4];
    {
      const int kj = j0 + col < L ? j0 + col : L - 1;
      const f16_t* kp = a.pool + (size_t)kv[kj] * C2 + head * 64 + half * 8;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) kf[kk] = as_half8(*(const uint4*)(kp + kk * 16));
    }
    // values: key j0 + lane / 2, chunks (lane & 1) * 4 .. + 3, into LDS
    {
      const int vk = j0 + (lane >> 1) < L ? j0 + (lane >> 1) : L - 1;
      const uint4* vp = (const uint4*)(a.pool + (size_t)kv[vk] * C2 + C + head * 64) + (lane & 1) * 4;
      uint4* dst = vsh + (lane >> 1) * 9 + (lane & 1) * 4;
      const uint4 v0 = vp[0], v1 = vp[1], v2 = vp[2], v3 = vp[3];
      dst[0] = v0; dst[1] = v1; dst[2] = v2; dst[3] = v3;
    }
    // positional rows (A operand rows): relative positions rb + col and rb + 32 + col
    half8 pf0[4], pf1[4];
    {
      const int rb = L - T + i0 - j0 - 31 + zero_row;
      const int p0 = min(max(rb + col, 0), last_row), p1 = min(max(rb + 32 + col, 0), last_row);
      const f16_t* pp0 = a.ptab + (size_t)p0 * C + head * 64 + half * 8;
      const f16_t* pp1 = a.ptab + (size_t)p1 * C + head * 64 + half * 8;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        pf0[kk] = as_half8(*(const uint4*)(pp0 + kk * 16));
        pf1[kk] = as_half8(*(const uint4*)(pp1 + kk * 16));
      }
    }
    f32x16 sacc, g0, g1;
#pragma unroll
    for (int r = 0; r < 16; ++r) { sacc[r] = 0.f; g0[r] = 0.f; g1[r] = 0.f; }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[kk], qu[kk], sacc, 0, 0, 0);
      g0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(pf0[kk], qv[kk], g0, 0, 0, 0);
      g1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(pf1[kk], qv[kk], g1, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int pr = (r >> 2) * 8 + half * 4 + (r & 3);
      gsh[pr * GS + col] = g0[r];
      gsh[(pr + 32) * GS + col] = g1[r];
    }
    __syncthreads();
    float sv[16];
    float mx = NEG;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jj = (r >> 2) * 8 + half * 4 + (r & 3);
      float x = (sacc[r] + gsh[(col - jj + 31) * GS + col]) * sl2;
      if (j0 + jj >= L) x = NEG;
      sv[r] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, xor32(mx));
    const float mn = fmaxf(m, mx), corr = __builtin_amdgcn_exp2f(m - mn);
    float ls = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sv[r] = __builtin_amdgcn_exp2f(sv[r] - mn);
      ls += sv[r];
    }
    ls += xor32(ls);
    l = l * corr + ls;
    m = mn;
#pragma unroll
    for (int r = 0; r < 16; ++r) { o0[r] *= corr; o1[r] *= corr; }
    // O^T += V^T . P^T over two 16-key slices: K index half * 8 + e of slice kk2 is key kk2 * 16 + (e / 4) * 8 +
    // half * 4 + e % 4, which is where this lane's probability sv[kk2 * 8 + e] sits
#pragma unroll
    for (int kk2 = 0; kk2 < 2; ++kk2) {
      half8 pb, va, vb;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pb[e] = (_Float16)sv[kk2 * 8 + e];
        const int key = kk2 * 16 + (e >> 2) * 8 + half * 4 + (e & 3);
        const _Float16* vr = (const _Float16*)(vsh + key * 9);
        va[e] = vr[col];
        vb[e] = vr[32 + col];
      }
      o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(vb, pb, o1, 0, 0, 0);
    }
    __syncthreads();  // LDS reads done before the next tile's writes
  }
  if (qi < T) {
    const float inv = 1.0f / l;
    bf16_t* op = a.out + (size_t)(start + qi) * C + head * 64 + half * 4;
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      const int r = grp * 4;
      *(uint2*)(op + grp * 8) = make_uint2(pack2(o0[r] * inv, o0[r + 1] * inv), pack2(o0[r + 2] * inv, o0[r + 3] * inv));
      *(uint2*)(op + 32 + grp * 8) = make_uint2(pack2(o1[r] * inv, o1[r + 1] * inv), pack2(o1[r + 2] * inv, o1[r + 3] * inv));
    }
  }
}

__global__ void __launch_bounds__(64) flow_speaker_kernel(const float* spk, const float* W, const float* b, float* out, int E, int mel) {
  const int r = blockIdx.x, lane = threadIdx.x;
  const float* x = spk + (size_t)r * E;
  float ss = 0.f;
  for (int e = lane; e < E; e += 64) ss += x[e] * x[e];
  const float inv = 1.0f / fmaxf(sqrtf(wave_sum(ss)), 1e-12f);
  for (int o = lane; o < mel; o += 64) {
    float acc = 0.f;
    const float* w = W + (size_t)o * E;
    for (int e = 0; e < E; ++e) acc += w[e] * (x[e] * inv);
    out[(size_t)r * mel + o] = acc + b[o];
  }
}

int blocks4(int n) { return (n + 3) / 4; }

}  // namespace

#define T2W_FLOW_VPL(C, CALL)                        \
  switch ((C) / 64) {                                \
    case 8: { constexpr int V = 8; CALL; } break;    \
    case 16: { constexpr int V = 16; CALL; } break;  \
    default: return hipErrorInvalidValue;            \
  }

hipError_t flow_embed(const float* table, const int* tok, const int* res, const float* w, const float* b, float eps, float xscale,
                      bf16_t* x0, f16_t* h, int n, int C, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  T2W_FLOW_VPL(C, hipLaunchKernelGGL((flow_embed_kernel<V>), dim3(blocks4(n)), dim3(256), 0, st, table, tok, res, w, b, eps, xscale, x0, h, n, C));
  return hipGetLastError();
}

hipError_t flow_look_place(bf16_t* G, bf16_t* cache, const int* g, const int* t1, const int* rd, const int* wr, int R, int C,
                           long long cstride, hipStream_t st) {
  if (R <= 0) return hipSuccess;
  if (C % 512) return hipErrorInvalidValue;
  hipLaunchKernelGGL(flow_look_place_kernel, dim3(R), dim3(64), 0, st, G, cache, g, t1, rd, wr, C, cstride);
  return hipGetLastError();
}

hipError_t flow_up_place(const f16_t* h, bf16_t* U, const int* up_dst, int n1, const int* u, const int* o1, const int* t1,
                         bf16_t* cache, const int* rd, const int* wr, int R, int C, long long cstride, hipStream_t st) {
  if (n1 + R <= 0) return hipSuccess;
  if (C % 512) return hipErrorInvalidValue;
  const int nbr = blocks4(n1);
  hipLaunchKernelGGL(flow_up_place_kernel, dim3(nbr + R), dim3(256), 0, st, h, U, up_dst, n1, nbr, u, o1, t1, cache, rd, wr, C, cstride);
  return hipGetLastError();
}

hipError_t flow_ln_scale_ln(const float* y, const float* w1, const float* b1, float eps1, float xscale, f16_t* h, const float* w2,
                            const float* b2, float eps2, bf16_t* a, int n, int C, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  T2W_FLOW_VPL(C, hipLaunchKernelGGL((flow_ln_scale_ln_kernel<V>), dim3(blocks4(n)), dim3(256), 0, st, y, w1, b1, eps1, xscale, h, w2, b2, eps2, a, n, C));
  return hipGetLastError();
}

hipError_t flow_kv_store(const f16_t* qkv, int ldq, f16_t* pool, const int* slot, int n, int C, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  if (C % 256 || ldq % 8) return hipErrorInvalidValue;
  hipLaunchKernelGGL(flow_kv_store_kernel, dim3(blocks4(n)), dim3(256), 0, st, qkv, ldq, pool, slot, n, C);
  return hipGetLastError();
}

hipError_t flow_rel_attention(const RelAttnArgs& a, hipStream_t st) {
  if (a.n_tiles <= 0) return hipSuccess;
  if (a.heads <= 0 || a.ldq % 8 || a.rmax < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(flow_rel_attn_kernel, dim3(a.n_tiles, a.heads), dim3(64), 0, st, a);
  return hipGetLastError();
}

hipError_t flow_speaker(const float* spk, const float* W, const float* b, float* out, int R, int E, int mel, hipStream_t st) {
  if (R <= 0) return hipSuccess;
  hipLaunchKernelGGL(flow_speaker_kernel, dim3(R), dim3(64), 0, st, spk, W, b, out, E, mel);
  return hipGetLastError();
}

}  // namespace t2w
