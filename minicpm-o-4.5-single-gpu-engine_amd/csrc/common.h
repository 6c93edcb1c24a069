// Shared device helpers of the Token2Wav HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace t2w {

typedef uint16_t bf16_t;  // storage type of bf16 activations and weights
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// float -> bf16, round to nearest even: gfx950's v_cvt_pk_bf16_f32 (one instruction per pair)
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

__device__ __forceinline__ float bf2f(bf16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// two bf16 packed in a 32-bit word (low half = first element)
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
// fp16 storage of the residual stream (the reference's activation dtype): round to nearest even, one value at a time
typedef uint16_t f16_t;

__device__ __forceinline__ f16_t f2h(float f) { return __builtin_bit_cast(f16_t, (_Float16)f); }
__device__ __forceinline__ float h2f(f16_t x) { return (float)__builtin_bit_cast(_Float16, x); }
__device__ __forceinline__ uint32_t pack2h(float a, float b) { return (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16); }
__device__ __forceinline__ float lo2h(uint32_t w) { return h2f((f16_t)(w & 0xffffu)); }
__device__ __forceinline__ float hi2h(uint32_t w) { return h2f((f16_t)(w >> 16)); }

__device__ __forceinline__ float lo2f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi2f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
  union { uint4 u; bf16x8 b; } c;
  c.u = v;
  return c.b;
}

// wave64 butterfly sum / max over all lanes (every lane gets the result)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// sum over the 16 lanes of a DPP row (lanes 16 r .. 16 r + 15), every lane gets it: quad swaps, then half-row and
// row mirrors (each step pairs a lane with one not yet summed in); VALU only, no LDS
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)); // row_half_mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)); // row_mirror
  return v;
}

// sum over an aligned group of 8 lanes, every lane gets it: DPP swaps within quads (lane ^ 1, lane ^ 2), then the
// half-row mirror pairs the two quads; the same sums as a butterfly over lane ^ 1, ^ 2, ^ 4 (after the first two
// steps a quad's lanes agree), with no LDS round trip
__device__ __forceinline__ float sum8(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)); // row_half_mirror
  return v;
}

// the same over aligned groups of 4 lanes (the butterfly's lane ^ 1, ^ 2 steps exactly) and the maximum over groups
// of 4 or 8 (any pairing gives the same maximum)
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  return v;
}
__device__ __forceinline__ float max8(float v) {
  v = quad_max(v);
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
}
// sum over aligned groups of L = 4, 8 or 16 lanes, the butterfly's sums over lane ^ 1 .. ^ (L / 2)
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(L == 4 || L == 8 || L == 16, "DPP groups");
  if constexpr (L == 4) return quad_sum(v);
  else if constexpr (L == 8) return sum8(v);
  else return row16_sum(v);
}

// x of lane l ^ 32 (the other half of the wave) through v_permlane32_swap, a VALU op (no LDS round trip): the swap of
// x with itself leaves lanes 32..63 of the first result holding lanes 0..31 and lanes 0..31 of the second holding
// lanes 32..63
__device__ __forceinline__ float xor32(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

// sum over the wave, the same value in every lane, with no LDS round trip: each 16-lane DPP row sums itself
// (row16_sum), then the four row sums are added in row order from scalar reads of lanes 0, 16, 32 and 48
__device__ __forceinline__ float wave_sum_rows(float v) {
  v = row16_sum(v);
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return ((r0 + r1) + r2) + r3;
}

// Rotary position embedding (RoFormer, consecutive channel pairs): y[0..NV) holds whole pairs of one head, pair e / 2
// turning by the angle pos * freq[e / 2] (the fp32 product, then an accurate sine and cosine of it)
template <int NV>
__device__ __forceinline__ void rope_rotate(float (&y)[NV], int pos, const float* freq) {
  static_assert(NV % 2 == 0, "whole channel pairs");
#pragma unroll
  for (int e = 0; e < NV; e += 2) {
    float sn, cs;
    sincosf((float)pos * freq[e >> 1], &sn, &cs);
    const float y0 = y[e], y1 = y[e + 1];
    y[e] = y0 * cs - y1 * sn;
    y[e + 1] = y0 * sn + y1 * cs;
  }
}

// MX fp8: OCP e4m3 values with one power-of-two (E8M0) scale per 32 consecutive K values.  The scale is the smallest
// power of two that keeps the block's largest magnitude within e4m3's 448, so nothing clips: with amax = 1.m * 2^E and
// 448 = 1.75 * 2^8, that exponent is E - 8, plus one when 1.m > 1.75.  Returns the unbiased exponent in [-126, 126].
__device__ __forceinline__ int mx_exp(float amax) {
  const uint32_t b = __float_as_uint(amax) & 0x7fffffffu;
  if (b < 0x00800000u) return -126;  // zero or subnormal block
  int e = (int)(b >> 23) - 127 - 8 + ((b & 0x7fffffu) > 0x600000u ? 1 : 0);
  return e < -126 ? -126 : (e > 126 ? 126 : e);
}

// four values times 2^-se, clamped to +-448 and rounded to nearest even e4m3 (v_cvt_pk_fp8_f32), packed low byte first
__device__ __forceinline__ uint32_t mx_pack4(float a, float b, float c, float d, int se) {
  const float inv = __uint_as_float((uint32_t)(127 - se) << 23);
  auto cl = [](float x) { return fminf(fmaxf(x, -448.0f), 448.0f); };
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a * inv), cl(b * inv), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(c * inv), cl(d * inv), w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3), written as x / (1 + 2^(-2 u log2 e)): one v_exp_f32 and
  // one v_rcp_f32 (1 ulp; the result is rounded to bf16).  A plain or __fdividef division compiles to the IEEE
  // division sequence here (scale, fmas, fixup), which made the GELU epilogue twice as slow as a plain one.
  const float c0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f, c1 = 0.044715f;
  const float t = c0 * (x + c1 * x * x * x);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// Activation of the plain bf16 GEMM epilogue (GemmArgs::act), applied after the bias.
enum Act { ACT_NONE = 0, ACT_SILU = 1, ACT_LRELU = 2 };

// x sigmoid(x) = x / (1 + 2^(-x log2 e)): one v_exp_f32 and one v_rcp_f32
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// ACT_LRELU is torch's leaky_relu at its default slope 0.01
__device__ __forceinline__ float act_apply(float x, int act) {
  return act == ACT_SILU ? silu(x) : (act == ACT_LRELU ? (x > 0.0f ? x : 0.01f * x) : x);
}

__device__ __forceinline__ float mish(float y) {
  // y tanh(softplus(y)) = y n (n + 2) / (n (n + 2) + 2) with n = e^y; above torch's softplus threshold 20 it is y
  if (y > 20.0f) return y;
  const float n = __expf(y);
  const float p = n * (n + 2.0f);
  return y * p * __builtin_amdgcn_rcpf(p + 2.0f);
}

}  // namespace t2w
