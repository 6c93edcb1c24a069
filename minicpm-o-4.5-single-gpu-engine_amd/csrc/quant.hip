// MX fp8 quantization of a bf16 activation matrix for the fp8 GEMMs: x [M, K] -> q [M, K] OCP e4m3 and
// s [M, K / 32] E8M0 block scales (the scale rule is mx_exp in common.h).
//
// Four threads share a 32-value block, eight values each: one 16-byte load, two shuffles for the block maximum, one
// 8-byte store of e4m3 codes; the block's first thread writes the scale byte.
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

__global__ void __launch_bounds__(256) quant_mx8_kernel(const bf16_t* x, int ldx, int M, int K, uint8_t* q, int ldq, uint8_t* s) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  const int per_row = K / 8;
  if (t >= (long)M * per_row) return;  // blocks of 4 threads are whole: K % 32 == 0
  const int m = (int)(t / per_row), k = (int)(t - (long)m * per_row) * 8;
  const uint4 u = *(const uint4*)(x + (size_t)m * ldx + k);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) { v[2 * j] = lo2f(w[j]); v[2 * j + 1] = hi2f(w[j]); }
  float a = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(v[j]));
  a = quad_max(a);  // the block's four lanes (DPP)
  const int se = mx_exp(a);
  *(uint2*)(q + (size_t)m * ldq + k) = make_uint2(mx_pack4(v[0], v[1], v[2], v[3], se), mx_pack4(v[4], v[5], v[6], v[7], se));
  if ((k & 31) == 0) s[(size_t)m * (K / 32) + k / 32] = (uint8_t)(se + 127);
}

// out[n, k] = bf16(e4m3(w8[n, k]) * ws[n]): the fp32 product rounded once to bf16; eight codes per thread
__global__ void __launch_bounds__(256) dequant_w8_kernel(const uint8_t* w8, const float* ws, int N, int K, bf16_t* out) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  const int per_row = K / 8;
  if (t >= (long)N * per_row) return;
  const int n = (int)(t / per_row), k = (int)(t - (long)n * per_row) * 8;
  const uint2 c = *(const uint2*)(w8 + (size_t)n * K + k);
  const float sc = ws[n];
  uint32_t o[4];
  const uint32_t w[2] = {c.x, c.y};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[j], false);  // bytes 0, 1
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[j], true);   // bytes 2, 3
    o[2 * j] = pack2(lo[0] * sc, lo[1] * sc);
    o[2 * j + 1] = pack2(hi[0] * sc, hi[1] * sc);
  }
  *(uint4*)(out + (size_t)n * K + k) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

hipError_t dequant_w8(const uint8_t* w8, const float* ws, int N, int K, bf16_t* out, hipStream_t st) {
  if (N <= 0 || K % 8) return N <= 0 ? hipSuccess : hipErrorInvalidValue;
  const long threads = (long)N * (K / 8);
  hipLaunchKernelGGL(dequant_w8_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, w8, ws, N, K, out);
  return hipGetLastError();
}

hipError_t quant_mx8(const bf16_t* x, int ldx, int M, int K, uint8_t* q, int ldq, uint8_t* s, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  const long threads = (long)M * (K / 8);
  hipLaunchKernelGGL(quant_mx8_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, x, ldx, M, K, q, ldq, s);
  return hipGetLastError();
}

}  // namespace t2w
