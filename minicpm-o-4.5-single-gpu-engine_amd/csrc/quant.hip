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
  a = fmaxf(a, __shfl_xor(a, 1, 64));
  a = fmaxf(a, __shfl_xor(a, 2, 64));
  const int se = mx_exp(a);
  *(uint2*)(q + (size_t)m * ldq + k) = make_uint2(mx_pack4(v[0], v[1], v[2], v[3], se), mx_pack4(v[4], v[5], v[6], v[7], se));
  if ((k & 31) == 0) s[(size_t)m * (K / 32) + k / 32] = (uint8_t)(se + 127);
}

}  // namespace

hipError_t quant_mx8(const bf16_t* x, int ldx, int M, int K, uint8_t* q, int ldq, uint8_t* s, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  const long threads = (long)M * (K / 8);
  hipLaunchKernelGGL(quant_mx8_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, x, ldx, M, K, q, ldq, s);
  return hipGetLastError();
}

}  // namespace t2w
