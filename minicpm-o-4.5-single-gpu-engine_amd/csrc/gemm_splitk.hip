// Split-K bf16 MFMA GEMM for calls with few rows (a streaming chunk: ~100 tokens), where a tile grid would leave the
// chip idle and the time is the weight stream from HBM.
//
// Pass 1: one wave per work item (64 output columns x up to 128 rows x a slice of K).  Operand fragments go straight
// from global memory into registers: W (the MFMA B side, columns n) and A (the A side, rows m) are read 64 contiguous
// bytes per lane per 64-K step, which the MFMA sees as four 16-K slices of a permuted K order (the same permutation on
// both sides, so the dot products are unchanged).  Rows past M load row M - 1 and are never stored.  The wave writes
// its fp32 partial tile to the workspace in the accumulators' own register order, one contiguous kilobyte per store
// (a work item's partial is [row tile i][column tile j][register quad q][lane][4]).
// Pass 2: one thread per (work item, i, j, q, lane) sums that float4 over the S splits in split order (deterministic)
// and applies the epilogue to its four outputs: rows m .. m + 3 of column n.
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

constexpr int SK_BN = 64;   // output columns per work item
constexpr int SK_BM = 128;  // rows per work item (4 MFMA row tiles)
constexpr int SK_ITEM4 = 4 * 2 * 4 * 64;  // float4 of one work item's partial

// NS > 0: every split has at most NS steps, all of whose loads are issued before the first MFMA (separate registers
// per step); NS == 0: any number of steps, two register stages.
template <bool TAPS, int NS>
__global__ void __launch_bounds__(64) splitk_partial_kernel(GemmArgs g, float* part, int steps_per_split) {
  const int n0 = blockIdx.x * SK_BN, ks = blockIdx.y, mbase = blockIdx.z * SK_BM;
  const int lane = threadIdx.x, h = lane >> 5, c = lane & 31;
  const int KS = g.K / 64;
  const int s0 = ks * steps_per_split, s1 = min(KS, s0 + steps_per_split);
  const int mt = min(4, (g.M - mbase + 31) / 32);  // live 32-row tiles (wave-uniform)

  // this lane's rows (A side) and columns (B side)
  int arow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) arow[i] = min(mbase + i * 32 + c, g.M - 1);
  const bf16_t* wrow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) wrow[j] = g.B + (size_t)min(n0 + j * 32 + c, g.N - 1) * g.ldb + h * 32;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // fragments of one 64-K step: W (B side) and A (A side), 64 contiguous bytes per lane and row
  auto load = [&](int step, uint4 (&wf)[2][4], uint4 (&af)[4][4]) {
    const int k0 = step * 64;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) wf[j][kk] = *(const uint4*)(wrow[j] + k0 + kk * 8);
    size_t aoff = k0;
    if (TAPS) {
      const int tap = k0 / g.tapC;  // a 64-K step never straddles two taps (tapC % 64 == 0)
      aoff = (size_t)tap * g.lda + (k0 - tap * g.tapC);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i >= mt) break;
      const bf16_t* ap = TAPS ? g.A + (size_t)g.a_src[arow[i]] * g.lda : g.A + (size_t)arow[i] * g.lda;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) af[i][kk] = *(const uint4*)(ap + aoff + h * 32 + kk * 8);
    }
  };
  auto mma = [&](const uint4 (&wf)[2][4], const uint4 (&af)[4][4]) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i >= mt) break;
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(af[i][kk]), as_bf16x8(wf[j][kk]), acc[i][j], 0, 0, 0);
      }
  };
  if (NS > 0) {
    uint4 wf[NS > 0 ? NS : 1][2][4], af[NS > 0 ? NS : 1][4][4];
#pragma unroll
    for (int t = 0; t < NS; ++t)
      if (s0 + t < s1) load(s0 + t, wf[t], af[t]);
#pragma unroll
    for (int t = 0; t < NS; ++t)
      if (s0 + t < s1) mma(wf[t], af[t]);
  } else {
    // two register stages: the loads of the next step are in flight while this step's MFMAs run
    uint4 w0[2][4], a0[4][4], w1[2][4], a1[4][4];
    int s = s0;
    if (s < s1) load(s, w0, a0);
    while (s < s1) {
      if (s + 1 < s1) load(s + 1, w1, a1);
      mma(w0, a0);
      if (++s >= s1) break;
      if (s + 1 < s1) load(s + 1, w0, a0);
      mma(w1, a1);
      ++s;
    }
  }

  // lane holds column n0 + j * 32 + c of rows mbase + i * 32 + q * 8 + h * 4 + e in register 4 q + e
  const int item = blockIdx.z * gridDim.x + blockIdx.x;
  float4* pb = (float4*)part + ((size_t)ks * gridDim.x * gridDim.z + item) * SK_ITEM4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i >= mt) break;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        pb[((i * 2 + j) * 4 + q) * 64 + lane] = make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
  }
}

template <int EPI>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs g, const float* part, int S, int ntile, int items) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= items * SK_ITEM4) return;
  const int lane = t & 63, q = (t >> 6) & 3, j = (t >> 8) & 1, i = (t >> 9) & 3, item = t >> 11;
  const int nt = item % ntile, mb = item / ntile;
  const int n = nt * SK_BN + j * 32 + (lane & 31);
  const int m0 = mb * SK_BM + i * 32 + q * 8 + (lane >> 5) * 4;
  if (n >= g.N || m0 >= g.M) return;
  const size_t plane = (size_t)items * SK_ITEM4;
  const float4* p = (const float4*)part + t;
  // partials summed in split order; up to 8 loads in flight before the adds
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < S; s0 += 8) {
    float4 b[8];
#pragma unroll
    for (int x = 0; x < 8; ++x)
      if (s0 + x < S) b[x] = p[(size_t)(s0 + x) * plane];
#pragma unroll
    for (int x = 0; x < 8; ++x)
      if (s0 + x < S) { a.x += b[x].x; a.y += b[x].y; a.z += b[x].z; a.w += b[x].w; }
  }
  const float bias = g.bias[n];
  const float gate = EPI == EPI_RESID_F16 ? g.gate[n] : 0.f;
  const float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = m0 + e;
    if (m >= g.M) break;
    float x = v[e] + bias;
    const size_t o = (size_t)m * g.ldc + n;
    if (EPI == EPI_GELU_BF16) x = gelu_tanh(x);
    if (EPI == EPI_BF16) x = act_apply(x, g.act);
    if (EPI == EPI_BF16 || EPI == EPI_GELU_BF16) ((bf16_t*)g.C)[o] = f2bf(x);
    else if (EPI == EPI_RESID_F16) ((f16_t*)g.C)[o] = f2h(h2f(((const f16_t*)g.C)[o]) + gate * x);
    else if (EPI == EPI_F16) ((f16_t*)g.C)[o] = f2h(x);
    else ((float*)g.C)[o] = x;
  }
}

}  // namespace

SplitPlan splitk_plan(int M, int N, int K, size_t ws_bytes) {
  SplitPlan p{0, 0};
  if (K % 64) return p;
  const int ntile = (N + SK_BN - 1) / SK_BN, mblk = (M + SK_BM - 1) / SK_BM, KS = K / 64;
  // two K steps per wave when that still gives at least 256 waves, else one; fewer splits (more steps) only when the
  // partials would not fit the workspace
  const int items = ntile * mblk;
  int steps = items * ((KS + 1) / 2) >= 256 ? 2 : 1;
  if (steps > KS) steps = KS;
  const size_t plane = (size_t)items * SK_ITEM4 * 16;
  while ((size_t)((KS + steps - 1) / steps) * plane > ws_bytes && steps < KS) ++steps;
  const int S = (KS + steps - 1) / steps;
  if ((size_t)S * plane > ws_bytes) return p;
  p.splits = (KS + steps - 1) / steps;
  p.steps = steps;
  return p;
}

hipError_t gemm_splitk(const GemmArgs& g, int epi, const SplitPlan& p, float* part, hipStream_t st) {
  const dim3 grid((g.N + SK_BN - 1) / SK_BN, p.splits, (g.M + SK_BM - 1) / SK_BM);
  const bool taps = g.a_src != nullptr;
  if (p.steps == 1) {
    if (taps) hipLaunchKernelGGL((splitk_partial_kernel<true, 1>), grid, dim3(64), 0, st, g, part, p.steps);
    else hipLaunchKernelGGL((splitk_partial_kernel<false, 1>), grid, dim3(64), 0, st, g, part, p.steps);
  } else if (p.steps == 2) {
    if (taps) hipLaunchKernelGGL((splitk_partial_kernel<true, 2>), grid, dim3(64), 0, st, g, part, p.steps);
    else hipLaunchKernelGGL((splitk_partial_kernel<false, 2>), grid, dim3(64), 0, st, g, part, p.steps);
  } else {
    if (taps) hipLaunchKernelGGL((splitk_partial_kernel<true, 0>), grid, dim3(64), 0, st, g, part, p.steps);
    else hipLaunchKernelGGL((splitk_partial_kernel<false, 0>), grid, dim3(64), 0, st, g, part, p.steps);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int ntile = grid.x, items = grid.x * grid.z;
  const int blocks = (items * SK_ITEM4 + 255) / 256;
  switch (epi) {
    case EPI_BF16: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_BF16>, dim3(blocks), dim3(256), 0, st, g, part, p.splits, ntile, items); break;
    case EPI_GELU_BF16: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_GELU_BF16>, dim3(blocks), dim3(256), 0, st, g, part, p.splits, ntile, items); break;
    case EPI_RESID_F16: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_RESID_F16>, dim3(blocks), dim3(256), 0, st, g, part, p.splits, ntile, items); break;
    case EPI_F16: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_F16>, dim3(blocks), dim3(256), 0, st, g, part, p.splits, ntile, items); break;
    case EPI_F32: hipLaunchKernelGGL(splitk_reduce_kernel<EPI_F32>, dim3(blocks), dim3(256), 0, st, g, part, p.splits, ntile, items); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace t2w
