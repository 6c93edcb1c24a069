// bf16 MFMA GEMM for calls with very few rows (a streaming chunk: ~100 tokens), in one kernel.
//
// At ~100 rows the time of a GEMM is the weight stream plus fixed per-kernel costs, and a split-K pass followed by a
// separate reduce kernel pays those costs twice and moves fp32 partials through HBM.  Here a workgroup of 16 waves
// owns 32 output columns x 32 rows and splits K over its waves: each wave loads its (at most three) 64-K steps of the
// W rows and activation rows into registers with whole-line loads (two steps in flight from the start), turns each
// step into MFMA fragments through its LDS slab (four 16-K slices of the same K permutation on both sides), then
// leaves its 32x32 fp32 block in LDS.  After one barrier the block is summed over the waves in wave order
// (deterministic) and the epilogue (bias, GELU, gated fp32 residual) writes four consecutive columns per lane.
//
// A workgroup moves its W and activation rows through one CU, and a CU's load throughput (not HBM) is what bounds
// these calls: ~100 rows x K = 3072 (conv taps) is 384 KB per workgroup on 128 CUs.  EPI_PART therefore also splits K
// over g.splits workgroups per tile (grid z), so that all CUs share the bytes, and leaves the sum of the splits, the
// bias and the gated residual to the row kernel that reads the result next (Pend).
//
// MFMA roles: W is the A operand (its 32 rows are output columns n0 ..), the activations the B operand (32 token
// rows), so a lane's four consecutive accumulator registers are four consecutive output columns of one token.
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

constexpr int GS_WAVES = 16;  // waves per workgroup, sharing K
constexpr int GS_MAXSTEPS = 3;  // 64-K steps per wave: K <= 16 * 3 * 64 = 3072

// 16-byte fragments as a native vector (an aggregate copy of uint4 into LDS keeps the loaded registers in scratch)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 frag(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

template <bool TAPS, int EPI>
__global__ void __launch_bounds__(64 * GS_WAVES) gemm_small_kernel(GemmArgs g) {
  // per wave 8 KB: the W and activation rows of one 64-K step (32 rows x 8 chunks of 16 bytes each), then its 32x32
  // block in register order (quad q, lane) for the reduction
  __shared__ u32x4 slab[GS_WAVES][512];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, c = lane & 31;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 32;
  const int KT = g.K / 64, z = blockIdx.z, S = gridDim.z;
  const int kb = z * KT / S, KS = (z + 1) * KT / S - kb;  // this workgroup's K split
  const int nw = blockDim.x >> 6;
  const int s0 = kb + w * KS / nw, s1 = kb + (w + 1) * KS / nw;  // this wave's steps (possibly none)
  // the epilogue's bias (and gate) of the four columns a thread of the first four waves finishes, loaded before the K
  // steps so that they are in registers when the block has been summed
  float4 eb = make_float4(0.f, 0.f, 0.f, 0.f), eg = eb;
  if (EPI != EPI_PART && tid < 256) {
    const int en = n0 + (tid >> 6) * 8 + ((tid & 63) >> 5) * 4;
    if (en + 3 < g.N) {
      eb = *(const float4*)(g.bias + en);
      if (EPI == EPI_RESID_F16) eg = *(const float4*)(g.gate + en);
    }
  }
  // Load instruction kk of a step covers rows kk * 8 + lane / 8, eight lanes per row (its 64 K values, one 128-byte
  // line): whole lines per instruction run at about 1.4x the CU's rate for 32-byte pieces of 32 rows.  The wave's slab
  // turns them into MFMA fragments (lane (c, h) takes bytes h * 64 + kk * 16 of row c), 16-byte chunks XOR-swizzled by
  // (row / 2) % 8 so that both the writes and the fragment reads are free of bank conflicts.
  const int lr = lane >> 3, lc = lane & 7;
  int arow[4];  // activation row (taps: frame) of each load instruction
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int m = min(m0 + kk * 8 + lr, g.M - 1);  // rows past M load row M - 1; their results are never stored
    arow[kk] = TAPS ? g.a_src[m] : m;
  }

  // two register sets: steps 0 and 1 in flight from the start, step 2 (K = 3072 unsplit) once step 0 is consumed
  u32x4 wf[2][4], af[2][4];
  auto load = [&](int t, u32x4 (&wd)[4], u32x4 (&ad)[4]) {
    const int k0 = (s0 + t) * 64;
    size_t aoff = k0;
    if (TAPS) {
      const int tap = k0 / g.tapC;  // a 64-K step never straddles two taps (tapC % 64 == 0)
      aoff = (size_t)tap * g.lda + (k0 - tap * g.tapC);
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      wd[kk] = *(const u32x4*)(g.B + (size_t)min(n0 + kk * 8 + lr, g.N - 1) * g.ldb + k0 + lc * 8);
      ad[kk] = *(const u32x4*)(g.A + (size_t)arow[kk] * g.lda + aoff + lc * 8);
    }
  };
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  u32x4* sl = slab[w];  // this wave's own: LDS accesses of one wave complete in order, no barrier needed
  auto consume = [&](const u32x4 (&wd)[4], const u32x4 (&ad)[4]) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int r = kk * 8 + lr, x = r * 8 + (lc ^ ((r >> 1) & 7));
      sl[x] = wd[kk];
      sl[256 + x] = ad[kk];
    }
    u32x4 wv[4], av[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int x = c * 8 + ((h * 4 + kk) ^ ((c >> 1) & 7));
      wv[kk] = sl[x];
      av[kk] = sl[256 + x];
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(wv[kk]), frag(av[kk]), acc, 0, 0, 0);
  };
  const int ns = s1 - s0;  // 0 .. GS_MAXSTEPS; one straight path per count (no register sets merged across branches)
  if (ns == 1) {
    load(0, wf[0], af[0]);
    consume(wf[0], af[0]);
  } else if (ns == 2) {
    load(0, wf[0], af[0]);
    load(1, wf[1], af[1]);
    consume(wf[0], af[0]);
    consume(wf[1], af[1]);
  } else if (ns == 3) {
    load(0, wf[0], af[0]);
    load(1, wf[1], af[1]);
    consume(wf[0], af[0]);
    load(2, wf[0], af[0]);
    consume(wf[1], af[1]);
    consume(wf[0], af[0]);
  }
  float4* red = (float4*)sl;
#pragma unroll
  for (int q = 0; q < 4; ++q) red[q * 64 + lane] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
  __syncthreads();

  // one float4 (four columns of one row) per thread of the first four waves, summed over the waves in order
  if (tid >= 256) return;
  const int q = tid >> 6, l = tid & 63;
  float4 a = ((const float4*)slab[0])[q * 64 + l];
#pragma unroll
  for (int x = 1; x < nw; ++x) {
    const float4 b = ((const float4*)slab[x])[q * 64 + l];
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
  }
  // lane l of the MFMA holds token m0 + l % 32 and columns n0 + q * 8 + (l / 32) * 4 + 0..3
  const int mo = m0 + (l & 31), n = n0 + q * 8 + (l >> 5) * 4;
  if (mo >= g.M || n >= g.N) return;
  const float v[4] = {a.x, a.y, a.z, a.w};
  float* part = (float*)g.C + (size_t)z * g.c_split;  // EPI_PART: this split's sums
  if (n + 3 < g.N) {
    if (EPI == EPI_PART) {
      *(float4*)(part + (size_t)mo * g.ldc + n) = a;
      return;
    }
    const float4 b = eb;
    float o[4] = {v[0] + b.x, v[1] + b.y, v[2] + b.z, v[3] + b.w};
    const size_t off = (size_t)mo * g.ldc + n;
    if (EPI == EPI_GELU_BF16) {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = gelu_tanh(o[e]);
    }
    if (EPI == EPI_BF16 && g.act) {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = act_apply(o[e], g.act);
    }
    if (EPI == EPI_BF16 || EPI == EPI_GELU_BF16) {
      *(uint2*)((bf16_t*)g.C + off) = make_uint2(pack2(o[0], o[1]), pack2(o[2], o[3]));
    } else if (EPI == EPI_RESID_F16) {
      const float4 gt = eg;
      uint2* hp = (uint2*)((f16_t*)g.C + off);
      const uint2 hv = *hp;
      *hp = make_uint2(pack2h(lo2h(hv.x) + gt.x * o[0], hi2h(hv.x) + gt.y * o[1]), pack2h(lo2h(hv.y) + gt.z * o[2], hi2h(hv.y) + gt.w * o[3]));
    } else if (EPI == EPI_F16) {
      *(uint2*)((f16_t*)g.C + off) = make_uint2(pack2h(o[0], o[1]), pack2h(o[2], o[3]));
    } else {
      *(float4*)((float*)g.C + off) = make_float4(o[0], o[1], o[2], o[3]);
    }
    return;
  }
  for (int e = 0; e < 4 && n + e < g.N; ++e) {  // the last columns of an N that is not a multiple of 4
    float x = v[e] + (EPI == EPI_PART ? 0.f : g.bias[n + e]);
    const size_t off = (size_t)mo * g.ldc + n + e;
    if (EPI == EPI_PART) { part[off] = v[e]; continue; }
    if (EPI == EPI_GELU_BF16) x = gelu_tanh(x);
    if (EPI == EPI_BF16) x = act_apply(x, g.act);
    if (EPI == EPI_BF16 || EPI == EPI_GELU_BF16) ((bf16_t*)g.C)[off] = f2bf(x);
    else if (EPI == EPI_RESID_F16) ((f16_t*)g.C)[off] = f2h(h2f(((const f16_t*)g.C)[off]) + g.gate[n + e] * x);
    else if (EPI == EPI_F16) ((f16_t*)g.C)[off] = f2h(x);
    else ((float*)g.C)[off] = x;
  }
}

// EPI_PART with 64-row tiles for calls of more than 32 rows: every W slice is read by half as many workgroups as with
// 32-row tiles (at ~100 rows the fourth 32-row tile held 4 rows and still read all of W).  A wave takes at most one
// 64-K step (K / splits <= 1024): its W rows and the first 32 activation rows go through the slab, then the other 32
// activation rows, both against the same W fragments.
template <bool TAPS>
__global__ void __launch_bounds__(64 * GS_WAVES) gemm_small_part64_kernel(GemmArgs g) {
  __shared__ u32x4 slab[GS_WAVES][512];  // per wave: W rows + 32 activation rows of its step, then its two blocks
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, c = lane & 31;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * 64;
  const int KT = g.K / 64, z = blockIdx.z, S = gridDim.z;
  const int kb = z * KT / S, KS = (z + 1) * KT / S - kb;
  const int nw = blockDim.x >> 6;
  const int s0 = kb + w * KS / nw, s1 = kb + (w + 1) * KS / nw;  // at most one step
  const int lr = lane >> 3, lc = lane & 7;
  f32x16 acc[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[rb][r] = 0.0f;
  u32x4* sl = slab[w];
  if (s0 < s1) {
    const int k0 = s0 * 64;
    size_t aoff = k0;
    if (TAPS) {
      const int tap = k0 / g.tapC;
      aoff = (size_t)tap * g.lda + (k0 - tap * g.tapC);
    }
    u32x4 wf[4], af[8];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      wf[kk] = *(const u32x4*)(g.B + (size_t)min(n0 + kk * 8 + lr, g.N - 1) * g.ldb + k0 + lc * 8);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int m = min(m0 + j * 8 + lr, g.M - 1);  // rows past M load row M - 1; their results are never stored
      af[j] = *(const u32x4*)(g.A + (size_t)(TAPS ? g.a_src[m] : m) * g.lda + aoff + lc * 8);
    }
    u32x4 wv[4], av[4];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int r = kk * 8 + lr, x = r * 8 + (lc ^ ((r >> 1) & 7));
        if (rb == 0) sl[x] = wf[kk];
        sl[256 + x] = af[rb * 4 + kk];
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int x = c * 8 + ((h * 4 + kk) ^ ((c >> 1) & 7));
        if (rb == 0) wv[kk] = sl[x];
        av[kk] = sl[256 + x];
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(wv[kk]), frag(av[kk]), acc[rb], 0, 0, 0);
    }
  }
  float4* red = (float4*)sl;  // [row block][quad][lane]
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(rb * 4 + q) * 64 + lane] = make_float4(acc[rb][4 * q], acc[rb][4 * q + 1], acc[rb][4 * q + 2], acc[rb][4 * q + 3]);
  __syncthreads();
  if (tid >= 512) return;  // one float4 per thread of the first eight waves, summed over the waves in order
  const int rb = tid >> 8, q = (tid >> 6) & 3, l = tid & 63;
  float4 a = ((const float4*)slab[0])[(rb * 4 + q) * 64 + l];
#pragma unroll
  for (int x = 1; x < nw; ++x) {
    const float4 b = ((const float4*)slab[x])[(rb * 4 + q) * 64 + l];
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
  }
  const int mo = m0 + rb * 32 + (l & 31), n = n0 + q * 8 + (l >> 5) * 4;
  if (mo >= g.M || n >= g.N) return;
  float* part = (float*)g.C + (size_t)z * g.c_split + (size_t)mo * g.ldc;
  if (n + 3 < g.N) {
    *(float4*)(part + n) = a;
    return;
  }
  const float v[4] = {a.x, a.y, a.z, a.w};
  for (int e = 0; e < 4 && n + e < g.N; ++e) part[n + e] = v[e];
}

// The qkv projection (N = 3 H) for few rows, with the per-head q / k LayerNorm and the key / value scatter fused:
// 64 columns (one head of q, k or v) x 32 rows per workgroup, K split over the 16 waves (one 64-K step each, so
// K <= 1024).  The block summed over the waves goes row-major through LDS, where the 16 lanes of one DPP row hold a
// row's 64 columns: bias, rounding to bf16 (the projection's own precision), LayerNorm + affine for q and k, then q
// to its token row and k, v to the token's key slot.
__global__ void __launch_bounds__(64 * GS_WAVES) gemm_small_qkv_kernel(GemmArgs g) {
  // per wave 8 KB: one 64-K step of the activation rows and of one column tile's W rows (the two tiles in turn), then
  // its two 32x32 blocks (column tiles) in register order for the reduction
  __shared__ u32x4 slab[GS_WAVES][512];
  __shared__ float rowm[32][68];  // the summed 32 x 64 block, row-major (padded rows)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, c = lane & 31;
  const int n0 = blockIdx.x * 64, m0 = blockIdx.y * 32;
  const int KS = g.K / 64;
  const int s0 = w * KS / GS_WAVES, s1 = (w + 1) * KS / GS_WAVES;  // at most one step
  // the epilogue's operands (threads of the first eight waves: token row er, columns ec4 .. ec4 + 3 of the head) are
  // loaded before the K step, so that they are in registers when the block has been summed
  const QkvOut& o = g.qk;
  const int er = tid >> 4, ec4 = (tid & 15) * 4;  // 16 consecutive lanes (a DPP row) per token row
  const int part = n0 / o.H;                       // q, k or v
  float4 eb = make_float4(0.f, 0.f, 0.f, 0.f), elw = eb, elb = eb;
  int eslot = 0;
  if (tid < 512) {
    eb = *(const float4*)(g.bias + n0 + ec4);
    if (part < 2) {
      elw = *(const float4*)((part ? o.kw : o.qw) + ec4);
      elb = *(const float4*)((part ? o.kb : o.qb) + ec4);
    }
    if (part > 0 && m0 + er < g.M) eslot = o.slots[m0 + er];
  }
  const int lr = lane >> 3, lc = lane & 7;  // whole-line loads and the slab's swizzle, as in gemm_small_kernel
  f32x16 acc[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[ct][r] = 0.0f;
  u32x4* sl = slab[w];
  if (s0 < s1) {
    const int k0 = s0 * 64;
    u32x4 wf[2][4], af[4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        wf[ct][kk] = *(const u32x4*)(g.B + (size_t)min(n0 + ct * 32 + kk * 8 + lr, g.N - 1) * g.ldb + k0 + lc * 8);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      af[kk] = *(const u32x4*)(g.A + (size_t)min(m0 + kk * 8 + lr, g.M - 1) * g.lda + k0 + lc * 8);
    u32x4 av[4], wv[4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int r = kk * 8 + lr, x = r * 8 + (lc ^ ((r >> 1) & 7));
        sl[x] = wf[ct][kk];
        if (ct == 0) sl[256 + x] = af[kk];
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int x = c * 8 + ((h * 4 + kk) ^ ((c >> 1) & 7));
        wv[kk] = sl[x];
        if (ct == 0) av[kk] = sl[256 + x];
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(wv[kk]), frag(av[kk]), acc[ct], 0, 0, 0);
    }
  }
  float4* red = (float4*)sl;  // [ct][q][lane]
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(ct * 4 + q) * 64 + lane] = make_float4(acc[ct][4 * q], acc[ct][4 * q + 1], acc[ct][4 * q + 2], acc[ct][4 * q + 3]);
  __syncthreads();
  if (tid < 512) {  // sum over the waves in order; lane l holds token m0 + l % 32, columns ct * 32 + q * 8 + (l / 32) * 4 + 0..3
    const int ct = tid >> 8, q = (tid >> 6) & 3, l = tid & 63;
    float4 a = ((const float4*)slab[0])[(ct * 4 + q) * 64 + l];
#pragma unroll
    for (int x = 1; x < GS_WAVES; ++x) {
      const float4 b = ((const float4*)slab[x])[(ct * 4 + q) * 64 + l];
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    }
    *(float4*)&rowm[l & 31][ct * 32 + q * 8 + (l >> 5) * 4] = a;
  }
  __syncthreads();
  if (tid >= 512) return;
  const int r = er, c4 = ec4;
  const float4 a = *(const float4*)&rowm[r][c4];
  const float4 b = eb;
  float y[4] = {bf2f(f2bf(a.x + b.x)), bf2f(f2bf(a.y + b.y)), bf2f(f2bf(a.z + b.z)), bf2f(f2bf(a.w + b.w))};
  const int hc = n0 - part * o.H + c4;  // column within the part
  if (part < 2) {
    const float mean = row16_sum(y[0] + y[1] + y[2] + y[3]) * (1.0f / 64.0f);
    float var = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) { y[e] -= mean; var += y[e] * y[e]; }
    const float rstd = rsqrtf(row16_sum(var) * (1.0f / 64.0f) + o.eps);
    const float4 lw = elw, lb = elb;
    y[0] = y[0] * rstd * lw.x + lb.x;
    y[1] = y[1] * rstd * lw.y + lb.y;
    y[2] = y[2] * rstd * lw.z + lb.z;
    y[3] = y[3] * rstd * lw.w + lb.w;
    if (o.rfreq) rope_rotate<4>(y, m0 + r < g.M ? o.pos[m0 + r] : 0, o.rfreq + (c4 >> 1));
  }
  const int mo = m0 + r;
  if (mo >= g.M) return;
  bf16_t* dst = part == 0 ? o.q_out + (size_t)mo * o.H : (part == 1 ? o.k_pool : o.v_pool) + (size_t)eslot * o.H;
  *(uint2*)(dst + hc) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
}

template <int EPI>
hipError_t launch_small(const GemmArgs& g, hipStream_t st) {
  const int S = EPI == EPI_PART ? g.splits : 1;
  // waves per workgroup: one per 64-K step up to 16 (at least the 4 that run the epilogue)
  const int nwv = max(4, min(GS_WAVES, (g.K / 64) / S));
  const dim3 grid((g.N + 31) / 32, (g.M + 31) / 32, S);
  if (g.a_src) hipLaunchKernelGGL((gemm_small_kernel<true, EPI>), grid, dim3(64 * nwv), 0, st, g);
  else hipLaunchKernelGGL((gemm_small_kernel<false, EPI>), grid, dim3(64 * nwv), 0, st, g);
  return hipGetLastError();
}

}  // namespace

bool gemm_small_fits(const GemmArgs& g, int epi) {
  if (epi == EPI_QKV)
    return g.M > 0 && g.M <= GEMM_SMALL_MAX_M && !g.w_scale && !g.a_src && g.K % 64 == 0 && g.K <= GS_WAVES * 64 &&
           g.qk.H % 64 == 0 && g.N == 3 * g.qk.H && g.lda % 8 == 0 && g.ldb % 8 == 0;
  if (epi == EPI_PART && (g.splits < 1 || g.splits > 4 || g.splits > g.K / 64)) return false;
  return g.M > 0 && g.M <= GEMM_SMALL_MAX_M && !g.w_scale && (epi <= EPI_F32 || epi == EPI_PART || epi == EPI_F16) && g.K % 64 == 0 &&
         g.K <= GS_WAVES * GS_MAXSTEPS * 64 && g.lda % 8 == 0 && g.ldb % 8 == 0 && g.ldc % 4 == 0 &&
         (!g.a_src || g.tapC % 64 == 0);
}

bool gemm_small_part64(const GemmArgs& g) {
  return g.a_src && g.M > 32 && (g.K / 64 + g.splits - 1) / g.splits <= GS_WAVES;
}

hipError_t gemm_small(const GemmArgs& g, int epi, hipStream_t st) {
  if (!gemm_small_fits(g, epi)) return hipErrorInvalidValue;
  if (epi == EPI_PART && gemm_small_part64(g)) {
    const int nwv = max(8, min(GS_WAVES, (g.K / 64 + g.splits - 1) / g.splits));
    const dim3 grid((g.N + 31) / 32, (g.M + 63) / 64, g.splits);
    if (g.a_src) hipLaunchKernelGGL(gemm_small_part64_kernel<true>, grid, dim3(64 * nwv), 0, st, g);
    else hipLaunchKernelGGL(gemm_small_part64_kernel<false>, grid, dim3(64 * nwv), 0, st, g);
    return hipGetLastError();
  }
  switch (epi) {
    case EPI_BF16: return launch_small<EPI_BF16>(g, st);
    case EPI_GELU_BF16: return launch_small<EPI_GELU_BF16>(g, st);
    case EPI_RESID_F16: return launch_small<EPI_RESID_F16>(g, st);
    case EPI_F16: return launch_small<EPI_F16>(g, st);
    case EPI_F32: return launch_small<EPI_F32>(g, st);
    case EPI_PART: return launch_small<EPI_PART>(g, st);
    case EPI_QKV:
      hipLaunchKernelGGL(gemm_small_qkv_kernel, dim3(g.N / 64, (g.M + 31) / 32), dim3(64 * GS_WAVES), 0, st, g);
      return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

}  // namespace t2w
