// bf16 MFMA GEMM for the DiT linears: C = epilogue(A[M,K] . W[N,K]^T + bias), fp32 accumulation.
//
// CDNA4 design: v_mfma_f32_32x32x16_bf16 tiles on wave64, LDS-staged A/W tiles of 64 K-values (128 B rows, 16-byte
// chunks XOR-swizzled by row so the fragment reads of 32 consecutive rows spread over all banks), two LDS stages with
// the next tile's global loads in flight during the MFMAs, XCD-aware block order.  The weight operand is passed to the
// MFMA as its "A" side so each lane ends up holding four consecutive output columns (16-byte fp32 / 8-byte bf16
// stores in the epilogue).
//
// A operand modes: dense rows, or "taps" rows for the kernel-3 causal convs: row m of A is the three frames starting
// at frame a_src[m] of a frame buffer whose rows are lda wide (no im2col copy in HBM; the host lays the two cached
// frames of every packed row in front of its frames).
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

int pick_cfg(const GemmArgs& g);

namespace {

constexpr int BK = 64;  // K values per stage (128 bytes of bf16 per tile row)

// 16-byte chunk c of tile row `row` lives at chunk c ^ ((row >> 1) & 7) of that row: 16 consecutive rows reading the same
// chunk (a 16-lane LDS phase of a fragment read) then cover all 64 banks, and 8 consecutive lanes writing one row stay
// within it.
__device__ __forceinline__ int swz_key(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ swz_key(row)); }

template <int EPI>
__device__ __forceinline__ void epilogue4(const GemmArgs& g, int m, int n, float (&v)[4]) {
    if (n + 3 < g.N) {
      const float4 bb = *(const float4*)(g.bias + n);
      v[0] += bb.x; v[1] += bb.y; v[2] += bb.z; v[3] += bb.w;
      if (EPI == EPI_BF16 || EPI == EPI_GELU_BF16) {
        if (EPI == EPI_GELU_BF16) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
        }
        uint2 o = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
        *(uint2*)((bf16_t*)g.C + (size_t)m * g.ldc + n) = o;
      } else if (EPI == EPI_RESID_F32) {
        float* hp = (float*)g.C + (size_t)m * g.ldc + n;
        float4 h = *(float4*)hp;
        const float4 gg = *(const float4*)(g.gate + n);
        h.x += gg.x * v[0]; h.y += gg.y * v[1]; h.z += gg.z * v[2]; h.w += gg.w * v[3];
        *(float4*)hp = h;
      } else {
        *(float4*)((float*)g.C + (size_t)m * g.ldc + n) = make_float4(v[0], v[1], v[2], v[3]);
      }
    } else {
      for (int e = 0; e < 4 && n + e < g.N; ++e) {
        float x = v[e] + g.bias[n + e];
        if (EPI == EPI_BF16) ((bf16_t*)g.C)[(size_t)m * g.ldc + n + e] = f2bf(x);
        else if (EPI == EPI_GELU_BF16) ((bf16_t*)g.C)[(size_t)m * g.ldc + n + e] = f2bf(gelu_tanh(x));
        else if (EPI == EPI_RESID_F32) ((float*)g.C)[(size_t)m * g.ldc + n + e] += g.gate[n + e] * x;
        else ((float*)g.C)[(size_t)m * g.ldc + n + e] = x;
      }
    }
}

template <int BM, int BN, int WM, int WN, int EPI, bool TAPS>
__global__ void __launch_bounds__(64 * WM * WN) gemm_kernel(GemmArgs g) {
  constexpr int NT = 64 * WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;  // 32x32 MFMA blocks per wave
  constexpr int APASS = BM * 8 / NT, BPASS = BN * 8 / NT;
  constexpr int STAGE = (BM + BN) * 8;  // uint4 per LDS stage
  static_assert(APASS * NT == BM * 8 && BPASS * NT == BN * 8, "tile / thread mismatch");

  extern __shared__ uint4 lds_dyn[];  // two stages of STAGE uint4: [A tile BM x 8 | W tile BN x 8]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  const int nblk = gm * gn;
  int b = blockIdx.x;
  const int full = (nblk / 8) * 8;  // blocks b, b+8, .. run on one XCD: give each XCD a contiguous band of tiles
  if (b < full) b = (b % 8) * (nblk / 8) + b / 8;
  const int mt = b / gn, nt = b % gn;
  const int m0 = mt * BM, n0 = nt * BN;

  // per-thread global load sources (rows fixed over the K loop)
  const bf16_t* asrc[APASS];
  bool aok[APASS];
  int arow[APASS], achunk[APASS];
#pragma unroll
  for (int p = 0; p < APASS; ++p) {
    int idx = tid + p * NT;
    arow[p] = idx >> 3;
    achunk[p] = idx & 7;
    int m = m0 + arow[p];
    aok[p] = m < g.M;
    int mm = aok[p] ? m : 0;
    if (TAPS)
      asrc[p] = g.A + (size_t)g.a_src[mm] * g.lda + achunk[p] * 8;
    else
      asrc[p] = g.A + (size_t)mm * g.lda + achunk[p] * 8;
  }
  const bf16_t* bsrc[BPASS];
  bool bok[BPASS];
  int brow[BPASS], bchunk[BPASS];
#pragma unroll
  for (int p = 0; p < BPASS; ++p) {
    int idx = tid + p * NT;
    brow[p] = idx >> 3;
    bchunk[p] = idx & 7;
    int n = n0 + brow[p];
    bok[p] = n < g.N;
    bsrc[p] = g.B + (size_t)(bok[p] ? n : 0) * g.ldb + bchunk[p] * 8;
  }

  uint4 ra[APASS], rb[BPASS];
  auto gload = [&](int k0) {
    size_t aoff;
    if (TAPS) {
      int tap = k0 / g.tapC;
      aoff = (size_t)tap * g.lda + (k0 - tap * g.tapC);
    } else {
      aoff = k0;
    }
#pragma unroll
    for (int p = 0; p < APASS; ++p) ra[p] = aok[p] ? *(const uint4*)(asrc[p] + aoff) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int p = 0; p < BPASS; ++p) rb[p] = bok[p] ? *(const uint4*)(bsrc[p] + k0) : make_uint4(0, 0, 0, 0);
  };
  auto lstore = [&](int s) {
#pragma unroll
    for (int p = 0; p < APASS; ++p) lds_dyn[s * STAGE + swz(arow[p], achunk[p])] = ra[p];
#pragma unroll
    for (int p = 0; p < BPASS; ++p) lds_dyn[s * STAGE + BM * 8 + swz(brow[p], bchunk[p])] = rb[p];
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = g.K / BK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int chunk = kk * 2 + (lane >> 5);
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        int row = wm * WTM + i * 32 + (lane & 31);
        af[i] = as_bf16x8(lds_dyn[s * STAGE + swz(row, chunk)]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        int row = wn * WTN + j * 32 + (lane & 31);
        bfr[j] = as_bf16x8(lds_dyn[s * STAGE + BM * 8 + swz(row, chunk)]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) lstore(s ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds row m = .. + lane%32 and columns n = .. + (r/4)*8 + (lane/32)*4 + r%4
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WTM + i * 32 + (lane & 31);
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WTN + j * 32 + q * 8 + (lane >> 5) * 4;
        if (n >= g.N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][q * 4 + e];
        epilogue4<EPI>(g, m, n, v);
      }
    }
  }
}

// Direct-to-LDS variant: every 16-byte chunk of the next K stage goes from global memory straight into its swizzled
// LDS slot (global_load_lds_dwordx4: a wave writes 1 KB of LDS, lane l at byte 16 l of the block, so each lane loads the
// chunk whose swizzled position is its own), with no VGPR staging; fragments of the next 16-wide K step are read while
// the current one's MFMAs issue.  Rows past M / N are clamped to the last valid row (their results are never stored).
template <int BM, int BN, int WM, int WN, int EPI, bool TAPS>
__global__ void __launch_bounds__(64 * WM * WN) gemm_lds_kernel(GemmArgs g) {
  constexpr int NT = 64 * WM * WN, NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int STAGE = (BM + BN) * 8;        // uint4 per stage
  constexpr int ABLK = BM / 8, BBLK = BN / 8;  // 1 KB blocks (8 rows) per stage
  constexpr int APW = ABLK / NW, BPW = BBLK / NW;
  static_assert(APW * NW == ABLK && BPW * NW == BBLK, "blocks / waves mismatch");
  extern __shared__ uint4 lds_dyn[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  const int nblk = gm * gn;
  int b = blockIdx.x;
  const int full = (nblk / 8) * 8;
  if (b < full) b = (b % 8) * (nblk / 8) + b / 8;
  const int mt = b / gn, nt = b % gn;
  const int m0 = mt * BM, n0 = nt * BN;

  // this lane's source chunk in each of its waves' 1 KB blocks: tile row blk*8 + l/8, logical chunk (l%8) ^ swz_key(row)
  const int lrow = lane >> 3;
  const bf16_t* asrc[APW];
  const bf16_t* bsrc[BPW];
#pragma unroll
  for (int p = 0; p < APW; ++p) {
    const int trow = (wave + p * NW) * 8 + lrow;
    const int lchunk = (lane & 7) ^ swz_key(trow);
    int m = m0 + trow;
    m = m < g.M ? m : g.M - 1;
    asrc[p] = TAPS ? g.A + (size_t)g.a_src[m] * g.lda + lchunk * 8 : g.A + (size_t)m * g.lda + lchunk * 8;
  }
#pragma unroll
  for (int p = 0; p < BPW; ++p) {
    const int trow = (wave + p * NW) * 8 + lrow;
    const int lchunk = (lane & 7) ^ swz_key(trow);
    int n = n0 + trow;
    n = n < g.N ? n : g.N - 1;
    bsrc[p] = g.B + (size_t)n * g.ldb + lchunk * 8;
  }
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  auto issue = [&](int k0, int s) {
    size_t aoff;
    if (TAPS) {
      const int tap = k0 / g.tapC;
      aoff = (size_t)tap * g.lda + (k0 - tap * g.tapC);
    } else {
      aoff = k0;
    }
#pragma unroll
    for (int p = 0; p < APW; ++p)
      __builtin_amdgcn_global_load_lds((const void*)(asrc[p] + aoff), (lds_ptr_t)(lds_dyn + s * STAGE + (wave + p * NW) * 64), 16, 0, 0);
#pragma unroll
    for (int p = 0; p < BPW; ++p)
      __builtin_amdgcn_global_load_lds((const void*)(bsrc[p] + k0), (lds_ptr_t)(lds_dyn + s * STAGE + BM * 8 + (wave + p * NW) * 64), 16, 0, 0);
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = g.K / BK;
  issue(0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int s = kt & 1;
    if (kt + 1 < KT) issue((kt + 1) * BK, s ^ 1);
    const uint4* L = lds_dyn + s * STAGE;
    bf16x8 af[2][TM], bfr[2][TN];
    auto frag = [&](int kk, int buf) {
      const int chunk = kk * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WTM + i * 32 + (lane & 31);
        af[buf][i] = as_bf16x8(L[swz(row, chunk)]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * WTN + j * 32 + (lane & 31);
        bfr[buf][j] = as_bf16x8(L[BM * 8 + swz(row, chunk)]);
      }
    };
    frag(0, 0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      if (kk + 1 < BK / 16) frag(kk + 1, (kk + 1) & 1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[kk & 1][j], af[kk & 1][i], acc[i][j], 0, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WTM + i * 32 + (lane & 31);
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WTN + j * 32 + q * 8 + (lane >> 5) * 4;
        if (n >= g.N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][q * 4 + e];
        epilogue4<EPI>(g, m, n, v);
      }
    }
  }
}

// Deep-pipelined direct-to-LDS variant: K stages of 32 (64-byte tile rows, 16-byte chunk c of row r at chunk
// c ^ ((r >> 2) & 3): 16 consecutive rows reading one chunk cover all 64 banks), an NS-deep LDS ring with the loads of
// stage kt + NS - 1 issued while stage kt computes, and a wait that only requires stage kt's own loads to have landed.
__device__ __forceinline__ int swz32(int row, int chunk) { return row * 4 + (chunk ^ ((row >> 2) & 3)); }

template <int LPT, int NS>
__device__ __forceinline__ void wait_stage(bool tail) {
  // outstanding loads are the stages after this one; vmcnt counts per-thread vector memory instructions in issue order
  if (tail) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    constexpr int N = (NS - 2) * LPT;
    static_assert(N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
  }
}

template <int BM, int BN, int WM, int WN, int NS, int EPI, bool TAPS>
__global__ void __launch_bounds__(64 * WM * WN) gemm_pipe_kernel(GemmArgs g) {
  constexpr int BKP = 32;
  constexpr int NT = 64 * WM * WN, NW = WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int STAGE = (BM + BN) * 4;          // uint4 per stage
  constexpr int ABLK = BM / 16, BBLK = BN / 16;  // 1 KB blocks (16 rows of 64 bytes)
  constexpr int APW = ABLK / NW, BPW = BBLK / NW;
  constexpr int LPT = APW + BPW;
  static_assert(APW * NW == ABLK && BPW * NW == BBLK, "blocks / waves mismatch");
  extern __shared__ uint4 lds_dyn[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  const int nblk = gm * gn;
  int b = blockIdx.x;
  const int full = (nblk / 8) * 8;
  if (b < full) b = (b % 8) * (nblk / 8) + b / 8;
  const int mt = b / gn, nt = b % gn;
  const int m0 = mt * BM, n0 = nt * BN;

  const int lrow = lane >> 2;  // row of the lane's chunk inside its 1 KB block (16 rows x 4 chunks)
  const bf16_t* asrc[APW];
  const bf16_t* bsrc[BPW];
#pragma unroll
  for (int p = 0; p < APW; ++p) {
    const int trow = (wave + p * NW) * 16 + lrow;
    const int lchunk = (lane & 3) ^ ((trow >> 2) & 3);
    int m = m0 + trow;
    m = m < g.M ? m : g.M - 1;
    asrc[p] = TAPS ? g.A + (size_t)g.a_src[m] * g.lda + lchunk * 8 : g.A + (size_t)m * g.lda + lchunk * 8;
  }
#pragma unroll
  for (int p = 0; p < BPW; ++p) {
    const int trow = (wave + p * NW) * 16 + lrow;
    const int lchunk = (lane & 3) ^ ((trow >> 2) & 3);
    int n = n0 + trow;
    n = n < g.N ? n : g.N - 1;
    bsrc[p] = g.B + (size_t)n * g.ldb + lchunk * 8;
  }
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  const int KT = g.K / BKP;
#define T2W_ISSUE(kt_)                                                                                                          \
  {                                                                                                                             \
    const int k0 = (kt_) * BKP;                                                                                                 \
    const int s_ = (kt_) % NS;                                                                                                  \
    size_t aoff;                                                                                                                \
    if (TAPS) {                                                                                                                 \
      const int tap = k0 / g.tapC;                                                                                              \
      aoff = (size_t)tap * g.lda + (k0 - tap * g.tapC);                                                                         \
    } else {                                                                                                                    \
      aoff = k0;                                                                                                                \
    }                                                                                                                           \
    _Pragma("unroll") for (int p = 0; p < APW; ++p) __builtin_amdgcn_global_load_lds(                                           \
        (const void*)(asrc[p] + aoff), (lds_ptr_t)(lds_dyn + s_ * STAGE + (wave + p * NW) * 64), 16, 0, 0);                      \
    _Pragma("unroll") for (int p = 0; p < BPW; ++p) __builtin_amdgcn_global_load_lds(                                           \
        (const void*)(bsrc[p] + k0), (lds_ptr_t)(lds_dyn + s_ * STAGE + BM * 4 + (wave + p * NW) * 64), 16, 0, 0);               \
  }

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < KT) T2W_ISSUE(p)
  for (int kt = 0; kt < KT; ++kt) {
    wait_stage<LPT, NS>(kt + NS - 2 >= KT);
    __syncthreads();  // stage kt landed for every thread; stage kt - 1 (about to be refilled) is no longer read
    if (kt + NS - 1 < KT) T2W_ISSUE(kt + NS - 1)
    const uint4* L = lds_dyn + (kt % NS) * STAGE;
    bf16x8 af[2][TM], bfr[2][TN];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int chunk = kk * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TM; ++i) af[kk][i] = as_bf16x8(L[swz32(wm * WTM + i * 32 + (lane & 31), chunk)]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[kk][j] = as_bf16x8(L[BM * 4 + swz32(wn * WTN + j * 32 + (lane & 31), chunk)]);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[kk][j], af[kk][i], acc[i][j], 0, 0, 0);
  }
#undef T2W_ISSUE

#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * WTM + i * 32 + (lane & 31);
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WTN + j * 32 + q * 8 + (lane >> 5) * 4;
        if (n >= g.N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][q * 4 + e];
        epilogue4<EPI>(g, m, n, v);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int EPI, bool TAPS>
hipError_t launch_cfg(const GemmArgs& g, hipStream_t st) {
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  const size_t lds = 2 * (size_t)(BM + BN) * 8 * sizeof(uint4);
  auto kern = gemm_kernel<BM, BN, WM, WN, EPI, TAPS>;
  static bool attr_set = false;  // one attribute call per instantiation (host side, idempotent)
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(gm * gn), dim3(64 * WM * WN), lds, st, g);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int EPI, bool TAPS>
hipError_t launch_lds(const GemmArgs& g, hipStream_t st) {
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  const size_t lds = 2 * (size_t)(BM + BN) * 8 * sizeof(uint4);
  auto kern = gemm_lds_kernel<BM, BN, WM, WN, EPI, TAPS>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(gm * gn), dim3(64 * WM * WN), lds, st, g);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int NS, int EPI, bool TAPS>
hipError_t launch_pipe(const GemmArgs& g, hipStream_t st) {
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  const size_t lds = (size_t)NS * (BM + BN) * 4 * sizeof(uint4);
  auto kern = gemm_pipe_kernel<BM, BN, WM, WN, NS, EPI, TAPS>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(gm * gn), dim3(64 * WM * WN), lds, st, g);
  return hipGetLastError();
}

// tile configurations: 0 = 128x128 (4 waves of 64x64), 1 = 256x128 (4 waves of 128x64), 2 = 128x256 (4 waves of 64x128),
// 3 = 256x256 (4 waves of 128x128), 4 = 256x256 (8 waves of 128x64)
template <int EPI, bool TAPS>
hipError_t launch_epi(const GemmArgs& g, int cfg, hipStream_t st) {
  if (cfg < 0) cfg = pick_cfg(g);
  switch (cfg) {
    case 0: return launch_cfg<128, 128, 2, 2, EPI, TAPS>(g, st);
    case 1: return launch_cfg<256, 128, 2, 2, EPI, TAPS>(g, st);
    case 2: return launch_cfg<128, 256, 2, 2, EPI, TAPS>(g, st);
    case 3: return launch_cfg<256, 256, 2, 2, EPI, TAPS>(g, st);
    case 4: return launch_cfg<256, 256, 2, 4, EPI, TAPS>(g, st);
    case 5: return launch_lds<256, 256, 2, 4, EPI, TAPS>(g, st);
    case 6: return launch_lds<256, 256, 2, 2, EPI, TAPS>(g, st);
    case 7: return launch_lds<256, 128, 2, 2, EPI, TAPS>(g, st);
    case 8: return launch_lds<128, 128, 2, 2, EPI, TAPS>(g, st);
    case 9: return launch_lds<256, 256, 4, 2, EPI, TAPS>(g, st);
    case 10: return launch_pipe<256, 256, 4, 2, 4, EPI, TAPS>(g, st);
    case 11: return launch_pipe<256, 256, 2, 2, 4, EPI, TAPS>(g, st);
    case 12: return launch_pipe<256, 256, 4, 2, 3, EPI, TAPS>(g, st);
    case 13: return launch_pipe<256, 128, 4, 2, 4, EPI, TAPS>(g, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

int pick_cfg(const GemmArgs& g) {
  // 256x256 tiles of 8 waves (64x128 per wave) with direct-to-LDS loads once there are enough rows to fill them
  if (g.M >= 1024 && g.N >= 256) return 9;
  return 8;
}

hipError_t gemm_bf16(const GemmArgs& g, int epi, hipStream_t st, int cfg) {
  if (g.M <= 0 || g.N <= 0) return hipSuccess;
  const bool taps = g.a_src != nullptr;
  switch (epi * 2 + (taps ? 1 : 0)) {
    case EPI_BF16 * 2: return launch_epi<EPI_BF16, false>(g, cfg, st);
    case EPI_BF16 * 2 + 1: return launch_epi<EPI_BF16, true>(g, cfg, st);
    case EPI_GELU_BF16 * 2: return launch_epi<EPI_GELU_BF16, false>(g, cfg, st);
    case EPI_GELU_BF16 * 2 + 1: return launch_epi<EPI_GELU_BF16, true>(g, cfg, st);
    case EPI_RESID_F32 * 2: return launch_epi<EPI_RESID_F32, false>(g, cfg, st);
    case EPI_RESID_F32 * 2 + 1: return launch_epi<EPI_RESID_F32, true>(g, cfg, st);
    case EPI_F32 * 2: return launch_epi<EPI_F32, false>(g, cfg, st);
    case EPI_F32 * 2 + 1: return launch_epi<EPI_F32, true>(g, cfg, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace t2w
