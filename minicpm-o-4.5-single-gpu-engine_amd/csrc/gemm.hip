// bf16 MFMA GEMM for the DiT linears: C = epilogue(A[M,K] . W[N,K]^T + bias), fp32 accumulation.
//
// CDNA4 design.  A workgroup owns a BM x BN output tile; its waves own WTM x WTN sub-tiles made of
// v_mfma_f32_16x16x32_bf16 blocks (fp8: 32x32x64).  K advances in stages of 64 (128-byte tile rows).  Every stage is copied straight
// from HBM/L2 into LDS with global_load_lds_dwordx4 (no register staging), 16-byte chunks XOR-swizzled by row so that
// the fragment reads of 16 consecutive rows cover all 64 LDS banks.  Two LDS stages: the loads of stage k + 2 are issued
// right after the barrier that retires stage k, and the first fragments of stage k + 1 are read before the last MFMAs
// of stage k, so neither the load latency nor the post-barrier LDS latency sits in front of the matrix pipe.  The
// fragment reads, the loads and the MFMAs of a stage are interleaved one by one (sched_group_barrier).
//
// The two stage buffers are separate __shared__ objects and the K loop is unrolled by two, so every LDS access names
// its buffer at compile time.  Behind one dynamically indexed array the compiler cannot tell the fragment reads of one
// stage from the in-flight DMA into the other and waits for all loads before every read, which serialises loads and
// MFMAs.  For the same reason the loads are issued without a branch: at the end of K the free buffer is refilled with
// the last stage (in bounds, never read).
//
// The weight operand is passed to the MFMA as its "A" side, so a lane ends up holding four consecutive output columns
// of one row.  The epilogue stages each wave's accumulators through LDS and writes whole rows: 32 lanes cover 512
// contiguous bytes of fp32 (or 256 of bf16), with bias, GELU or the gated fp32 residual applied on the way out.
//
// fp8 mode: A and W hold OCP e4m3 codes, so a 128-byte stage row carries 128 K values and the stage is two
// v_mfma_scale_f32_32x32x64_f8f6f4 steps.  The MFMA applies A's MX block scales itself: a lane holds 16 bytes of each
// 32-value K block of its row ([k0 + 16 h, +16) and [k0 + 32 + 16 h, +16) for lane half h) and supplies the scale byte
// of block h, as E8M0.  The scale dwords of a stage (four blocks per row) are loaded with the stage; W's per-channel
// scale multiplies the accumulator in the epilogue.
//
// A operand modes: dense rows, or "taps" rows for the kernel-3 causal convs: row m of A is the three frames starting
// at frame a_src[m] of a frame buffer whose rows are lda wide (no im2col copy in HBM; the host lays the two cached
// frames of every packed row in front of its frames).
#include "common.h"
#include "t2w_internal.h"
#include "gemm_tile.h"

namespace t2w {

int pick_cfg(const GemmArgs& g);

namespace {

// The K loop and epilogue of one tile for the waves of tile type T (stage buffers named at compile time once inlined).
template <typename T, int EPI, int BM, int BN>
__device__ __forceinline__ void tile_body(const GemmArgs& g, uint4* sA0, uint4* sA1, uint4* sB0, uint4* sB1, int m0, int n0) {
  T t(g, m0, n0);

  typename T::acc_t acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int r = 0; r < (int)(sizeof(typename T::acc_t) / 4); ++r) acc[i][j][r] = 0.0f;
  typename T::frag_t af[2][T::TM], bf[2][T::TN];
  uint32_t sd0[T::NSC], sd1[T::NSC];  // fp8: activation scale dwords of the stages in buffers 0 and 1

  const int KT = g.K / T::BKE;
  t.issue(sA0, sB0, sd0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  t.issue(sA1, sB1, sd1, min(1, KT - 1));
  t.frag(sA0, sB0, 0, af[0], bf[0]);
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    t.stage(acc, af, bf, sA0, sB0, sd0, sA1, sB1, kt, KT);
    t.stage(acc, af, bf, sA1, sB1, sd1, sA0, sB0, kt + 1, KT);
  }
  if (kt < KT) t.stage(acc, af, bf, sA0, sB0, sd0, sA1, sB1, kt, KT);

  // retire the tail loads and every wave's last fragment reads before the stage buffers become epilogue slabs
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();
  constexpr int SLAB = 32 * T::WTN / 4;  // float4 per wave slab
  constexpr int CAPA = BM * 8 / SLAB, CAPB = BN * 8 / SLAB;
  static_assert(2 * CAPA + 2 * CAPB >= T::NW, "epilogue slabs do not fit the stage buffers");
  const int w = t.wave;
  float4* st = w < CAPA ? (float4*)sA0 + w * SLAB
             : w < 2 * CAPA ? (float4*)sA1 + (w - CAPA) * SLAB
             : w < 2 * CAPA + CAPB ? (float4*)sB0 + (w - 2 * CAPA) * SLAB
                                   : (float4*)sB1 + (w - 2 * CAPA - CAPB) * SLAB;
  t.template store<EPI>(acc, st, m0, n0);
}

template <int BM, int BN, int WM, int WN, int EPI, bool TAPS, bool FP8>
__global__ void __launch_bounds__(64 * WM * WN) gemm_kernel(GemmArgs g) {
  __shared__ uint4 sA0[BM * 8], sA1[BM * 8], sB0[BN * 8], sB1[BN * 8];

  // XCD-aware order: consecutive workgroups go to different XCDs, so the tiles of one XCD are a contiguous run (they
  // share A rows and W columns in that XCD's L2)
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  const int nblk = gm * gn, full = (nblk / 8) * 8;
  int b = blockIdx.x;
  if (b < full) b = (b % 8) * (nblk / 8) + b / 8;
  // wide grids (more than 8 column tiles, e.g. qkv) walk groups of 4 row tiles column by column, so that the tiles
  // one XCD runs at a time share 4 A row blocks and 8 W column blocks instead of all W columns of one row block
  int mb = b / gn, nb = b % gn;
  if (gn > 8) {
    const int grp = b / (4 * gn), rows = min(4, gm - grp * 4), r = b - grp * 4 * gn;
    mb = grp * 4 + r % rows;
    nb = r / rows;
  }
  const int m0 = mb * BM, n0 = nb * BN;
  if constexpr (BM == 208) {
    // 13 row blocks of 16: the first wave row owns 7 (rows 0..111), the second 6 (rows 112..207); waves w and w + 4
    // share a SIMD, so every SIMD runs 13 row blocks x 4 column blocks.  Both wave types pass the same barriers.
    static_assert(WM == 2 && WN == 4 && BN == 256 && !FP8, "208-row tiles: 2 x 4 waves, bf16");
    if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < WN)
      tile_body<Tile<BM, BN, WM, WN, TAPS, FP8, 7, 0>, EPI, BM, BN>(g, sA0, sA1, sB0, sB1, m0, n0);
    else
      tile_body<Tile<BM, BN, WM, WN, TAPS, FP8, 6, 112>, EPI, BM, BN>(g, sA0, sA1, sB0, sB1, m0, n0);
  } else {
    tile_body<Tile<BM, BN, WM, WN, TAPS, FP8>, EPI, BM, BN>(g, sA0, sA1, sB0, sB1, m0, n0);
  }
}

template <int BM, int BN, int WM, int WN, int EPI, bool TAPS>
hipError_t launch_tile(const GemmArgs& g, hipStream_t st) {
  const int gm = (g.M + BM - 1) / BM, gn = (g.N + BN - 1) / BN;
  if (g.w_scale) {
    if constexpr (BM == 208)
      return hipErrorInvalidValue;  // bf16 only
    else
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, EPI, TAPS, true>), dim3(gm * gn), dim3(64 * WM * WN), 0, st, g);
  } else {
    if constexpr (EPI == EPI_GELU_MX8)
      return hipErrorInvalidValue;  // fp8 output only follows fp8 GEMMs
    else
      hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, EPI, TAPS, false>), dim3(gm * gn), dim3(64 * WM * WN), 0, st, g);
  }
  return hipGetLastError();
}

// g without its first r rows: activation rows (taps: their frame ids; fp8: codes and their scale rows), output rows
// (fp8 output: codes and block scales), qkv rows and slots
template <int EPI>
GemmArgs rows_from(const GemmArgs& g, int r) {
  GemmArgs h = g;
  h.M = g.M - r;
  if (g.a_src) {
    h.a_src = g.a_src + r;
  } else if (g.w_scale) {
    h.A = (const bf16_t*)((const uint8_t*)g.A + (size_t)r * g.lda);
    h.a_scale = g.a_scale + (size_t)r * g.a_sld;
  } else {
    h.A = g.A + (size_t)r * g.lda;
  }
  if (EPI == EPI_F32) {
    h.C = (float*)g.C + (size_t)r * g.ldc;
  } else if (EPI == EPI_GELU_MX8) {
    h.C = (uint8_t*)g.C + (size_t)r * g.ldc;
    h.c_scale = g.c_scale + (size_t)r * g.c_sld;
  } else {
    h.C = (uint16_t*)g.C + (size_t)r * g.ldc;  // bf16 or fp16 rows
  }
  if (EPI == EPI_QKV) {
    h.qk.q_out = g.qk.q_out + (size_t)r * g.qk.H;
    h.qk.slots = g.qk.slots + r;
    if (g.qk.pos) h.qk.pos = g.qk.pos + r;
  }
  return h;
}

// tile configurations: 0 = 128x128 (4 waves of 64x64), 1 = 256x256 (8 waves of 64x128), 2 = 256x128 (8 waves of 64x64),
// 3 = 208x256 (bf16; 8 waves of 112x64 and 96x64)
template <int EPI, bool TAPS>
hipError_t launch_epi(const GemmArgs& g, int cfg, hipStream_t st) {
  const bool by_shape = cfg < 0;
  if (cfg < 0) cfg = pick_cfg(g);
  // A 256x256 grid whose last round would leave most of the 256 CUs idle (the fp8 qkv at 12,800 tokens: 600 tiles =
  // two rounds + 88) runs the rows of its full rounds on 256x256 tiles and the rest on 256x128 tiles, one round of
  // half-size tiles instead of a third round of mostly idle CUs.  The products are the same per output element.
  if (by_shape && cfg == 1) {
    const long gn = (g.N + 255) / 256, tiles = (long)((g.M + 255) / 256) * gn;
    const long rounds = (tiles + 255) / 256, last = tiles - (rounds - 1) * 256;
    const int rows1 = (int)((rounds - 1) * 256 / gn) * 256;
    const long tiles2 = (long)((g.M - rows1 + 255) / 256) * ((g.N + 127) / 128);
    if (rounds >= 2 && 2 * last < 256 && rows1 > 0 && rows1 < g.M && tiles2 <= 256) {
      GemmArgs g1 = g;
      g1.M = rows1;
      const hipError_t e = launch_tile<256, 256, 4, 2, EPI, TAPS>(g1, st);
      if (e != hipSuccess) return e;
      return launch_tile<256, 128, 4, 2, EPI, TAPS>(rows_from<EPI>(g, rows1), st);
    }
  }
  switch (cfg) {
    case 0: return launch_tile<128, 128, 2, 2, EPI, TAPS>(g, st);
    case 1: return launch_tile<256, 256, 4, 2, EPI, TAPS>(g, st);
    case 2: return launch_tile<256, 128, 4, 2, EPI, TAPS>(g, st);
    case 3: return launch_tile<208, 256, 2, 4, EPI, TAPS>(g, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

int pick_cfg(const GemmArgs& g) {
  // 256x256 tiles once there are enough rows to fill them (bf16 and fp8 alike).  qkv (N = 3072) took 256x128 while its
  // epilogue wrote 4 columns per lane (105 us vs 114 at 12800 rows); with 16-byte stores 256x256 is the faster one
  // (DiT solve 132.1 -> 129.6 ms on the same box).  fc1 (N = 2048, GELU) takes 256x256 since its epilogue uses the
  // hardware reciprocal (DiT solve 143.5 -> 142.0 ms against 128x128)
  if (g.M < 1024 || g.N < 256) return 0;
  // A 256x256 grid that fills under 70% of its last round of 256 CUs (prompt setups of 1,000-9,000 tokens) loses to the
  // 128x128 grid when that one's cost is clearly lower.  Measured per round of 256 tiles at K = 1024: 256x256 ~30 us,
  // 128x128 ~7.5 us plus ~7 us once (e.g. 3,000 rows, N = 1024: 26.5 vs 14.0 us; 8,000 rows: 29.4 vs 22.8 us; 12,800
  // rows: 33.2 vs 37.3 us, where the 256x256 grid is 78% full)
  const long t1 = (long)((g.M + 255) / 256) * ((g.N + 255) / 256), t0 = (long)((g.M + 127) / 128) * ((g.N + 127) / 128);
  const long r1 = (t1 + 255) / 256, r0 = (t0 + 255) / 256;
  if (10 * t1 < 7 * 256 * r1 && 75 * r0 + 70 < 270 * r1) return 0;
  // 256x256 wins over 128x128.  The 208x256 tile holds 13/16 of the rows (and MFMA work per SIMD) of a 256x256 one:
  // where its grid needs no more rounds of 256 CUs, every round is shorter.  Measured at 12,800 tokens (us per launch,
  // 256x256 -> 208x256): N = 1024, K = 1024 37.2 -> 35.2 (248 tiles in one round instead of 200 on 200 CUs); taps
  // K = 3072 77.7 -> 72.1; N = 2048 63.8 -> 59.0; N = 3072 89.4 -> 84.5 (three rounds either way; the split into
  // 256x256 and 256x128 tiles in launch_epi: 87.0).  bf16 only (fp8 blocks are 32 rows).
  const long t3 = (long)((g.M + 207) / 208) * ((g.N + 255) / 256), r3 = (t3 + 255) / 256;
  return !g.w_scale && r3 <= r1 ? 3 : 1;
}

bool gemm_splits(const GemmArgs& g) {
  if (!g.ws || g.w_scale || g.M <= 0) return false;
  // a grid of fewer than 128 tiles leaves most of the 256 CUs idle: split K instead
  const int c = pick_cfg(g), bm = c == 0 ? 128 : (c == 3 ? 208 : 256), bn = c == 1 || c == 3 ? 256 : 128;
  const long tiles = (long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
  return tiles < 128 && splitk_plan(g.M, g.N, g.K, g.ws_bytes).splits > 1;
}

hipError_t gemm_bf16(const GemmArgs& g, int epi, hipStream_t st, int cfg) {
  if (g.M <= 0 || g.N <= 0) return hipSuccess;
  // the tile kernels address both operands by 32-bit byte offsets (taps mode: frame rows up to M + 65536)
  const size_t es = g.w_scale ? 1 : 2;
  if ((size_t)(g.M + 65536) * g.lda * es >= ((size_t)1 << 32) || (size_t)g.N * g.ldb * es >= ((size_t)1 << 32))
    return hipErrorInvalidValue;
  if (cfg < 0 && gemm_small_fits(g, epi)) return gemm_small(g, epi, st);
  // the tile epilogues store bf16 rows 16 bytes per lane
  const bool bf16_out = epi == EPI_BF16 || epi == EPI_GELU_BF16 || epi == EPI_RESID_F16 || epi == EPI_F16;  // 16-bit rows
  if (bf16_out && (g.ldc % 8 || ((size_t)g.C & 15)) && !(cfg < 0 && gemm_splits(g))) return hipErrorInvalidValue;
  if (cfg < 0 && gemm_splits(g)) {
    if (epi == EPI_QKV || epi == EPI_GELU_MX8) return hipErrorInvalidValue;  // tile-path epilogues
    return gemm_splitk(g, epi, splitk_plan(g.M, g.N, g.K, g.ws_bytes), g.ws, st);
  }
  const bool taps = g.a_src != nullptr;
  switch (epi * 2 + (taps ? 1 : 0)) {
    case EPI_BF16 * 2: return launch_epi<EPI_BF16, false>(g, cfg, st);
    case EPI_BF16 * 2 + 1: return launch_epi<EPI_BF16, true>(g, cfg, st);
    case EPI_GELU_BF16 * 2: return launch_epi<EPI_GELU_BF16, false>(g, cfg, st);
    case EPI_GELU_BF16 * 2 + 1: return launch_epi<EPI_GELU_BF16, true>(g, cfg, st);
    case EPI_RESID_F16 * 2: return launch_epi<EPI_RESID_F16, false>(g, cfg, st);
    case EPI_RESID_F16 * 2 + 1: return launch_epi<EPI_RESID_F16, true>(g, cfg, st);
    case EPI_F16 * 2: return launch_epi<EPI_F16, false>(g, cfg, st);
    case EPI_F32 * 2: return launch_epi<EPI_F32, false>(g, cfg, st);
    case EPI_F32 * 2 + 1: return launch_epi<EPI_F32, true>(g, cfg, st);
    case EPI_GELU_MX8 * 2:
      if (!g.w_scale || !g.c_scale || g.N % 32) return hipErrorInvalidValue;
      return launch_epi<EPI_GELU_MX8, false>(g, cfg, st);
    case EPI_QKV * 2:
      // the tile epilogue does not rotate q and k (rope_qk after it does): a rotary table here is a caller error
      if (g.N != 3 * g.qk.H || g.qk.H % 256 || g.qk.rfreq) return hipErrorInvalidValue;
      return launch_epi<EPI_QKV, false>(g, cfg, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace t2w
