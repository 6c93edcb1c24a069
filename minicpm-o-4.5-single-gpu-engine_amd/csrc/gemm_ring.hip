// Four-wave bf16 MFMA GEMM with a four-deep LDS ring (the DiT's large projections, >= ~1k rows).
//
// A workgroup of 4 waves owns a 256 x 256 output tile, each wave 128 x 128 (4 x 4 blocks of v_mfma_f32_32x32x16_bf16,
// accumulators in AGPRs).  K advances in stages of 32 values (64 bytes per tile row); the A and B rows of a stage
// (32 KB) arrive by buffer loads straight into LDS (buffer_load_dwordx4 ... lds), and a ring of four stage slots keeps
// three stages in flight ahead of the one being multiplied.  Per stage and wave: 32 MFMAs, 16 fragment reads, 8
// loads, one barrier, laid out by hand in groups of two MFMAs with one fragment read and at most one load each.
// Compared with the eight-wave 64 x 128 layout (gemm.hip) the LDS reads per MFMA drop by a third (128 KB instead of
// 192 KB per 64 K of a tile), which leaves the LDS port slack for the loads.
//
// The loads are inline assembly, so the compiler does not see them as LDS writes: the kernel places every wait on
// them itself (the compiler would otherwise wait for all loads in flight before every fragment read it cannot prove
// disjoint from them).  Buffer offsets are 32-bit: the activation operand must span < 4 GB from its base.
#include "gemm_tile.h"

namespace t2w {

namespace {

constexpr int RBM = 256, RBN = 256, RNW = 4, RWM = 2, RWN = 2, RWT = 128, RTM = 4, RTN = 4;
constexpr int RBK = 32;                // K values per stage
constexpr int RS = 4;                  // ring slots
constexpr int RAPW = RBM / 16 / RNW;   // 1 KB (16-row) load blocks per wave and stage (A); the same for B
constexpr int RLPS = 2 * RAPW;         // loads per thread and stage
constexpr int RSLOT = (RBM + RBN) * 4; // uint4 per slot: A rows, then B rows, 4 chunks of 16 bytes per row

typedef int i32x4 __attribute__((ext_vector_type(4)));

// chunk c (0..3) of row r of a slot lives at chunk c ^ ((r >> 2) & 3): the 16 rows of one 16-lane LDS phase of a
// fragment read then cover all 64 banks
__device__ __forceinline__ int rswz(int r, int c) { return r * 4 + (c ^ ((r >> 2) & 3)); }

// raw buffer resource over [base, base + 4 GB - 1)
__device__ __forceinline__ i32x4 rsrc(const char* base) {
  const uint64_t a = (uint64_t)base;
  i32x4 r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xffffu);
  r[2] = -1;
  r[3] = 0x00020000;
  return r;
}

// 16 bytes per lane from rs + voff into LDS at lds + lane * 16
__device__ __forceinline__ void dma16(i32x4 rs, const uint4* lds, uint32_t voff) {
  const uint32_t la = (uint32_t)(size_t)(__attribute__((address_space(3))) const void*)lds;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(la), "v"(voff), "s"(rs) : "m0");
}

// own loads waited down to N in flight and own LDS reads done (a wait the compiler sees), then the workgroup barrier
// without a fence (a fence would wait for every load in flight)
template <int N>
__device__ __forceinline__ void wait_bar() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70);  // vmcnt(N) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool TAPS>
struct Ring {
  const GemmArgs& g;
  const char* abase;  // dense: the tile's first A row; taps: A itself (rows come from a_src)
  const char* bbase;  // the tile's first B row
  uint32_t aoff[RAPW], boff[RAPW];  // this lane's byte offsets: row of its load block, swizzled 16-byte chunk
  int wave, lane, wm, wn;

  __device__ __forceinline__ Ring(const GemmArgs& g_, int m0, int n0) : g(g_) {
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave / RWN;
    wn = wave % RWN;
    const int lrow = lane >> 2;
    const uint32_t ch = (uint32_t)(((lane & 3) ^ ((lrow >> 2) & 3)) * 16);
    abase = TAPS ? (const char*)g.A : (const char*)(g.A + (size_t)m0 * g.lda);
    bbase = (const char*)(g.B + (size_t)n0 * g.ldb);
#pragma unroll
    for (int p = 0; p < RAPW; ++p) {
      const int trow = (wave + p * RNW) * 16 + lrow;
      const int m = min(m0 + trow, g.M - 1);  // rows past M load row M - 1; their results are never stored
      aoff[p] = (TAPS ? (uint32_t)g.a_src[m] * (uint32_t)g.lda * 2u : (uint32_t)((m - m0) * g.lda * 2)) + ch;
      const int n = min(n0 + trow, g.N - 1);
      boff[p] = (uint32_t)((n - n0) * g.ldb * 2) + ch;
    }
  }

  // one half (A rows, or B rows) of stage kt into slot R: RAPW loads of this thread, load block p
  __device__ __forceinline__ void load_a(uint4* R, int kt, int p) const {
    const int k0 = kt * RBK;
    size_t ko = (size_t)k0 * 2;
    if (TAPS) {
      const int tap = k0 / g.tapC;  // a stage never straddles two taps (tapC % 32 == 0)
      ko = ((size_t)tap * g.lda + (k0 - tap * g.tapC)) * 2;
    }
    dma16(rsrc(abase + ko), R + (wave + p * RNW) * 64, aoff[p]);
  }
  __device__ __forceinline__ void load_b(uint4* R, int kt, int p) const {
    dma16(rsrc(bbase + (size_t)kt * RBK * 2), R + RBM * 4 + (wave + p * RNW) * 64, boff[p]);
  }
  __device__ __forceinline__ void load_stage(uint4* R, int kt) const {
#pragma unroll
    for (int p = 0; p < RAPW; ++p) load_a(R, kt, p);
#pragma unroll
    for (int p = 0; p < RAPW; ++p) load_b(R, kt, p);
  }

  // fragment x (0..3: A block x, 4..7: B block x - 4) of K step kk (0, 1) from slot R
  __device__ __forceinline__ void read1(const uint4* R, int kk, int x, bf16x8 (&af)[RTM], bf16x8 (&bf)[RTN]) const {
    const int chunk = kk * 2 + (lane >> 5);
    if (x < RTM) af[x] = as_bf16x8(R[rswz(wm * RWT + x * 32 + (lane & 31), chunk)]);
    else bf[x - RTM] = as_bf16x8(R[RBM * 4 + rswz(wn * RWT + (x - RTM) * 32 + (lane & 31), chunk)]);
  }

  // Stage kt from slot R (its K step 0 fragments already in af[0], bf[0]).  First half: MFMAs of K step 0, fragment
  // reads of K step 1, and the B rows of stage kt - 1 + RS into slot Rp (refilled since the previous stage); barrier;
  // second half: MFMAs of K step 1, K step 0 fragments of the next slot Rn, and the A rows of stage kt + RS into R.
  // Past the last stage the last stage is loaded again, so that the number of loads in flight never changes.
  __device__ __forceinline__ void stage(f32x16 (&acc)[RTM][RTN], bf16x8 (&af)[2][RTM], bf16x8 (&bf)[2][RTN], uint4* Rp,
                                        uint4* R, const uint4* Rn, int kt, int KT) const {
    const int kb = min(kt - 1 + RS, KT - 1), ka = min(kt + RS, KT - 1);
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      const int q0 = 2 * x, q1 = 2 * x + 1;
      acc[q0 / 4][q0 % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[0][q0 % 4], af[0][q0 / 4], acc[q0 / 4][q0 % 4], 0, 0, 0);
      read1(R, 1, x, af[1], bf[1]);
      acc[q1 / 4][q1 % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[0][q1 % 4], af[0][q1 / 4], acc[q1 / 4][q1 % 4], 0, 0, 0);
      if (kt > 0 && (x & 1)) load_b(Rp, kb, x >> 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    // own loads of stage kt + 1 landed (those of stages kt + 2 .. kt + RS - 1 may be in flight), own reads of R done
    wait_bar<(RS - 2) * RLPS>();
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      const int q0 = 2 * x, q1 = 2 * x + 1;
      acc[q0 / 4][q0 % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[1][q0 % 4], af[1][q0 / 4], acc[q0 / 4][q0 % 4], 0, 0, 0);
      read1(Rn, 0, x, af[0], bf[0]);
      acc[q1 / 4][q1 % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[1][q1 % 4], af[1][q1 / 4], acc[q1 / 4][q1 % 4], 0, 0, 0);
      if (x & 1) load_a(R, ka, x >> 1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
};

template <int EPI, bool TAPS>
__global__ void __launch_bounds__(256) gemm_ring_kernel(GemmArgs g) {
  __shared__ uint4 r0[RSLOT], r1[RSLOT], r2[RSLOT], r3[RSLOT];
  // XCD-aware order: consecutive workgroups go to different XCDs, so the tiles of one XCD are a contiguous run
  const int gm = (g.M + RBM - 1) / RBM, gn = (g.N + RBN - 1) / RBN;
  const int nblk = gm * gn, full = (nblk / 8) * 8;
  int b = blockIdx.x;
  if (b < full) b = (b % 8) * (nblk / 8) + b / 8;
  const int m0 = (b / gn) * RBM, n0 = (b % gn) * RBN;
  const Ring<TAPS> t(g, m0, n0);

  f32x16 acc[RTM][RTN];
#pragma unroll
  for (int i = 0; i < RTM; ++i)
#pragma unroll
    for (int j = 0; j < RTN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  bf16x8 af[2][RTM], bf[2][RTN];
  const int KT = g.K / RBK;  // a multiple of RS
  t.load_stage(r0, 0);
  t.load_stage(r1, 1);
  t.load_stage(r2, 2);
  t.load_stage(r3, 3);
  wait_bar<(RS - 1) * RLPS>();  // stage 0 landed everywhere
#pragma unroll
  for (int x = 0; x < 8; ++x) t.read1(r0, 0, x, af[0], bf[0]);
  for (int kt = 0; kt < KT; kt += RS) {
    t.stage(acc, af, bf, r3, r0, r1, kt, KT);
    t.stage(acc, af, bf, r0, r1, r2, kt + 1, KT);
    t.stage(acc, af, bf, r1, r2, r3, kt + 2, KT);
    t.stage(acc, af, bf, r2, r3, r0, kt + 3, KT);
  }
  // every load (the repeated tail stages included) has landed and every wave is done with the ring: the slots become
  // the epilogue's slabs (16 KB per wave)
  wait_bar<0>();
  float4* st = (float4*)(t.wave < 2 ? r0 : r1) + (t.wave & 1) * (32 * RWT / 4);
  tile_store<EPI, RTM, RTN, RWT, RWT>(g, acc, st, m0 + t.wm * RWT, n0 + t.wn * RWT, t.lane);
}

template <int EPI, bool TAPS>
hipError_t launch_ring(const GemmArgs& g, hipStream_t st) {
  const int nblk = ((g.M + RBM - 1) / RBM) * ((g.N + RBN - 1) / RBN);
  hipLaunchKernelGGL((gemm_ring_kernel<EPI, TAPS>), dim3(nblk), dim3(256), 0, st, g);
  return hipGetLastError();
}

}  // namespace

bool gemm_ring_fits(const GemmArgs& g, int epi) {
  if (g.w_scale || epi == EPI_GELU_MX8) return false;
  if (g.K % (RBK * RS) || g.lda % 8 || g.ldb % 8) return false;
  if (epi == EPI_QKV && (g.N != 3 * g.qk.H || g.qk.H % 256)) return false;
  // 32-bit buffer offsets: taps rows are frames a_src[m] < M + 2 (rows) <= 2 M + 2 of A, dense rows stay in the tile
  const double span = g.a_src ? (2.0 * g.M + 2.0) * g.lda * 2.0 + (double)g.K * 2.0 : 0.0;
  if (span >= 4294967295.0 || (double)RBN * g.ldb * 2.0 >= 4294967295.0) return false;
  if (g.a_src && g.tapC % RBK) return false;
  return true;
}

hipError_t gemm_ring(const GemmArgs& g, int epi, hipStream_t st) {
  if (!gemm_ring_fits(g, epi)) return hipErrorInvalidValue;
  const bool taps = g.a_src != nullptr;
  switch (epi * 2 + (taps ? 1 : 0)) {
    case EPI_BF16 * 2: return launch_ring<EPI_BF16, false>(g, st);
    case EPI_BF16 * 2 + 1: return launch_ring<EPI_BF16, true>(g, st);
    case EPI_GELU_BF16 * 2: return launch_ring<EPI_GELU_BF16, false>(g, st);
    case EPI_GELU_BF16 * 2 + 1: return launch_ring<EPI_GELU_BF16, true>(g, st);
    case EPI_RESID_F32 * 2: return launch_ring<EPI_RESID_F32, false>(g, st);
    case EPI_RESID_F32 * 2 + 1: return launch_ring<EPI_RESID_F32, true>(g, st);
    case EPI_F32 * 2: return launch_ring<EPI_F32, false>(g, st);
    case EPI_F32 * 2 + 1: return launch_ring<EPI_F32, true>(g, st);
    case EPI_QKV * 2: return launch_ring<EPI_QKV, false>(g, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace t2w
