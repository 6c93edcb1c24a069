// The eight-wave tile machinery of the bf16 / fp8 MFMA GEMM (gemm.hip): LDS swizzle, epilogue columns and the Tile
// (loads, fragments, MFMAs, K stage), and the row-coalesced epilogue tile_store.
#pragma once

#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

constexpr int BK = 64;  // K values per stage (128 bytes of bf16 per tile row)

// 16-byte chunk c of tile row `row` lives at chunk c ^ ((row >> 1) & 7) of that row: 16 consecutive rows reading the same
// chunk (a 16-lane LDS phase of a fragment read) then cover all 64 banks, and 8 consecutive lanes writing one row stay
// within it.
__device__ __forceinline__ int swz_key(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ swz_key(row)); }

// Output columns n .. n + 3 of one lane: bias (and gate) loaded once, before any output row is touched.  SC: the fp8
// tiles, whose weights carry per-channel scales; elsewhere the scale is the constant 1 and its multiply folds away --
// except for fp16 outputs, where acc * scale + bias and the fp16 conversion stay one mixed-precision FMA with a single
// rounding (a plain fp32 add would round twice)
template <int EPI, bool SC0>
struct Cols {
  static constexpr bool SC = SC0 || EPI == EPI_F16;
  float4 bias, gate, wsc;
  int n;
  bool full;  // all four columns inside N
  int act;
  __device__ __forceinline__ Cols(const GemmArgs& g, int n_) : n(n_), full(n_ + 3 < g.N), act(EPI == EPI_BF16 ? g.act : 0) {
    bias = gate = make_float4(0.f, 0.f, 0.f, 0.f);
    wsc = make_float4(1.f, 1.f, 1.f, 1.f);
    if (full) {
      bias = *(const float4*)(g.bias + n);
      if (EPI == EPI_RESID_F16) gate = *(const float4*)(g.gate + n);
      if (SC && g.w_scale) wsc = *(const float4*)(g.w_scale + n);
    }
  }
  // finished output of accumulator values a for full columns (h: the residual row's current values)
  __device__ __forceinline__ float4 apply(float4 a, float4 h) const {
    float v[4] = {a.x * wsc.x + bias.x, a.y * wsc.y + bias.y, a.z * wsc.z + bias.z, a.w * wsc.w + bias.w};
    if (EPI == EPI_GELU_BF16 || EPI == EPI_GELU_MX8) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
    }
    if (EPI == EPI_BF16 && act) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = act_apply(v[e], act);
    }
    if (EPI == EPI_RESID_F16) return make_float4(h.x + gate.x * v[0], h.y + gate.y * v[1], h.z + gate.z * v[2], h.w + gate.w * v[3]);
    return make_float4(v[0], v[1], v[2], v[3]);
  }
  __device__ __forceinline__ void put(const GemmArgs& g, int m, float4 o) const {
    if (EPI == EPI_BF16 || EPI == EPI_GELU_BF16)
      *(uint2*)((bf16_t*)g.C + (size_t)m * g.ldc + n) = make_uint2(pack2(o.x, o.y), pack2(o.z, o.w));
    else if (EPI == EPI_RESID_F16 || EPI == EPI_F16)
      *(uint2*)((f16_t*)g.C + (size_t)m * g.ldc + n) = make_uint2(pack2h(o.x, o.y), pack2h(o.z, o.w));
    else
      *(float4*)((float*)g.C + (size_t)m * g.ldc + n) = o;
  }
  // columns past N: element by element
  __device__ __forceinline__ void put_partial(const GemmArgs& g, int m, float4 a) const {
    const float v[4] = {a.x, a.y, a.z, a.w};
    for (int e = 0; e < 4 && n + e < g.N; ++e) {
      const float x = v[e] * (SC && g.w_scale ? g.w_scale[n + e] : 1.0f) + g.bias[n + e];
      const size_t o = (size_t)m * g.ldc + n + e;
      if (EPI == EPI_BF16) ((bf16_t*)g.C)[o] = f2bf(act_apply(x, act));
      else if (EPI == EPI_GELU_BF16) ((bf16_t*)g.C)[o] = f2bf(gelu_tanh(x));
      else if (EPI == EPI_RESID_F16) ((f16_t*)g.C)[o] = f2h(h2f(((const f16_t*)g.C)[o]) + g.gate[n + e] * x);
      else if (EPI == EPI_F16) ((f16_t*)g.C)[o] = f2h(x);
      else ((float*)g.C)[o] = x;
    }
  }
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ i32x8 join8(uint4 a, uint4 b) {
  i32x8 r;
  r[0] = (int)a.x; r[1] = (int)a.y; r[2] = (int)a.z; r[3] = (int)a.w;
  r[4] = (int)b.x; r[5] = (int)b.y; r[6] = (int)b.z; r[7] = (int)b.w;
  return r;
}

template <bool FP8>
struct FragT { typedef bf16x8 type; };
template <>
struct FragT<true> { typedef i32x8 type; };
template <int MBE>
struct AccT { typedef f32x16 type; };
template <>
struct AccT<16> { typedef f32x4 type; };

// Writes one wave's accumulators (a WTM x WTN block at rows mw.., columns nw..; acc[i][j] = MFMA block (i, j) of edge
// MBE: for 32 x 32 blocks lane l holds column nw + j * 32 + q * 8 + (l / 32) * 4 + (0..3) of row mw + i * 32 + l % 32 in
// registers q * 4 .., for 16 x 16 blocks columns nw + j * 16 + (l / 16) * 4 + (0..3) of row mw + i * 16 + l % 16) through
// its LDS slab st (32 x WTN fp32, 16-byte chunks XOR-swizzled by row) so that each global access of the epilogue covers
// whole rows.  bf16 and fp16 outputs go out 16 bytes per lane (8 columns; the fp16 residual's rows of a batch are all
// loaded before its first store); fp32 outputs 4 columns per lane.  16-byte outputs need ldc % 8 == 0 and a 16-byte
// aligned C (gemm_bf16 checks).
template <int EPI, int MBE, int TM, int TN, int WTM, int WTN, typename AccT>
__device__ __forceinline__ void tile_store(const GemmArgs& g, const AccT (&acc)[TM][TN], float4* st, int mw, int nw, int lane) {
  constexpr int CPR = WTN / 4;   // 16-byte chunks per slab row
  constexpr int RPI = 64 / CPR;  // slab rows per read-back instruction
  constexpr int NRB = 32 / RPI;  // read-back instructions per slab
  constexpr int RB = NRB < 8 ? NRB : 8;
  constexpr bool WIDE = (EPI == EPI_BF16 || EPI == EPI_GELU_BF16 || EPI == EPI_QKV || EPI == EPI_RESID_F16 || EPI == EPI_F16) &&
                        WTN % 8 == 0;
  constexpr int CW = WTN / 8, RW = 64 / CW;  // wide: lanes per slab row, slab rows per instruction
  const int cc = WIDE ? (lane % CW) * 2 : lane % CPR;
  constexpr bool SC = MBE == 32;  // the fp8 tiles (32 x 32 blocks) are the scaled ones
  const Cols<EPI, SC> cols(g, nw + cc * 4);
  const Cols<EPI, SC> cols2(g, nw + cc * 4 + 4);  // wide: the lane's second four columns
  // EPI_QKV: this lane's part (q, k, v), column and head offset, and the LayerNorm affine of its four columns
  int qpart = 0, qcol = 0;
  float4 qlw = make_float4(0.f, 0.f, 0.f, 0.f), qlb = qlw, qlw2 = qlw, qlb2 = qlw;  // wide: 8 columns
  if constexpr (EPI == EPI_QKV) {
    qpart = cols.n / g.qk.H;
    qcol = cols.n - qpart * g.qk.H;
    if (qpart < 2) {
      qlw = *(const float4*)((qpart ? g.qk.kw : g.qk.qw) + (qcol & 63));
      qlb = *(const float4*)((qpart ? g.qk.kb : g.qk.qb) + (qcol & 63));
      if (WIDE) {
        qlw2 = *(const float4*)((qpart ? g.qk.kw : g.qk.qw) + (qcol & 63) + 4);
        qlb2 = *(const float4*)((qpart ? g.qk.kb : g.qk.qb) + (qcol & 63) + 4);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < (WTM + 31) / 32; ++i) {  // one 32-row slab at a time (bf16: the last may hold 16 rows)
    const int nrow = (i + 1) * 32 <= WTM ? 32 : 16;  // rows of this slab (a constant once unrolled)
    if constexpr (MBE == 32) {
      const int r = lane & 31;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = j * 8 + q * 2 + (lane >> 5);
          st[r * CPR + (c ^ (r & (CPR - 1)))] =
              make_float4(acc[i][j][q * 4], acc[i][j][q * 4 + 1], acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
        }
    } else {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        if (2 * i + a >= TM) break;
        const int r = a * 16 + (lane & 15);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int c = j * 4 + (lane >> 4);
          st[r * CPR + (c ^ (r & (CPR - 1)))] = make_float4(acc[2 * i + a][j][0], acc[2 * i + a][j][1], acc[2 * i + a][j][2], acc[2 * i + a][j][3]);
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (WIDE && EPI == EPI_QKV) {
      // the 8 lanes holding one row's 64 columns of one head (heads are 64-aligned in the tile): bias, bf16 rounding,
      // LayerNorm + affine for q and k (sums over the 8 lanes), q to its row, k and v to the token's key slot; the
      // batch's slot ids are loaded before its first store
      constexpr int NB = 32 / RW;
      const QkvOut& o = g.qk;
      float4 a0[NB], a1[NB];
      int slot[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b * RW >= nrow) break;
        const int row = b * RW + lane / CW;
        const int m = mw + i * 32 + row;
        a0[b] = st[row * CPR + (cc ^ (row & (CPR - 1)))];
        a1[b] = st[row * CPR + ((cc + 1) ^ (row & (CPR - 1)))];
        slot[b] = qpart > 0 && m < g.M ? o.slots[m] : 0;
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b * RW >= nrow) break;
        const int m = mw + i * 32 + b * RW + lane / CW;
        float y[8] = {a0[b].x * cols.wsc.x + cols.bias.x, a0[b].y * cols.wsc.y + cols.bias.y,
                      a0[b].z * cols.wsc.z + cols.bias.z, a0[b].w * cols.wsc.w + cols.bias.w,
                      a1[b].x * cols2.wsc.x + cols2.bias.x, a1[b].y * cols2.wsc.y + cols2.bias.y,
                      a1[b].z * cols2.wsc.z + cols2.bias.z, a1[b].w * cols2.wsc.w + cols2.bias.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = bf2f(f2bf(y[e]));  // the projection is rounded to bf16 first
        if (qpart < 2) {
          float sm = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) sm += y[e];
          sm = sum8(sm);
          const float mean = sm * (1.0f / 64.0f);
          float q = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) { y[e] -= mean; q += y[e] * y[e]; }
          q = sum8(q);
          const float rstd = rsqrtf(q * (1.0f / 64.0f) + o.eps);
          const float lw[8] = {qlw.x, qlw.y, qlw.z, qlw.w, qlw2.x, qlw2.y, qlw2.z, qlw2.w};
          const float lb[8] = {qlb.x, qlb.y, qlb.z, qlb.w, qlb2.x, qlb2.y, qlb2.z, qlb2.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] = y[e] * rstd * lw[e] + lb[e];
        }
        if (m < g.M) {
          bf16_t* dst = qpart == 0 ? o.q_out + (size_t)m * o.H : (qpart == 1 ? o.k_pool : o.v_pool) + (size_t)slot[b] * o.H;
          *(uint4*)(dst + qcol) = make_uint4(pack2(y[0], y[1]), pack2(y[2], y[3]), pack2(y[4], y[5]), pack2(y[6], y[7]));
        }
      }
    } else if constexpr (WIDE) {
      constexpr int NB = 32 / RW;
      uint4 hv[NB];  // EPI_RESID_F16: the residual's current 8 values of each row of the batch, loaded up front
      if constexpr (EPI == EPI_RESID_F16) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          if (b * RW >= nrow) break;
          const int m = mw + i * 32 + b * RW + lane / CW;
          hv[b] = make_uint4(0u, 0u, 0u, 0u);
          if (m < g.M && cols2.full) hv[b] = *(const uint4*)((const f16_t*)g.C + (size_t)m * g.ldc + cols.n);
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b * RW >= nrow) break;
        const int row = b * RW + lane / CW;
        const int m = mw + i * 32 + row;
        const float4 v0 = st[row * CPR + (cc ^ (row & (CPR - 1)))];
        const float4 v1 = st[row * CPR + ((cc + 1) ^ (row & (CPR - 1)))];
        if (m >= g.M) continue;
        if (cols2.full) {
          if constexpr (EPI == EPI_RESID_F16 || EPI == EPI_F16) {
            float4 h0 = v0, h1 = v1;
            if constexpr (EPI == EPI_RESID_F16) {
              h0 = make_float4(lo2h(hv[b].x), hi2h(hv[b].x), lo2h(hv[b].y), hi2h(hv[b].y));
              h1 = make_float4(lo2h(hv[b].z), hi2h(hv[b].z), lo2h(hv[b].w), hi2h(hv[b].w));
            }
            const float4 o0 = cols.apply(v0, h0), o1 = cols2.apply(v1, h1);
            *(uint4*)((f16_t*)g.C + (size_t)m * g.ldc + cols.n) =
                make_uint4(pack2h(o0.x, o0.y), pack2h(o0.z, o0.w), pack2h(o1.x, o1.y), pack2h(o1.z, o1.w));
          } else {
            const float4 o0 = cols.apply(v0, v0), o1 = cols2.apply(v1, v1);
            *(uint4*)((bf16_t*)g.C + (size_t)m * g.ldc + cols.n) =
                make_uint4(pack2(o0.x, o0.y), pack2(o0.z, o0.w), pack2(o1.x, o1.y), pack2(o1.z, o1.w));
          }
        } else {
          cols.put_partial(g, m, v0);
          cols2.put_partial(g, m, v1);
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < NRB; b += RB) {
        if (b * RPI >= nrow) break;
        float4 v[RB], h[RB];
        int m[RB], slot[RB];
#pragma unroll
        for (int x = 0; x < RB; ++x) {
          if ((b + x) * RPI >= nrow) break;
          const int row = (b + x) * RPI + lane / CPR;
          m[x] = mw + i * 32 + row;
          v[x] = st[row * CPR + (cc ^ (row & (CPR - 1)))];
          h[x] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (EPI == EPI_RESID_F16 && cols.full && m[x] < g.M) {
            const uint2 hw = *(const uint2*)((const f16_t*)g.C + (size_t)m[x] * g.ldc + cols.n);
            h[x] = make_float4(lo2h(hw.x), hi2h(hw.x), lo2h(hw.y), hi2h(hw.y));
          }
          slot[x] = 0;
          if (EPI == EPI_QKV && qpart > 0 && m[x] < g.M) slot[x] = g.qk.slots[m[x]];
        }
#pragma unroll
        for (int x = 0; x < RB; ++x) {
          if ((b + x) * RPI >= nrow) break;
          if constexpr (EPI == EPI_QKV) {
            // the 16 lanes (one DPP row) holding this row's 64 columns of one head: heads are 64-aligned in the tile
            const QkvOut& o = g.qk;
            float y[4] = {v[x].x * cols.wsc.x + cols.bias.x, v[x].y * cols.wsc.y + cols.bias.y,
                          v[x].z * cols.wsc.z + cols.bias.z, v[x].w * cols.wsc.w + cols.bias.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = bf2f(f2bf(y[e]));  // the projection is rounded to bf16 first
            if (qpart < 2) {
              const float mean = row16_sum(y[0] + y[1] + y[2] + y[3]) * (1.0f / 64.0f);
              float q = 0.f;
#pragma unroll
              for (int e = 0; e < 4; ++e) { y[e] -= mean; q += y[e] * y[e]; }
              const float rstd = rsqrtf(row16_sum(q) * (1.0f / 64.0f) + o.eps);
              y[0] = y[0] * rstd * qlw.x + qlb.x;
              y[1] = y[1] * rstd * qlw.y + qlb.y;
              y[2] = y[2] * rstd * qlw.z + qlb.z;
              y[3] = y[3] * rstd * qlw.w + qlb.w;
            }
            if (m[x] < g.M) {
              bf16_t* dst = qpart == 0 ? o.q_out + (size_t)m[x] * o.H : (qpart == 1 ? o.k_pool : o.v_pool) + (size_t)slot[x] * o.H;
              *(uint2*)(dst + qcol) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
            }
          } else if constexpr (EPI == EPI_GELU_MX8) {
            // the 8 lanes holding this row's 32 consecutive columns share one block scale (N % 32 == 0)
            const float4 o = cols.apply(v[x], h[x]);
            float a = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
            a = max8(a);
            const int se = mx_exp(a);
            if (m[x] < g.M && cols.full) {
              *(uint32_t*)((uint8_t*)g.C + (size_t)m[x] * g.ldc + cols.n) = mx_pack4(o.x, o.y, o.z, o.w, se);
              if ((cc & 7) == 0) g.c_scale[(size_t)m[x] * g.c_sld + (cols.n >> 5)] = (uint8_t)(se + 127);
            }
          } else {
            if (m[x] >= g.M) continue;
            if (cols.full) cols.put(g, m[x], cols.apply(v[x], h[x]));
            else cols.put_partial(g, m[x], v[x]);
          }
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// TMX > 0: an uneven row split (bf16 only): this wave type owns TMX 16-row blocks from tile row ROW0 (the kernel
// instantiates one Tile per wave row and picks by wave), e.g. a 208-row tile as 112 + 96 rows
template <int BM, int BN, int WM, int WN, bool TAPS, bool FP8, int TMX = 0, int ROW0 = 0>
struct Tile {
  static constexpr int NW = WM * WN;
  // bf16 runs v_mfma_f32_16x16x32_bf16 blocks (same bytes per FLOP as 32x32x16, measured ~10% faster next to the
  // stage's global->LDS traffic), fp8 the scaled 32x32x64 blocks
  static constexpr int MBE = FP8 ? 32 : 16;           // MFMA block edge
  static constexpr int WTM = TMX ? TMX * MBE : BM / WM, WTN = BN / WN;  // wave sub-tile
  static constexpr int TM = WTM / MBE, TN = WTN / MBE;  // MFMA blocks per wave
  // 1 KB (8-row) load blocks per stage and wave; A rows past the last whole round (BM = 208: 16 rows) go two per wave
  // as one 4-byte-per-lane load (every wave issues the same loads, so no branch splits the interleaved stage)
  static constexpr int APW = BM / 8 / NW, BPW = BN / 8 / NW;
  static constexpr int AREMR = BM - APW * NW * 8;  // A rows of the remainder
  static constexpr bool AREM = AREMR != 0;
  static constexpr int ES = FP8 ? 1 : 2;              // bytes per element
  static constexpr int BKE = BK * 2 / ES;             // K values per 128-byte stage row
  static constexpr int NKK = 2;                       // MFMA K steps per stage (32 bf16 or 64 fp8 values each)
  static constexpr int NSC = FP8 ? TM : 1;            // scale dwords per lane and stage
  static_assert((AREMR == 0 || AREMR == 2 * NW) && BPW * NW * 8 == BN, "tile rows / waves mismatch");
  static_assert(WTM % 32 == 0 || (!FP8 && WTM % 16 == 0), "the epilogue works in 32-row slabs (bf16: a last 16-row one)");
  static_assert(TMX == 0 || !FP8, "uneven row splits are bf16 only");
  typedef typename FragT<FP8>::type frag_t;
  typedef typename AccT<MBE>::type acc_t;

  // byte offsets of this lane's load rows from g.A / g.B (32-bit: gemm_bf16 keeps both operands under 4 GB), so the
  // loads take the operand base from scalar registers
  uint32_t asrc[APW];
  uint32_t bsrc[BPW];
  uint32_t arem;  // the remainder rows: this lane's 4 bytes
  const uint8_t* sbase[NSC];  // fp8: this lane's activation rows' scale rows
  const GemmArgs& g;
  int lane, wave, wm, wn;
  int mrow;  // this wave's first tile row

  __device__ __forceinline__ Tile(const GemmArgs& g_, int m0, int n0) : g(g_) {
    const int tid = threadIdx.x;
    lane = tid & 63;
    wave = tid >> 6;
    wm = wave / WN;
    wn = wave % WN;
    mrow = TMX ? ROW0 : wm * WTM;
    // this lane's 16 bytes of each of its wave's load blocks: tile row blk * 8 + lane / 8, logical chunk (lane % 8) ^ key
    const int lrow = lane >> 3;
#pragma unroll
    for (int p = 0; p < APW; ++p) {
      const int trow = (wave + p * NW) * 8 + lrow;
      const int m = min(m0 + trow, g.M - 1);  // rows past M load row M - 1; their results are never stored
      const int ch = (lane & 7) ^ swz_key(trow);
      asrc[p] = (uint32_t)(TAPS ? g.a_src[m] : m) * (uint32_t)(g.lda * ES) + ch * 16;
    }
    if constexpr (AREM) {
      // wave w loads rows APW NW 8 + 2 w and + 1: lane l the 4 bytes at LDS chunk position (l % 32) / 4 of row
      // + l / 32, i.e. logical chunk position ^ key
      const int trow = APW * NW * 8 + 2 * wave + (lane >> 5);
      const int m = min(m0 + trow, g.M - 1);
      const int ch = ((lane & 31) >> 2) ^ swz_key(trow);
      arem = (uint32_t)(TAPS ? g.a_src[m] : m) * (uint32_t)(g.lda * ES) + ch * 16 + (lane & 3) * 4;
    }
#pragma unroll
    for (int p = 0; p < BPW; ++p) {
      const int trow = (wave + p * NW) * 8 + lrow;
      bsrc[p] = (uint32_t)min(n0 + trow, g.N - 1) * (uint32_t)(g.ldb * ES) + ((lane & 7) ^ swz_key(trow)) * 16;
    }
    if (FP8) {
#pragma unroll
      for (int i = 0; i < NSC; ++i) {
        const int m = min(m0 + mrow + i * 32 + (lane & 31), g.M - 1);
        sbase[i] = g.a_scale + (size_t)(TAPS ? g.a_src[m] : m) * g.a_sld;
      }
    }
  }

  // loads of stage kt into (la, lb) and, in fp8 mode, its activation scale dwords into sd
  __device__ __forceinline__ void issue(uint4* la, uint4* lb, uint32_t (&sd)[NSC], int kt) const {
    const int k0 = kt * BKE;
    size_t aoff = (size_t)k0 * ES;
    int srow = 0, sblk = k0 / 32;
    if (TAPS) {
      const int tap = k0 / g.tapC;  // a stage never straddles two taps (tapC % BKE == 0)
      aoff = ((size_t)tap * g.lda + (k0 - tap * g.tapC)) * ES;
      srow = tap;
      sblk = (k0 - tap * g.tapC) / 32;
    }
    const uint8_t* A = (const uint8_t*)g.A;
    const uint8_t* B = (const uint8_t*)g.B;
    if constexpr (AREM)
      __builtin_amdgcn_global_load_lds((const void*)(A + (arem + (uint32_t)aoff)), (lds_ptr_t)(la + (APW * NW * 8 + 2 * wave) * 8), 4, 0, 0);
#pragma unroll
    for (int p = 0; p < APW; ++p)
      __builtin_amdgcn_global_load_lds((const void*)(A + (asrc[p] + (uint32_t)aoff)), (lds_ptr_t)(la + (wave + p * NW) * 64), 16, 0, 0);
#pragma unroll
    for (int p = 0; p < BPW; ++p)
      __builtin_amdgcn_global_load_lds((const void*)(B + (bsrc[p] + (uint32_t)(k0 * ES))), (lds_ptr_t)(lb + (wave + p * NW) * 64), 16, 0, 0);
    if (FP8) {
#pragma unroll
      for (int i = 0; i < NSC; ++i) sd[i] = *(const uint32_t*)(sbase[i] + (size_t)srow * g.a_sld + sblk);
    }
  }

  __device__ __forceinline__ void frag(const uint4* La, const uint4* Lb, int kk, frag_t (&af)[TM], frag_t (&bf)[TN]) const {
    if constexpr (FP8) {
      const int c0 = kk * 4 + (lane >> 5);  // 16-byte pieces of the two 32-value blocks of this K step
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = mrow + i * 32 + (lane & 31);
        af[i] = join8(La[swz(r, c0)], La[swz(r, c0 + 2)]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WTN + j * 32 + (lane & 31);
        bf[j] = join8(Lb[swz(r, c0)], Lb[swz(r, c0 + 2)]);
      }
    } else {
      // 16 x 32 operand blocks: lane l holds row l % 16, K values [8 (l / 16), +8) of the step
      const int chunk = kk * 4 + (lane >> 4);
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = as_bf16x8(La[swz(mrow + i * 16 + (lane & 15), chunk)]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = as_bf16x8(Lb[swz(wn * WTN + j * 16 + (lane & 15), chunk)]);
    }
  }

  __device__ __forceinline__ void mma(acc_t (&acc)[TM][TN], const frag_t (&af)[TM], const frag_t (&bf)[TN],
                                      const uint32_t (&sd)[NSC], int kk) const {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (FP8) {
        const int sc = (int)((sd[i] >> (8 * (kk * 2 + (lane >> 5)))) & 255u);  // E8M0 of this lane's block
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], af[i], acc[i][j], 0, 0, 0, 127, 0, sc);
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
      }
    }
  }

  // One 32-K step of 16 x 16 blocks, columns outermost: right after the MFMAs of column j, B fragment j (and A
  // fragment j into an for j < TM, or with more row than column blocks A fragments [j TM / TN, (j + 1) TM / TN)) of
  // step kn of buffers (La, Lb) is read, so one register set holds B across steps.  With V the stage's global->LDS
  // loads (already issued in program order) are spread over the columns.
  template <bool V>
  __device__ __forceinline__ void step16(acc_t (&acc)[TM][TN], const frag_t (&ac)[TM], frag_t (&an)[TM], frag_t (&bf)[TN],
                                         const uint4* La, const uint4* Lb, int kn) const {
    const int chunk = kn * 4 + (lane >> 4);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], ac[i], acc[i][j], 0, 0, 0);
      bf[j] = as_bf16x8(Lb[swz(wn * WTN + j * 16 + (lane & 15), chunk)]);
      // A fragments of the next step: fragment j after column j (TM <= TN), else fragments [j TM / TN, (j + 1) TM / TN)
      if constexpr (TM <= TN) {
        if (j < TM) an[j] = as_bf16x8(La[swz(mrow + j * 16 + (lane & 15), chunk)]);
      } else {
#pragma unroll
        for (int i = j * TM / TN; i < (j + 1) * TM / TN; ++i) an[i] = as_bf16x8(La[swz(mrow + i * 16 + (lane & 15), chunk)]);
      }
    }
    constexpr int NV = APW + (AREM ? 1 : 0) + BPW, VPC = (NV + TN - 1) / TN;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, TM, 0);
      if (V && j * VPC < NV) __builtin_amdgcn_sched_group_barrier(0x020, VPC, 0);
      if (nA(j) >= 2) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
      else if (nA(j) == 1) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  }
  // A fragments read after column j's MFMAs
  static constexpr int nA(int j) { return TM <= TN ? (j < TM ? 1 : 0) : (j + 1) * TM / TN - j * TM / TN; }

  // fp8, 64 x 128 wave tiles: one 64-K step of 32 x 32 x 64 scaled blocks, columns outermost, with B fragment j (and, for
  // j < TM, A fragment j into an) of step kn of (La, Lb) read right after column j's MFMAs, as step16 does: one B
  // register set across steps keeps the wider fp8 fragments within the register budget.  sc: the activation scale
  // dwords of the step's stage.
  template <bool V>
  __device__ __forceinline__ void step8(acc_t (&acc)[TM][TN], const frag_t (&ac)[TM], frag_t (&an)[TM], frag_t (&bf)[TN],
                                        const uint4* La, const uint4* Lb, int kn, const uint32_t (&sc)[NSC], int kk) const {
    const int c0 = kn * 4 + (lane >> 5);
    int e8[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) e8[i] = (int)((sc[i] >> (8 * (kk * 2 + (lane >> 5)))) & 255u);  // E8M0 of the lane's block
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf[j], ac[i], acc[i][j], 0, 0, 0, 127, 0, e8[i]);
      {
        const int r = wn * WTN + j * 32 + (lane & 31);
        bf[j] = join8(Lb[swz(r, c0)], Lb[swz(r, c0 + 2)]);
      }
      if (j < TM) {
        const int r = mrow + j * 32 + (lane & 31);
        an[j] = join8(La[swz(r, c0)], La[swz(r, c0 + 2)]);
      }
    }
    constexpr int NV = APW + BPW + NSC, VPC = (NV + TN - 1) / TN;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      __builtin_amdgcn_sched_group_barrier(0x008, TM, 0);
      if (V && j * VPC < NV) __builtin_amdgcn_sched_group_barrier(0x020, VPC, 0);
      if (j < TM) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      else __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  }

  // One K stage from buffers (La, Lb) with scales sd.  Stage kt + 1 must already be in flight into (Na, Nb); after the
  // barrier the loads of stage kt + 2 go into (La, Lb, sd).
  __device__ __forceinline__ void stage(acc_t (&acc)[TM][TN], frag_t (&af)[2][TM], frag_t (&bf)[2][TN], uint4* La,
                                        uint4* Lb, uint32_t (&sd)[NSC], const uint4* Na, const uint4* Nb, int kt, int KT) const {
    if constexpr (MBE == 16) {
      // bf16: step 0 reads step 1's fragments from (La, Lb); after the barrier step 1 reads the next stage's step 0
      static_assert(NKK == 2 && APW + BPW <= TN * 2, "step16 interleave");
      step16<false>(acc, af[0], af[1], bf[0], La, Lb, 1);
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      __syncthreads();
      issue(La, Lb, sd, min(kt + 2, KT - 1));
      step16<true>(acc, af[1], af[0], bf[0], Na, Nb, 0);
      return;
    }
    if constexpr (FP8 && TN > TM) {
      // step 0 reads step 1's fragments from (La, Lb); after the barrier step 1 (this stage's scales, saved before the
      // next stage's scale loads overwrite sd) reads the next stage's step 0 from (Na, Nb)
      static_assert(NKK == 2, "fp8 stage of two 64-K steps");
      step8<false>(acc, af[0], af[1], bf[0], La, Lb, 1, sd, 0);
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      __syncthreads();
      uint32_t sl[NSC];
#pragma unroll
      for (int i = 0; i < NSC; ++i) sl[i] = sd[i];
      issue(La, Lb, sd, min(kt + 2, KT - 1));
      step8<true>(acc, af[1], af[0], bf[0], Na, Nb, 0, sl, 1);
      return;
    }
    constexpr int RPF = FP8 ? 2 : 1;  // LDS reads per fragment
    constexpr int NV = APW + BPW + (FP8 ? NSC : 0), ND = (TM + TN) * RPF, NM = TM * TN;
#pragma unroll
    for (int kk = 0; kk < NKK - 1; ++kk) {
      frag(La, Lb, kk + 1, af[(kk + 1) & 1], bf[(kk + 1) & 1]);
      mma(acc, af[kk & 1], bf[kk & 1], sd, kk);
      // MFMA, fragment read(s), MFMA, ... then the remaining MFMAs
      constexpr int DPM = (ND + NM - 1) / NM;
#pragma unroll
      for (int x = 0; x < NM; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (x * DPM < ND) __builtin_amdgcn_sched_group_barrier(0x100, DPM, 0);
      }
    }
    // stage kt + 1 has landed (this wave's loads) and is visible (everyone's), and nobody reads (La, Lb) any more
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __syncthreads();
    uint32_t sl[NSC];
#pragma unroll
    for (int i = 0; i < NSC; ++i) sl[i] = sd[i];
    issue(La, Lb, sd, min(kt + 2, KT - 1));
    frag(Na, Nb, 0, af[0], bf[0]);
    mma(acc, af[(NKK - 1) & 1], bf[(NKK - 1) & 1], sl, NKK - 1);
    // MFMA, load(s), fragment read(s), MFMA, ...
    constexpr int VPM = (NV + NM - 1) / NM, DPM = (ND + NM - 1) / NM;
#pragma unroll
    for (int x = 0; x < NM; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (x * VPM < NV) __builtin_amdgcn_sched_group_barrier(0x020, VPM, 0);
      if (x * DPM < ND) __builtin_amdgcn_sched_group_barrier(0x100, DPM, 0);
    }
  }

  template <int EPI>
  __device__ __forceinline__ void store(const acc_t (&acc)[TM][TN], float4* st, int m0, int n0) const {
    tile_store<EPI, MBE, TM, TN, WTM, WTN>(g, acc, st, m0 + mrow, n0 + wn * WTN, lane);
  }
};

}  // namespace

}  // namespace t2w
