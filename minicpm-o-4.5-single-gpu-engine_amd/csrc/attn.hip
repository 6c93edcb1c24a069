// Block-causal attention of the DiT over paged key slots (head dim 64, bf16 in, fp32 online softmax, bf16 out).
//
// Replaces the reference's FlashInfer BatchPrefillWithPagedKVCacheWrapper call (page size 1, non-causal;
// engine/runtime/dit_fast.py:147-153, 291): every packed row attends from its new frames to its own key list, which
// holds the row's new frames first and then its cached frames (the reference's [new, cache] order; the set is what
// matters, there is no positional encoding).  With chunk > 0 a new frame sees only the new frames of its own and
// earlier chunks (the chunk-causal mask of whole-sequence solves); cached frames are always visible.
//
// CDNA4 mapping: a workgroup of two waves owns 64 queries of one head; each wave 32 of them.  Keys come in tiles of
// 64 (two 32-key MFMA halves per barrier), gathered by slot id with 16-byte loads into registers one tile ahead (the
// slot ids themselves two tiles ahead, so the dependent id -> key load chain is hidden), then stored to LDS: K and V
// both row-major (key-major) with the 16-byte chunks XOR-swizzled by key.  Scores are computed transposed,
// S^T = K . Q^T (v_mfma_f32_32x32x16_bf16, the wave's Q fragment stays in registers), so each lane holds 16 of the 32
// keys of its own query (two runs of 4 consecutive keys per 8 probabilities) and the softmax needs one cross-half
// exchange; O^T += V^T . P^T takes its V^T fragments with LDS transpose reads (ds_read_b64_tr_b16: in each group of 16
// lanes, lane j names a row of four 16-bit values and lane i receives element i % 4 of rows i / 4 + 4 e, e = 0..3), two
// per fragment, each giving a lane 4 consecutive keys of its own channel d -- exactly the keys whose probabilities
// the score MFMA left in that lane.
//
// Large calls whose caller bounds every key list (AttnArgs.kv_max <= 512) take a row-resident form instead: one
// workgroup per (row, head) copies the whole list into LDS once with global_load_lds and runs every query block of the
// row from there (attn_row_kernel); the per-query arithmetic and its order are the tile kernel's, so are the bits.
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

constexpr float NEG = -1.0e30f;

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// V^T fragment of the P.V MFMA from a key-major V tile in LDS (16-byte chunks swizzled by key): lane l gets channel
// d = d0 + l % 32 and keys kb + 4 (l / 32) + {0..3} (elements 0..3) and kb + 8 + 4 (l / 32) + {0..3} (elements 4..7),
// the keys whose probabilities the score MFMA leaves in the lanes of that half
__device__ __forceinline__ bf16x8 vt_frag(const uint4* vtile, int kb, int d0, int lane) {
  const int g = lane >> 4, j = lane & 15;
  const int key = kb + 4 * (g >> 1) + (j >> 2);  // the row this lane names: 4 keys x 4 runs of 4 channels per group
  const int d = d0 + 16 * (g & 1) + 4 * (j & 3);
  const bf16_t* base = (const bf16_t*)vtile;
  const int k2 = key + 8;
  const bf16_t* p1 = base + key * 64 + ((((d >> 3) ^ (key & 7)) << 3) | (d & 7));
  const bf16_t* p2 = base + k2 * 64 + ((((d >> 3) ^ (k2 & 7)) << 3) | (d & 7));
  const v4s_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)p1);
  const v4s_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)p2);
  const uint4 u = make_uint4((uint32_t)(uint16_t)a.x | ((uint32_t)(uint16_t)a.y << 16), (uint32_t)(uint16_t)a.z | ((uint32_t)(uint16_t)a.w << 16),
                             (uint32_t)(uint16_t)b.x | ((uint32_t)(uint16_t)b.y << 16), (uint32_t)(uint16_t)b.z | ((uint32_t)(uint16_t)b.w << 16));
  return as_bf16x8(u);
}

// The maximum of the 32 scores a lane holds for its query in a 64-key tile (MFMA results or -inf, never NaN), in 16
// v_max3_f32: through fmaxf each MFMA result is first canonicalised by a v_max_f32 of its own (56 instructions in all)
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ float tile_score_max(const f32x16 (&sc)[2]) {
  float m0 = max3_raw(sc[0][0], sc[0][1], sc[0][2]), m1 = max3_raw(sc[1][0], sc[1][1], sc[1][2]);
#pragma unroll
  for (int r = 3; r < 15; r += 2) {
    m0 = max3_raw(m0, sc[0][r], sc[0][r + 1]);
    m1 = max3_raw(m1, sc[1][r], sc[1][r + 1]);
  }
  return max3_raw(max3_raw(m0, sc[0][15], sc[1][15]), m1, m1);
}

// NaN outputs for queries [q0, q1) of a row whose key list breaks what the kernels assume: longer than the caller's
// bound, or shorter than the row's own tokens (a row's new frames are the first entries of its list)
__device__ __forceinline__ void nan_rows(const AttnArgs& a, int start, int q0, int q1, int head, int tid, int nthreads) {
  const int H = a.heads * 64;
  for (int i = q0 * 64 + tid; i < q1 * 64; i += nthreads) {
    const size_t o = (size_t)(start + i / 64) * H + head * 64 + i % 64;
    if (a.out8) {
      a.out8[o] = 0x7f;  // e4m3 NaN
      if (i % 32 == 0) a.out8s[(size_t)(start + i / 64) * (H / 32) + head * 2 + (i % 64) / 32] = 0xff;  // E8M0 NaN
    } else {
      a.out[o] = 0x7fc0;  // bf16 NaN
    }
  }
}

// KS > 1 (few workgroups, e.g. a streaming chunk): KS groups of two waves share the 64 queries and take every KS-th
// key tile each; their softmax states (max, sum, output) are merged through LDS at the end.
template <int KS>
__global__ void __launch_bounds__(128 * KS, 2) attn_kernel(AttnArgs a) {
  __shared__ uint4 ks[KS][2][64 * 8];      // [key][16-byte chunk ^ (key & 7)], 64 keys
  __shared__ uint4 vt[KS][2][64 * 8];      // [key][16-byte chunk ^ (key & 7)], 64 keys
  // XCD-aware order: consecutive workgroups go to different XCDs, so each XCD takes a contiguous run of (head, tile)
  // pairs; the query tiles of one row and head then share that row's keys and values in one L2
  const int nblk = gridDim.x * gridDim.y, full = (nblk / 8) * 8;
  int lin = blockIdx.y * gridDim.x + blockIdx.x;
  if (lin < full) lin = (lin % 8) * (nblk / 8) + lin / 8;
  const int tile = lin % gridDim.x, head = lin / gridDim.x;
  const int gi = threadIdx.x >> 7, tid = threadIdx.x & 127, lane = tid & 63, wave = tid >> 6;
  const int row = a.tiles[2 * tile];
  const int q0 = a.tiles[2 * tile + 1];
  const int T = a.row_len[row];
  if (q0 >= T) return;  // a filler tile past its row's end (padded tile lists): the whole workgroup leaves together
  const int start = a.row_start[row], kvoff = a.row_kv_off[row], kvlen = a.row_kv_len[row];
  if (kvlen < T) {  // a malformed table: NaN outputs instead of key reads past the row's list (workgroup-uniform exit)
    nan_rows(a, start, q0, min(q0 + 64, T), head, threadIdx.x, 128 * KS);
    return;
  }
  const int H = a.heads * 64;
  const int half = lane >> 5, col = lane & 31;
  const int qpos0 = q0 + wave * 32;
  const bool active = qpos0 < T;  // inactive waves still load tiles for their partner

  const int myq = qpos0 + col;
  const int qc = myq < T ? myq : T - 1;
  const int lim_me = a.chunk > 0 ? min(T, (qc / a.chunk + 1) * a.chunk) : T;
  const int tile_last = min(q0 + 63, T - 1);
  const int lim_max = a.chunk > 0 ? min(T, (tile_last / a.chunk + 1) * a.chunk) : T;

  bf16x8 qf[4];
  {
    const bf16_t* qp = a.q + (size_t)(start + qc) * H + head * 64 + half * 8;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = as_bf16x8(*(const uint4*)(qp + kk * 16));
  }

  // key tiles of 64: new keys [0, lim_max), then cached keys [T, kvlen)
  const int n1 = (lim_max + 63) / 64, n2 = (kvlen - T + 63) / 64;
  const int ntiles = n1 + n2;
  // loader role: key lk of the tile, 16-byte chunks lc .. lc + 3 of its K and V rows
  const int lk = tid >> 1, lc = (tid & 1) * 4;
#define T2W_TILE_RANGE(t, kb, ke)                 \
  if ((t) < n1) { kb = (t) * 64; ke = lim_max; }  \
  else { kb = T + ((t) - n1) * 64; ke = kvlen; }
#define T2W_SLOT_OF(t, out)                                   \
  {                                                           \
    int kb_, ke_;                                             \
    T2W_TILE_RANGE(t, kb_, ke_)                               \
    out = a.kv_idx[kvoff + (kb_ + lk < ke_ ? kb_ + lk : kb_)]; \
  }
  // two register sets (a, b) of one tile each: the loads of tile t + 2 KS are issued while tile t is multiplied and
  // tile t + KS (loaded one step earlier) goes to LDS
  uint4 rk0a, rk1a, rk2a, rk3a, rv0a, rv1a, rv2a, rv3a, rk0b, rk1b, rk2b, rk3b, rv0b, rv1b, rv2b, rv3b;
#define T2W_GLOAD(slot, X)                                                         \
  {                                                                                     \
    const uint4* kp = (const uint4*)(a.k_pool + (size_t)(slot) * H + head * 64 + lc * 8); \
    const uint4* vp = (const uint4*)(a.v_pool + (size_t)(slot) * H + head * 64 + lc * 8); \
    rk0##X = kp[0]; rk1##X = kp[1]; rk2##X = kp[2]; rk3##X = kp[3];                     \
    rv0##X = vp[0]; rv1##X = vp[1]; rv2##X = vp[2]; rv3##X = vp[3];                     \
  }
#define T2W_LSTORE(s, X)                                         \
  {                                                              \
    uint4* kr = ks[gi][s] + lk * 8;                              \
    kr[(lc + 0) ^ (lk & 7)] = rk0##X;                           \
    kr[(lc + 1) ^ (lk & 7)] = rk1##X;                           \
    kr[(lc + 2) ^ (lk & 7)] = rk2##X;                           \
    kr[(lc + 3) ^ (lk & 7)] = rk3##X;                           \
    uint4* vr = vt[gi][s] + lk * 8;                              \
    vr[(lc + 0) ^ (lk & 7)] = rv0##X;                           \
    vr[(lc + 1) ^ (lk & 7)] = rv1##X;                           \
    vr[(lc + 2) ^ (lk & 7)] = rv2##X;                           \
    vr[(lc + 3) ^ (lk & 7)] = rv3##X;                           \
  }

  f32x16 o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) { o0[r] = 0.f; o1[r] = 0.f; }
  float m = NEG, l = 0.f;  // running max (raw score units) and sum
  const float sl2 = a.scale * 1.4426950408889634f;
  const int lim_w0 = a.chunk > 0 ? min(T, (qpos0 / a.chunk + 1) * a.chunk) : T;  // the wave's first query's limit

  // group gi takes tiles gi, gi + KS, ...; every group runs the same number of iterations (the barriers are shared)
  const int niter = (ntiles + KS - 1) / KS;
  int slot_next = 0;
  if (gi < ntiles) {
    int s0;
    T2W_SLOT_OF(gi, s0)
    T2W_GLOAD(s0, a)
    T2W_LSTORE(0, a)
  }
  if (gi + KS < ntiles) {
    int s1;
    T2W_SLOT_OF(gi + KS, s1)
    T2W_GLOAD(s1, b)
  }
  if (gi + 2 * KS < ntiles) T2W_SLOT_OF(gi + 2 * KS, slot_next)
  __syncthreads();
  // one key tile t from LDS buffer s: scores, online softmax, P.V
  auto tile_step = [&](const int t, const int s) {
    if (active && t < ntiles) {
      int kb, ke;
      T2W_TILE_RANGE(t, kb, ke)
      const bool cached = t >= n1;
      // visible new keys of this query end at lim_me; cached keys at ke.  lim_lo: the wave's smallest limit (its first
      // query's: limits grow with the position), for the all-visible test
      const int lim = cached ? ke : min(ke, lim_me);
      const int lim_lo = cached ? ke : min(ke, lim_w0);
      const bool two = kb + 32 < ke;  // the second 32-key half holds keys
      // scores of both halves first: one max, one rescale and one exponent pass per 64 keys
      f32x16 sc[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[sub][r] = 0.f;
        if (sub == 0 || two) {
          const int krow = sub * 32 + col;
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const int chunk = kk * 2 + half;
            sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ks[gi][s][krow * 8 + (chunk ^ (krow & 7))]), qf[kk], sc[sub], 0, 0, 0);
          }
        }
      }
      // lane holds query col, keys kb + sub * 32 + (r/4)*8 + half*4 + r%4; invisible keys score -inf (raw units)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int sb = kb + sub * 32;
        if (sb + 32 > lim_lo || (sub == 1 && !two)) {  // wave-uniform: some key of this half is invisible to some query
          const int nvis = lim - (sb + half * 4);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int off = (r >> 2) * 8 + (r & 3);
            sc[sub][r] = off < nvis ? sc[sub][r] : -__builtin_inff();
          }
        }
      }
      float mx = tile_score_max(sc);
      mx = fmaxf(mx, xor32(mx));
      // m starts at a finite -1e30: keys all invisible so far give exp2(-inf) = 0 and leave m, l and o alone
      const float mn = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f((m - mn) * sl2);
      const float mb = -mn * sl2;
      // probabilities, packed to bf16 as they are made (the P.V operands), their fp32 sum on the side
      float rs = 0.f;
      uint4 pf[2][2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float e[8];
#pragma unroll
          for (int x = 0; x < 8; ++x) {
            e[x] = __builtin_amdgcn_exp2f(fmaf(sc[sub][8 * hh + x], sl2, mb));
            rs += e[x];
          }
          pf[sub][hh] = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
        }
      rs += xor32(rs);
      l = l * alpha + rs;
      m = mn;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {  // the running max moved for some query of the wave
#pragma unroll
        for (int r = 0; r < 16; ++r) { o0[r] *= alpha; o1[r] *= alpha; }
      }
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        if (sub == 1 && !two) break;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const bf16x8 v0 = vt_frag(vt[gi][s], sub * 32 + hh * 16, 0, lane);
          const bf16x8 v1 = vt_frag(vt[gi][s], sub * 32 + hh * 16, 32, lane);
          o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v0, as_bf16x8(pf[sub][hh]), o0, 0, 0, 0);
          o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v1, as_bf16x8(pf[sub][hh]), o1, 0, 0, 0);
        }
      }
    }
  };
  // unrolled by two so that each step names its register sets at compile time
  for (int it = 0; it < niter; it += 2) {
    {
      const int t = it * KS + gi;
      if (t + 2 * KS < ntiles) T2W_GLOAD(slot_next, a)
      if (t + 3 * KS < ntiles) T2W_SLOT_OF(t + 3 * KS, slot_next)
      tile_step(t, 0);
      if (t + KS < ntiles) T2W_LSTORE(1, b)
      __syncthreads();
    }
    if (it + 1 < niter) {
      const int t = (it + 1) * KS + gi;
      if (t + 2 * KS < ntiles) T2W_GLOAD(slot_next, b)
      if (t + 3 * KS < ntiles) T2W_SLOT_OF(t + 3 * KS, slot_next)
      tile_step(t, 1);
      if (t + KS < ntiles) T2W_LSTORE(0, a)
      __syncthreads();
    }
  }
#undef T2W_TILE_RANGE
#undef T2W_SLOT_OF
#undef T2W_GLOAD
#undef T2W_LSTORE
  if constexpr (KS > 1) {
    // merge: groups 1.. leave (max, sum, output) per lane in their (now free) tile buffers, group 0 folds them in
    // group order, rescaling each by 2^((m_g - m*) scale)
    // per wave: o0 in the group's K buffers (16 x 64 floats), o1, m and l in its V buffers (18 x 64 floats)
    float* xk = (float*)ks[gi] + wave * (16 * 64);
    float* xv = (float*)vt[gi] + wave * (18 * 64);
    if (gi > 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) { xk[r * 64 + lane] = o0[r]; xv[r * 64 + lane] = o1[r]; }
      xv[16 * 64 + lane] = m;
      xv[17 * 64 + lane] = l;
    }
    __syncthreads();
    if (gi > 0) return;
#pragma unroll
    for (int g2 = 1; g2 < KS; ++g2) {
      const float* yk = (const float*)ks[g2] + wave * (16 * 64);
      const float* yv = (const float*)vt[g2] + wave * (18 * 64);
      const float mg = yv[16 * 64 + lane], lg = yv[17 * 64 + lane];
      const float mn = fmaxf(m, mg);
      const float fa = __builtin_amdgcn_exp2f((m - mn) * sl2), fb = __builtin_amdgcn_exp2f((mg - mn) * sl2);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        o0[r] = o0[r] * fa + yk[r * 64 + lane] * fb;
        o1[r] = o1[r] * fa + yv[r * 64 + lane] * fb;
      }
      l = l * fa + lg * fb;
      m = mn;
    }
  }
  if (!active || myq >= T) return;
  const float inv = 1.0f / l;
  if (a.out8) {
    // MX fp8: d 0-31 (o0) and 32-63 (o1) are the head's two blocks, each spread over this lane and its partner
    float m0 = 0.f, m1 = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) { m0 = fmaxf(m0, fabsf(o0[r])); m1 = fmaxf(m1, fabsf(o1[r])); }
    m0 = fmaxf(m0, xor32(m0)) * inv;
    m1 = fmaxf(m1, xor32(m1)) * inv;
    const int e0 = mx_exp(m0), e1 = mx_exp(m1);
    uint8_t* qp = a.out8 + (size_t)(start + myq) * H + head * 64;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = g * 8 + half * 4;
      *(uint32_t*)(qp + d) = mx_pack4(o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv, o0[4 * g + 3] * inv, e0);
      *(uint32_t*)(qp + 32 + d) = mx_pack4(o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv, o1[4 * g + 3] * inv, e1);
    }
    if (half == 0) {
      uint8_t* sp = a.out8s + (size_t)(start + myq) * (H / 32) + head * 2;
      sp[0] = (uint8_t)(e0 + 127);
      sp[1] = (uint8_t)(e1 + 127);
    }
    return;
  }
  bf16_t* op = a.out + (size_t)(start + myq) * H + head * 64;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int d = g * 8 + half * 4;
    *(uint2*)(op + d) = make_uint2(pack2(o0[4 * g] * inv, o0[4 * g + 1] * inv), pack2(o0[4 * g + 2] * inv, o0[4 * g + 3] * inv));
    *(uint2*)(op + 32 + d) = make_uint2(pack2(o1[4 * g] * inv, o1[4 * g + 1] * inv), pack2(o1[4 * g + 2] * inv, o1[4 * g + 3] * inv));
  }
}

// One 64-key tile [kb, kb + 64) of a key list held in LDS (K and V rows key-major, 16-byte chunks swizzled by key) for
// the wave's 32 queries: scores S^T = K . Q^T, masks (keys at or past lim invisible; lim_lo the wave's smallest limit),
// online softmax and O^T += V^T . P^T, in the order and arithmetic of attn_kernel's tile_step
__device__ __forceinline__ void lds_key_tile(const uint4* Ks, const uint4* Vs, int kb, int ke, int lim, int lim_lo, const bf16x8 (&qf)[4],
                                             float sl2, int lane, f32x16& o0, f32x16& o1, float& m, float& l) {
  const int half = lane >> 5, col = lane & 31;
  const bool two = kb + 32 < ke;
  f32x16 sc[2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[sub][r] = 0.f;
    if (sub == 0 || two) {
      const int kr = kb + sub * 32 + col;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int chunk = kk * 2 + half;
        sc[sub] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(Ks[kr * 8 + (chunk ^ (kr & 7))]), qf[kk], sc[sub], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int sb = kb + sub * 32;
    if (sb + 32 > lim_lo || (sub == 1 && !two)) {
      const int nvis = lim - (sb + half * 4);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int off = (r >> 2) * 8 + (r & 3);
        sc[sub][r] = off < nvis ? sc[sub][r] : -__builtin_inff();
      }
    }
  }
  float mx = tile_score_max(sc);
  mx = fmaxf(mx, xor32(mx));
  const float mn = fmaxf(m, mx);
  const float alpha = __builtin_amdgcn_exp2f((m - mn) * sl2);
  const float mb = -mn * sl2;
  float rs = 0.f;
  uint4 pf[2][2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float e[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        e[x] = __builtin_amdgcn_exp2f(fmaf(sc[sub][8 * hh + x], sl2, mb));
        rs += e[x];
      }
      pf[sub][hh] = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
    }
  rs += xor32(rs);
  l = l * alpha + rs;
  m = mn;
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) { o0[r] *= alpha; o1[r] *= alpha; }
  }
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (sub == 1 && !two) break;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const bf16x8 v0 = vt_frag(Vs, kb + sub * 32 + hh * 16, 0, lane);
      const bf16x8 v1 = vt_frag(Vs, kb + sub * 32 + hh * 16, 32, lane);
      o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v0, as_bf16x8(pf[sub][hh]), o0, 0, 0, 0);
      o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v1, as_bf16x8(pf[sub][hh]), o1, 0, 0, 0);
    }
  }
}

// Row-resident form for large calls whose key lists fit in LDS: one workgroup of NWV waves per (row, head) copies the
// row's whole key and value lists for the head into LDS once (global_load_lds by slot id, the same key-major 16-byte
// chunk swizzle as the tiles above, and past the list's end up to 63 clamped, finite keys that a last tile overhangs),
// then each wave takes one 32-query block (T <= kv_max <= 32 NWV) and runs its key tiles straight from LDS: no
// gathers, stores or barriers inside the key loop, and the keys and values of a row are read from the pools once per
// head instead of once per 64-query tile.  LDS holds round8(kv_max + 63) keys:
// with kv_max <= 256 two workgroups of 8 waves share a CU (80 KB each; one copies while the other computes), longer
// lists take one workgroup of 16 waves per CU (up to 144 KB); either way four waves per SIMD, registers capped at
// 128 per lane.  Per query the arithmetic is that of attn_kernel, in the same order, so the outputs are the same bits.
__host__ __device__ constexpr int row_krows(int kv_max) { return (kv_max + 63 + 7) / 8 * 8; }
constexpr int ROW_KROWS = row_krows(ATTN_ROW_KMAX);

// The key list kv_idx[kvoff ..][0 .. kvlen) of one head into LDS (K and V key-major, 16-byte chunks swizzled by key,
// rows up to round8(kvlen + 63) with the keys past the end clamped to the last), then waits for it and a barrier.
// 8-key blocks go to the workgroup's 8 waves in turn; lane l fetches key 8 b + l / 8's chunk (l % 8) ^ key.
template <int NWV>
__device__ __forceinline__ void load_key_list(uint4* Ks, uint4* Vs, const AttnArgs& a, int kvoff, int kvlen, int head, int wave,
                                              int lane) {
  const int H = a.heads * 64;
  const int nb8 = row_krows(kvlen) / 8;
  constexpr int MAXB = (ROW_KROWS / 8 + NWV - 1) / NWV;
  int slot[MAXB];
#pragma unroll
  for (int i = 0; i < MAXB; ++i) {
    const int b8 = wave + NWV * i, key = b8 * 8 + (lane >> 3);
    slot[i] = b8 < nb8 ? a.kv_idx[kvoff + min(key, kvlen - 1)] : 0;
  }
  const int ch = ((lane & 7) ^ ((lane >> 3) & 7)) * 8;  // the key's row-local index is b8 * 8 + lane / 8: key & 7 = lane / 8
#pragma unroll
  for (int i = 0; i < MAXB; ++i) {
    const int b8 = wave + NWV * i;
    if (b8 < nb8) {
      const size_t go = (size_t)slot[i] * H + head * 64 + ch;
      __builtin_amdgcn_global_load_lds((const void*)(a.k_pool + go), (lds_ptr_t)(Ks + b8 * 64), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(a.v_pool + go), (lds_ptr_t)(Vs + b8 * 64), 16, 0, 0);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

template <int NWV>
__global__ void __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(4, 4))) attn_row_kernel(AttnArgs a) {
  extern __shared__ uint4 lds[];  // K rows [KR][8 chunks], then V rows [KR][8 chunks]
  const int KR = row_krows(a.kv_max);
  uint4* Ks = lds;
  uint4* Vs = lds + KR * 8;
  const int head = blockIdx.x, row = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = a.row_len[row];
  if (T <= 0) return;
  const int start = a.row_start[row], kvoff = a.row_kv_off[row], kvlen = a.row_kv_len[row];
  const int H = a.heads * 64;
  if (kvlen > a.kv_max || T > 32 * NWV || kvlen < T) {  // longer than the caller's bound, or shorter than the row's
                                                       // own tokens: NaN outputs instead of copies past the LDS lists
    nan_rows(a, start, 0, T, head, tid, 64 * NWV);
    return;
  }
  load_key_list<NWV>(Ks, Vs, a, kvoff, kvlen, head, wave, lane);
  const int half = lane >> 5, col = lane & 31;
  const float sl2 = a.scale * 1.4426950408889634f;
  // T <= kv_max <= 32 NWV: at most one 32-query block per wave.  Blocks by cost (latest first) go to the waves in a
  // snake over the SIMDs (wave w runs on SIMD w % 4; round r = w / 4 hands SIMD s the (4 r + s)-th costliest block, or
  // the (4 r + 3 - s)-th on odd rounds), so each SIMD gets a mix of long and short blocks
  const int nblk = (T + 31) / 32;
  {
    const int r = wave >> 2, sm = wave & 3;
    const int bi = r * 4 + ((r & 1) ? 3 - sm : sm);
    if (bi >= nblk) return;
    const int q0 = (nblk - 1 - bi) * 32;
    const int myq = q0 + col, qc = myq < T ? myq : T - 1;
    const int lim_me = a.chunk > 0 ? min(T, (qc / a.chunk + 1) * a.chunk) : T;
    const int last = min(q0 + 31, T - 1);
    const int lim_max = a.chunk > 0 ? min(T, (last / a.chunk + 1) * a.chunk) : T;
    const int lim_w0 = a.chunk > 0 ? min(T, (q0 / a.chunk + 1) * a.chunk) : T;
    bf16x8 qf[4];
    {
      const bf16_t* qp = a.q + (size_t)(start + qc) * H + head * 64 + half * 8;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qf[kk] = as_bf16x8(*(const uint4*)(qp + kk * 16));
    }
    f32x16 o0, o1;
#pragma unroll
    for (int r = 0; r < 16; ++r) { o0[r] = 0.f; o1[r] = 0.f; }
    float m = NEG, l = 0.f;
    const int n1 = (lim_max + 63) / 64, n2 = (kvlen - T + 63) / 64;
    for (int t = 0; t < n1 + n2; ++t) {
      const bool cached = t >= n1;
      const int kb = cached ? T + (t - n1) * 64 : t * 64, ke = cached ? kvlen : lim_max;
      const int lim = cached ? ke : min(ke, lim_me);
      const int lim_lo = cached ? ke : min(ke, lim_w0);
      lds_key_tile(Ks, Vs, kb, ke, lim, lim_lo, qf, sl2, lane, o0, o1, m, l);
    }
    if (myq >= T) return;
    const float inv = 1.0f / l;
    if (a.out8) {
      float m0 = 0.f, m1 = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) { m0 = fmaxf(m0, fabsf(o0[r])); m1 = fmaxf(m1, fabsf(o1[r])); }
      m0 = fmaxf(m0, xor32(m0)) * inv;
      m1 = fmaxf(m1, xor32(m1)) * inv;
      const int e0 = mx_exp(m0), e1 = mx_exp(m1);
      uint8_t* qp = a.out8 + (size_t)(start + myq) * H + head * 64;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = g * 8 + half * 4;
        *(uint32_t*)(qp + d) = mx_pack4(o0[4 * g] * inv, o0[4 * g + 1] * inv, o0[4 * g + 2] * inv, o0[4 * g + 3] * inv, e0);
        *(uint32_t*)(qp + 32 + d) = mx_pack4(o1[4 * g] * inv, o1[4 * g + 1] * inv, o1[4 * g + 2] * inv, o1[4 * g + 3] * inv, e1);
      }
      if (half == 0) {
        uint8_t* sp = a.out8s + (size_t)(start + myq) * (H / 32) + head * 2;
        sp[0] = (uint8_t)(e0 + 127);
        sp[1] = (uint8_t)(e1 + 127);
      }
      return;
    }
    bf16_t* op = a.out + (size_t)(start + myq) * H + head * 64;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = g * 8 + half * 4;
      *(uint2*)(op + d) = make_uint2(pack2(o0[4 * g] * inv, o0[4 * g + 1] * inv), pack2(o0[4 * g + 2] * inv, o0[4 * g + 3] * inv));
      *(uint2*)(op + 32 + d) = make_uint2(pack2(o1[4 * g] * inv, o1[4 * g + 1] * inv), pack2(o1[4 * g + 2] * inv, o1[4 * g + 3] * inv));
    }
  }
}

}  // namespace

hipError_t attention(const AttnArgs& a, hipStream_t st) {
  if (a.n_tiles <= 0) return hipSuccess;
  // a grid of fewer workgroups than CUs (a streaming chunk) splits each workgroup's key tiles over four wave groups
  if (a.n_tiles * a.heads < 256) {
    hipLaunchKernelGGL(attn_kernel<4>, dim3(a.n_tiles, a.heads), dim3(512), 0, st, a);
  } else if (a.kv_max > 0 && a.kv_max <= ATTN_ROW_KMAX && (long)a.n_rows * a.heads >= 256 && a.n_tiles >= 3 * a.n_rows) {
    // rows of three or more query tiles on average: with fewer, most of a row workgroup's waves would idle while its
    // whole key list is copied (the tile kernel is faster there)
    static const hipError_t attr = [] {  // once per process (thread-safe initialisation): the LDS above 64 KB
      const int bytes = 2 * ROW_KROWS * 8 * (int)sizeof(uint4);
      hipError_t e = hipFuncSetAttribute((const void*)attn_row_kernel<8>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
      if (e == hipSuccess) e = hipFuncSetAttribute((const void*)attn_row_kernel<16>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
      return e;
    }();
    if (attr != hipSuccess) return attr;
    const size_t lds = 2 * (size_t)row_krows(a.kv_max) * 8 * sizeof(uint4);
    if (a.kv_max <= 256)  // two workgroups of 8 waves per CU
      hipLaunchKernelGGL(attn_row_kernel<8>, dim3(a.heads, a.n_rows), dim3(64 * 8), lds, st, a);
    else  // one workgroup of 16 waves per CU
      hipLaunchKernelGGL(attn_row_kernel<16>, dim3(a.heads, a.n_rows), dim3(64 * 16), lds, st, a);
  } else {
    hipLaunchKernelGGL(attn_kernel<1>, dim3(a.n_tiles, a.heads), dim3(128), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace t2w
