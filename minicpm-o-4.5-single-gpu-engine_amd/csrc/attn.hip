// Block-causal attention of the DiT over paged key slots (head dim 64, bf16 in, fp32 online softmax, bf16 out).
//
// Replaces the reference's FlashInfer BatchPrefillWithPagedKVCacheWrapper call (page size 1, non-causal;
// engine/runtime/dit_fast.py:147-153, 291): every packed row attends from its new frames to its own key list, which
// holds the row's new frames first and then its cached frames (the reference's [new, cache] order; the set is what
// matters, there is no positional encoding).  With chunk > 0 a new frame sees only the new frames of its own and
// earlier chunks (the chunk-causal mask of whole-sequence solves); cached frames are always visible.
//
// CDNA4 mapping: a workgroup of two waves owns 64 queries of one head; each wave 32 of them.  Keys come in tiles of
// 32, gathered by slot id with 16-byte loads into registers one tile ahead, then stored to LDS: K row-major with the
// 16-byte chunks XOR-swizzled by key, V transposed (d-major) with its keys permuted so that the probabilities the
// score MFMA leaves in a lane are exactly the K-slice the P.V MFMA wants from that lane.  Scores are computed
// transposed, S^T = K . Q^T (v_mfma_f32_32x32x16_bf16, the wave's Q fragment stays in registers), so each lane holds
// 16 of the 32 keys of its own query and the softmax needs one cross-half exchange; O^T += V^T . P^T.
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

constexpr float NEG = -1.0e30f;

// key k of a 32-key tile -> its column in the transposed V tile: bits 2 and 3 swapped
__device__ __forceinline__ int vpos(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

__global__ void __launch_bounds__(128) attn_kernel(AttnArgs a) {
  __shared__ uint4 ks[2][32 * 8];   // [key][16-byte chunk ^ (key & 7)]
  __shared__ uint4 vt[2][64 * 4];   // [d][16-byte chunk ^ ((d >> 1) & 3)] of 32 permuted keys
  const int tile = blockIdx.x, head = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = a.tiles[2 * tile];
  const int q0 = a.tiles[2 * tile + 1];
  const int T = a.row_len[row];
  const int start = a.row_start[row], kvoff = a.row_kv_off[row], kvlen = a.row_kv_len[row];
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

  // key tiles: new keys [0, lim_max) then cached keys [T, kvlen), 32 at a time
  const int n1 = (lim_max + 31) / 32, n2 = (kvlen - T + 31) / 32;
  const int ntiles = n1 + n2;
  // loader role: key lk = tid / 4 of the tile, 16-byte chunks 2 (tid % 4) and 2 (tid % 4) + 1 of its K and V rows
  const int lk = tid >> 2, lc = (tid & 3) * 2;
  uint4 rk[2], rv[2];
  auto tile_base = [&](int t, int& kb, int& ke) {
    if (t < n1) { kb = t * 32; ke = lim_max; }
    else { kb = T + (t - n1) * 32; ke = kvlen; }
  };
  auto gload = [&](int t) {
    int kb, ke;
    tile_base(t, kb, ke);
    const int k = kb + lk < ke ? kb + lk : kb;
    const size_t slot = (size_t)a.kv_idx[kvoff + k];
    const bf16_t* kp = a.k_pool + slot * H + head * 64 + lc * 8;
    const bf16_t* vp = a.v_pool + slot * H + head * 64 + lc * 8;
    rk[0] = *(const uint4*)kp;
    rk[1] = *(const uint4*)(kp + 8);
    rv[0] = *(const uint4*)vp;
    rv[1] = *(const uint4*)(vp + 8);
  };
  auto lstore = [&](int s) {
    ks[s][lk * 8 + ((lc) ^ (lk & 7))] = rk[0];
    ks[s][lk * 8 + ((lc + 1) ^ (lk & 7))] = rk[1];
    bf16_t* vb = (bf16_t*)vt[s];
    const int p = vpos(lk);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t w[4] = {rv[u].x, rv[u].y, rv[u].z, rv[u].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = (lc + u) * 8 + e;
        const bf16_t val = (bf16_t)((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffff));
        vb[d * 32 + (((p >> 3) ^ ((d >> 1) & 3)) << 3) + (p & 7)] = val;
      }
    }
  };

  f32x16 o0, o1;
#pragma unroll
  for (int r = 0; r < 16; ++r) { o0[r] = 0.f; o1[r] = 0.f; }
  float m = NEG, l = 0.f;
  const float sl2 = a.scale * 1.4426950408889634f;

  if (ntiles > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int s = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    if (active) {
      int kb, ke;
      tile_base(t, kb, ke);
      const bool cached = t >= n1;
      f32x16 sc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int chunk = kk * 2 + half;
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ks[s][col * 8 + (chunk ^ (col & 7))]), qf[kk], sc, 0, 0, 0);
      }
      // lane holds query col, keys kb + (r/4)*8 + half*4 + r%4
      float mx = NEG;
      bool vis[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + (r >> 2) * 8 + half * 4 + (r & 3);
        vis[r] = key < ke && (cached || key < lim_me);
        sc[r] = vis[r] ? sc[r] * sl2 : NEG;
        mx = fmaxf(mx, sc[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m, mx);
      const float alpha = exp2f(m - mn);
      float rs = 0.f;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = vis[r] ? exp2f(sc[r] - mn) : 0.f;
        rs += p[r];
      }
      rs += __shfl_xor(rs, 32, 64);
      l = l * alpha + rs;
      m = mn;
#pragma unroll
      for (int r = 0; r < 16; ++r) { o0[r] *= alpha; o1[r] *= alpha; }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        union { uint4 u; bf16x8 b; } pf;
        pf.u = make_uint4(pack2(p[8 * hh], p[8 * hh + 1]), pack2(p[8 * hh + 2], p[8 * hh + 3]), pack2(p[8 * hh + 4], p[8 * hh + 5]),
                          pack2(p[8 * hh + 6], p[8 * hh + 7]));
        const int chunk = hh * 2 + half;
        const int d0 = col, d1 = 32 + col;
        const uint4 v0 = vt[s][d0 * 4 + (chunk ^ ((d0 >> 1) & 3))];
        const uint4 v1 = vt[s][d1 * 4 + (chunk ^ ((d1 >> 1) & 3))];
        o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(v0), pf.b, o0, 0, 0, 0);
        o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(v1), pf.b, o1, 0, 0, 0);
      }
    }
    if (t + 1 < ntiles) lstore(s ^ 1);
    __syncthreads();
  }
  if (!active || myq >= T) return;
  const float inv = 1.0f / l;
  bf16_t* op = a.out + (size_t)(start + myq) * H + head * 64;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int d = g * 8 + half * 4;
    *(uint2*)(op + d) = make_uint2(pack2(o0[4 * g] * inv, o0[4 * g + 1] * inv), pack2(o0[4 * g + 2] * inv, o0[4 * g + 3] * inv));
    *(uint2*)(op + 32 + d) = make_uint2(pack2(o1[4 * g] * inv, o1[4 * g + 1] * inv), pack2(o1[4 * g + 2] * inv, o1[4 * g + 3] * inv));
  }
}

}  // namespace

hipError_t attention(const AttnArgs& a, hipStream_t st) {
  if (a.n_tiles <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_kernel, dim3(a.n_tiles, a.heads), dim3(128), 0, st, a);
  return hipGetLastError();
}

}  // namespace t2w
