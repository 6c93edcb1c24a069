// Block-causal attention of the DiT over paged key slots (head dim 64, bf16 in, fp32 online softmax, bf16 out).
//
// Replaces the reference's FlashInfer BatchPrefillWithPagedKVCacheWrapper call (page size 1, non-causal;
// engine/runtime/dit_fast.py:147-153, 291): every packed row attends from its new frames to its own key list, which
// holds the row's new frames first and then its cached frames (the reference's [new, cache] order; the set is what
// matters, there is no positional encoding).  With chunk > 0 a new frame sees only the new frames of its own and
// earlier chunks (the chunk-causal mask of whole-sequence solves); cached frames are always visible.
//
// CDNA4 mapping: one wave owns 32 queries of one head.  Scores are computed transposed, S^T = K . Q^T with
// v_mfma_f32_32x32x16_bf16 (the wave's Q fragment stays in registers), so each lane holds 16 of the 32 keys of its own
// query and the softmax statistics need a single cross-half exchange.  The probabilities then feed O^T += V^T . P^T
// directly from registers: the key order inside each 16-key MFMA is permuted to the order the score layout produced,
// and V is fetched in that order (for a fixed key index the 32 lanes of a half read 64 contiguous bytes).
#include "common.h"
#include "t2w_internal.h"

namespace t2w {

namespace {

constexpr float NEG = -1.0e30f;

__global__ void __launch_bounds__(128) attn_kernel(AttnArgs a) {
  const int tile = blockIdx.x, head = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = a.tiles[2 * tile];
  const int qpos0 = a.tiles[2 * tile + 1] + wave * 32;
  const int T = a.row_len[row];
  if (qpos0 >= T) return;
  const int start = a.row_start[row], kvoff = a.row_kv_off[row], kvlen = a.row_kv_len[row];
  const int H = a.heads * 64;
  const int half = lane >> 5, col = lane & 31;

  const int myq = qpos0 + col;
  const int qc = myq < T ? myq : T - 1;
  const int qlast = (qpos0 + 31 < T ? qpos0 + 31 : T - 1);
  const int lim_me = a.chunk > 0 ? min(T, (qc / a.chunk + 1) * a.chunk) : T;
  const int lim_max = a.chunk > 0 ? min(T, (qlast / a.chunk + 1) * a.chunk) : T;

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
  const float sl2 = a.scale * 1.4426950408889634f;

  for (int seg = 0; seg < 2; ++seg) {
    const int kb = seg == 0 ? 0 : T;
    const int ke = seg == 0 ? lim_max : kvlen;
    for (int k0 = kb; k0 < ke; k0 += 32) {
      const int kidx = k0 + col;
      const int slot = a.kv_idx[kvoff + (kidx < ke ? kidx : kb)];
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
      {
        const bf16_t* kp = a.k_pool + (size_t)slot * H + head * 64 + half * 8;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(*(const uint4*)(kp + kk * 16)), qf[kk], s, 0, 0, 0);
      }
      // lane holds query col, keys k0 + (r/4)*8 + half*4 + r%4
      float mx = NEG;
      bool vis[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + (r >> 2) * 8 + half * 4 + (r & 3);
        vis[r] = key < ke && (seg == 1 || key < lim_me);
        s[r] = vis[r] ? s[r] * sl2 : NEG;
        mx = fmaxf(mx, s[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mn = fmaxf(m, mx);
      const float alpha = exp2f(m - mn);
      float rs = 0.f;
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = vis[r] ? exp2f(s[r] - mn) : 0.f;
        rs += p[r];
      }
      rs += __shfl_xor(rs, 32, 64);
      l = l * alpha + rs;
      m = mn;
#pragma unroll
      for (int r = 0; r < 16; ++r) { o0[r] *= alpha; o1[r] *= alpha; }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        bf16x8 pf;
        {
          union { uint4 u; bf16x8 b; } c;
          c.u = make_uint4(pack2(p[8 * hh], p[8 * hh + 1]), pack2(p[8 * hh + 2], p[8 * hh + 3]),
                           pack2(p[8 * hh + 4], p[8 * hh + 5]), pack2(p[8 * hh + 6], p[8 * hh + 7]));
          pf = c.b;
        }
        uint32_t vw0[4], vw1[4];
#pragma unroll
        for (int v = 0; v < 8; v += 2) {
          uint32_t e0[2], e1[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int kl = 16 * hh + ((v + u) >> 2) * 8 + half * 4 + ((v + u) & 3);
            const int sl = __shfl(slot, kl, 64);
            const bf16_t* vp = a.v_pool + (size_t)sl * H + head * 64 + col;
            e0[u] = vp[0];
            e1[u] = vp[32];
          }
          vw0[v >> 1] = e0[0] | (e0[1] << 16);
          vw1[v >> 1] = e1[0] | (e1[1] << 16);
        }
        o0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(make_uint4(vw0[0], vw0[1], vw0[2], vw0[3])), pf, o0, 0, 0, 0);
        o1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(make_uint4(vw1[0], vw1[1], vw1[2], vw1[3])), pf, o1, 0, 0, 0);
      }
    }
  }
  if (myq >= T) return;
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
