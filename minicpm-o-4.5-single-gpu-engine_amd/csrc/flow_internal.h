// Kernels of the flow encoder (codec tokens -> mu): row kernels, the placement of cached conv frames, the key/value
// store and the relative-position attention.  C (the encoder width) is a multiple of 512; heads of 64.
#pragma once

#include "common.h"

namespace t2w {

// Rows of the pre-lookahead conv's input: row r takes table row tok[r] (tok[r] < 0: a zero row, the lookahead
// padding of a final window), LayerNorm (affine, eps) times xscale, bf16 to x0[r]; and, when res[r] >= 0, the same
// values as fp16 to row res[r] of the residual stream h.
hipError_t flow_embed(const float* table, const int* tok, const int* res, const float* w, const float* b, float eps,
                      float xscale, bf16_t* x0, f16_t* h, int n, int C, hipStream_t st);

// The pre-lookahead conv2's two cached frames: stream s copies frames 0, 1 of its cache slot rd[s] into rows g[s],
// g[s] + 1 of the conv1 output G, and writes its new cache (the last two of [cache | conv1 outputs], t1[s] outputs at
// rows g[s] + 2 ..) to frames 0, 1 of slot wr[s].  Cache slots: cstride elements apart.
hipError_t flow_look_place(bf16_t* G, bf16_t* cache, const int* g, const int* t1, const int* rd, const int* wr, int R, int C,
                           long long cstride, hipStream_t st);

// The upsampling's input: row m of the residual stream h (n1 rows) as bf16 to rows up_dst[m] and up_dst[m] + 1 of U
// (nearest x2); stream s copies its four cached frames (cache frames 2..5 of slot rd[s]) into rows u[s] .. u[s] + 3 and
// writes its new cache (the last four of [cache | upsampled frames]; stream rows o1[s] .. of h) to frames 2..5 of wr[s].
hipError_t flow_up_place(const f16_t* h, bf16_t* U, const int* up_dst, int n1, const int* u, const int* o1, const int* t1,
                         bf16_t* cache, const int* rd, const int* wr, int R, int C, long long cstride, hipStream_t st);

// Row m of y (fp32): LayerNorm (w1, b1, eps1) times xscale, rounded to fp16 into h[m]; then LayerNorm (w2, b2, eps2) of
// that fp16 row, bf16 to a[m].
hipError_t flow_ln_scale_ln(const float* y, const float* w1, const float* b1, float eps1, float xscale, f16_t* h,
                            const float* w2, const float* b2, float eps2, bf16_t* a, int n, int C, hipStream_t st);

// Keys and values of new rows: qkv row m (fp16, q | k | v, C each) -> k | v of slot slot[m] of the pool (2 C per slot).
hipError_t flow_kv_store(const f16_t* qkv, int ldq, f16_t* pool, const int* slot, int n, int C, hipStream_t st);

struct RelAttnArgs {
  const f16_t* qkv;       // [rows, ldq]: q at column h * 64 (keys and values are read from the pool)
  int ldq;
  const f16_t* pool;      // [slots, 2 C]: k | v
  const f16_t* ptab;      // [2 rmax - 1, C]: linear_pos of the sinusoid of relative position r at row r + rmax - 1
  int rmax;
  const float* bias_u;    // [C] (head h at h * 64)
  const float* bias_v;
  bf16_t* out;            // [rows, C]
  const int* kv_idx;      // per stream: its key slots in time order (cached frames, then its new frames)
  const int* kv_off;      // [R]
  const int* kv_len;      // [R] keys L (T new included); L <= rmax
  const int* row_start;   // [R] first query row
  const int* row_len;     // [R] queries T
  const int* tiles;       // [n_tiles, 2]: (stream, first query) of each 32-query tile
  int n_tiles, heads;
  float scale;
};
hipError_t flow_rel_attention(const RelAttnArgs& a, hipStream_t st);

// Speaker embeddings: out[r] = W normalize(spk[r]) + b (W [mel, E] fp32; F.normalize's eps 1e-12).
hipError_t flow_speaker(const float* spk, const float* W, const float* b, float* out, int R, int E, int mel, hipStream_t st);

}  // namespace t2w
