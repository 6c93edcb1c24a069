// Internal launch interfaces shared by the kernel files and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch_timer.h"

namespace t2w {

typedef uint16_t bf16_t;
typedef uint16_t f16_t;  // storage type of the fp16 residual stream

// EPI_GELU_MX8: GELU, then MX fp8 codes to C (bytes, ldc) and block scales to c_scale (N % 32 == 0)
// EPI_QKV: the attention projection (N = 3 H): q and k rounded to bf16, per-head LayerNorm + affine, q to its token
// row of q_out, k and v to the token's key slot of the pools (fields qk.*); tile path only
// EPI_PART (small-row GEMM only): K split over `splits` workgroups per tile, split z writes its fp32 sum without bias
// to C + z * c_split (rows ldc apart); a row kernel that takes the sums as a Pend finishes the GEMM's epilogue
// Epilogues.  EPI_RESID_F16: the gated residual C(fp16) = fp16(C + gate * (acc + bias)), the residual stream kept in the
// reference's fp16 with fp32 arithmetic; EPI_F16: fp16 out.
enum Epi { EPI_BF16 = 0, EPI_GELU_BF16 = 1, EPI_RESID_F16 = 2, EPI_F32 = 3, EPI_GELU_MX8 = 4, EPI_QKV = 5, EPI_PART = 6, EPI_F16 = 7 };

struct QkvOut {
  bf16_t* q_out;        // [M, H]
  bf16_t* k_pool;       // [slots, H]
  bf16_t* v_pool;
  const int* slots;     // [M] key slot of each token
  const float *qw, *qb, *kw, *kb;  // [64] each
  float eps;
  int H;
  const float* rfreq = nullptr;  // rotary embedding of q and k after their LayerNorm: [32] pair frequencies (null: none)
  const int* pos = nullptr;      // [M] stream position of each token (with rfreq)
};

struct GemmArgs {
  const bf16_t* A;     // dense: A[m * lda + k]; taps: A[(a_src[m] + k / tapC) * lda + k % tapC]
  int lda;
  const int* a_src;    // taps mode when non-null
  int tapC;
  const bf16_t* B;     // weights [N, K] row-major
  int ldb;
  const float* bias;   // [N]
  const float* gate;   // [N], EPI_RESID_F16: C += gate * (acc + bias)
  void* C;
  int ldc;
  int M, N, K;         // K % 64 == 0
  float* ws;           // split-K partials (null: tile kernels only)
  size_t ws_bytes;
  // fp8 mode (w_scale non-null): A and B hold OCP e4m3 codes (lda, ldb, K in elements = bytes); A's MX scales are
  // a_scale[row * a_sld + k / 32] (E8M0; taps mode: row = frame), W row n is scaled by w_scale[n] in the epilogue
  const uint8_t* a_scale;
  int a_sld;
  const float* w_scale;
  uint8_t* c_scale;    // EPI_GELU_MX8: output block scales c_scale[m * c_sld + n / 32]
  int c_sld;
  QkvOut qk;           // EPI_QKV
  int splits;          // EPI_PART: K splits (1..4)
  size_t c_split;      // EPI_PART: elements between the splits' sums
  int act;             // EPI_BF16: activation after the bias (Act: none, SiLU, leaky ReLU 0.01)
};

// K-split sums of a GEMM whose epilogue is left to the next row kernel (EPI_PART): the GEMM's value at (n, c) is
// sum_s part[s * stride + n * ld + c] + bias[c]; with gate non-null it is a gated residual, h += gate * value.
struct Pend {
  const float* part = nullptr;  // null: nothing pending
  int S = 0;
  size_t stride = 0;
  int ld = 0;
  const float* bias = nullptr;
  const float* gate = nullptr;
};

// cfg < 0: by shape (split-K through g.ws when a tile grid would be too small to fill the chip)
hipError_t gemm_bf16(const GemmArgs& g, int epi, hipStream_t st, int cfg = -1);
bool gemm_splits(const GemmArgs& g);  // whether gemm_bf16 (cfg < 0) takes the split-K path for g

// One-kernel GEMM for calls of at most GEMM_SMALL_MAX_M rows (K split over the waves of a workgroup, reduced in LDS):
// plain epilogues (EPI_BF16 .. EPI_F32; K % 64 == 0, K <= 3072, ldc % 4 == 0), EPI_PART (the same, K also split over
// g.splits workgroups) and EPI_QKV (dense A, K <= 1024, N = 3 qk.H, qk.H % 64 == 0).  gemm_bf16 (cfg < 0) takes it
// whenever it fits (EPI_PART only through gemm_small).
constexpr int GEMM_SMALL_MAX_M = 128;
bool gemm_small_fits(const GemmArgs& g, int epi);
hipError_t gemm_small(const GemmArgs& g, int epi, hipStream_t st);
// whether an EPI_PART call runs on 64-row tiles (taps mode, more than 32 rows, at most 16 64-K steps per split)
bool gemm_small_part64(const GemmArgs& g);

struct SplitPlan {
  int splits;  // 0: split-K not possible for this shape / workspace
  int steps;   // 64-K steps per split
};
SplitPlan splitk_plan(int M, int N, int K, size_t ws_bytes);

// MX fp8 quantization: x [M, K] bf16 (rows ldx apart) -> q [M, K] e4m3 (rows ldq apart), s [M, K / 32] E8M0; K % 32 == 0
hipError_t quant_mx8(const bf16_t* x, int ldx, int M, int K, uint8_t* q, int ldq, uint8_t* s, hipStream_t st);
hipError_t gemm_splitk(const GemmArgs& g, int epi, const SplitPlan& p, float* part, hipStream_t st);
// e4m3 weights with per-output-channel scales to bf16: out [N, K] = bf16(e4m3(w8) * ws[n]); K % 8 == 0
hipError_t dequant_w8(const uint8_t* w8, const float* ws, int N, int K, bf16_t* out, hipStream_t st);

// Per-token row kernels of the DiT block (H = hidden, one wave per token); h is the fp16 residual stream [N, H].
// With pd.part set they first finish a pending gated residual (h updated in place) or, for ln_mish_conv, take the
// pending GEMM's bf16-rounded value as their input row instead of y.
// Byte ranges (device memory) that a row kernel without a pending GEMM also reads, in workgroups of its own after its
// rows, so that the weights of the GEMMs that follow are in the device's caches (the 256 MB memory-side cache) when
// they start; the values are discarded.  Up to two ranges, 16-byte aligned.
struct Prefetch {
  const void* p[2] = {nullptr, nullptr};
  size_t bytes[2] = {0, 0};
};
hipError_t ln_mod(f16_t* h, const float* shift, const float* scale1, float eps, bf16_t* out, int N, int H,
                  hipStream_t st, const Pend& pd = Pend(), const Prefetch& pf = Prefetch());
// ln_mod with MX fp8 output: codes q [N, H], block scales qs [N, H / 32]
hipError_t ln_mod_mx8(const f16_t* h, const float* shift, const float* scale1, float eps, uint8_t* q, uint8_t* qs, int N,
                      int H, hipStream_t st, const Prefetch& pf = Prefetch());

struct ConvPlace {   // where the normed frames of a causal conv go (the padded frame buffer and the conv caches)
  bf16_t* P;          // [N + 2 R, H]: per row r its two cached frames, then its T_r frames
  const int* tok_row; // [N]
  const int* tok_pos; // [N]
  const int* row_start;  // [R] first token of row r
  const int* row_len;    // [R]
  const bf16_t* cache_base;  // conv cache pool; row r reads frames at cache_base + rd[r] * cache_stride
  bf16_t* cache_out_base;    // and writes its new frames at cache_out_base + wr[r] * cache_stride
  const int* rd;
  const int* wr;
  long long cache_stride;    // elements between row slots
  int N, R;
  uint8_t* P8 = nullptr;     // fp8 mode: the frame buffer as MX fp8 codes [N + 2 R, H] (P unused)
  uint8_t* P8s = nullptr;    // and its block scales [N + 2 R, H / 32]
};

hipError_t ln_mod_conv(f16_t* h, const float* shift, const float* scale1, float eps, const ConvPlace& cp, int H,
                       hipStream_t st, const Pend& pd = Pend(), const Prefetch& pf = Prefetch());
hipError_t ln_mish_conv(const bf16_t* y, const float* w, const float* b, float eps, const ConvPlace& cp, int H,
                        hipStream_t st, const Pend& pd = Pend(), const Prefetch& pf = Prefetch());
// rotary embedding of the q rows [N, H] and of the keys at slots[n] after the tile GEMM's q / k epilogue: channel pair
// (2i, 2i + 1) of each head turned by pos[n] * rfreq[i] (bf16 in and out)
hipError_t rope_qk(bf16_t* q, bf16_t* k_pool, const int* slots, const int* pos, const float* rfreq, int N, int H, hipStream_t st);
hipError_t qk_norm_scatter(const bf16_t* qkv, const float* qw, const float* qb, const float* kw, const float* kb,
                           float eps, bf16_t* q_out, bf16_t* k_pool, bf16_t* v_pool, const int* slots, int N, int heads,
                           hipStream_t st, const float* rfreq = nullptr, const int* pos = nullptr);

struct AttnArgs {
  const bf16_t* q;        // [N, heads, 64]
  const bf16_t* k_pool;   // [slots, heads, 64]
  const bf16_t* v_pool;
  bf16_t* out;            // [N, heads * 64]
  const int* kv_idx;      // concatenated per-row key slot lists: the row's new tokens first, then its cached keys
  const int* row_start;   // [R] first token
  const int* row_len;     // [R] new tokens T_r
  const int* row_kv_off;  // [R] offset into kv_idx
  const int* row_kv_len;  // [R] keys in the list (T_r + cached)
  const int* tiles;       // [n_tiles, 2]: (row, first query position) of each 64-query tile
  int n_tiles, heads, chunk;  // chunk > 0: a new frame sees new frames of its own and earlier chunks only
  float scale;
  uint8_t* out8 = nullptr;   // fp8 mode: MX fp8 codes [tokens, H] (out unused) and block scales [tokens, H / 32]
  uint8_t* out8s = nullptr;
  int n_rows = 0;            // rows of the call (the row-resident kernel's grid)
  int kv_max = 0;            // 0, or the caller's bound on every row's key-list length (for every replay of a graph)
};
constexpr int ATTN_ROW_KMAX = 512;  // the longest key list the row-resident attention holds in LDS
hipError_t attention(const AttnArgs& a, hipStream_t st);

hipError_t pack_inputs(const float* x0, const float* stat, bf16_t* a_in, float* x, int half, int mel, hipStream_t st);
hipError_t euler_update(float* x, const float* dphi, bf16_t* a_in, float* out, int half, int mel, float dt, float cfg,
                        hipStream_t st);

// Timestep conditioning tables (run once per model): rows of fp32 vectors.
hipError_t temb_sinusoid(const float* ts, const float* freqs, float* out, int S, int half, hipStream_t st);
hipError_t gemv_rows_f32(const float* in, int ld_in, int in_act, const float* W, const float* b, float* out, int ld_out,
                         int S, int O, int K, int out_act, hipStream_t st);
hipError_t add_one_cols(float* tab, int rows, int stride, int offset, int n, hipStream_t st);

hipError_t convert_rows_bf16(const float* src, bf16_t* dst, long long n, hipStream_t st);
hipError_t copy_rows_bf16(const bf16_t* src, bf16_t* dst, const int* src_row, const int* dst_row, int n_rows,
                          long long row_elems, hipStream_t st);

}  // namespace t2w
