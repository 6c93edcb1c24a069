/* C ABI of the MI355X Token2Wav hot path (libt2w_hip.so, gfx950).
 *
 * Plain pointers and sizes only.  Every tensor argument is a device pointer unless stated otherwise; weights are bf16
 * [out, in] row-major, biases / norm affines / tables fp32.  Every launch goes on the caller's stream (a hipStream_t
 * passed as void*); nothing here synchronises.  Functions return 0 on success, a nonzero status otherwise, with the
 * message in t2w_last_error() (thread-local).
 *
 * Reference interfaces replaced (paths in the reference repository):
 *   t2w_dit_solve        FastDiT.solve body (engine/runtime/dit_fast.py:269-344, graph replay :458-472) and
 *                        BatchedToken2Wav._solve (engine/runtime/token2wav_batch.py:632-702)
 *   t2w_dit_forward      BatchedToken2Wav._estimator_temb (engine/runtime/token2wav_batch.py:787-810)
 *   t2w_dit_build_mods   FastDiT._modulations (engine/runtime/dit_fast.py:157-178)
 *   t2w_gemm_bf16        F.linear of the block GEMMs (engine/runtime/dit_fast.py:283-301)
 *   t2w_attention        FlashInfer BatchPrefillWithPagedKVCacheWrapper.run (engine/runtime/dit_fast.py:291)
 *   t2w_qk_norm_scatter  dit_kernels.qk_norm_scatter (engine/runtime/dit_kernels.py:132-142)
 *   t2w_ln_mod           dit_kernels.ln_mod (engine/runtime/dit_kernels.py:27-31)
 *   t2w_hift_forward     hift_forward_noise + _hift_decode + istft_overlap_add (engine/models/token2wav.py:128-236),
 *                        with the hift_lean Snake / folded weight norm (engine/runtime/hift_lean.py:27-30, 107-134)
 *   t2w_graph_*          torch.cuda.CUDAGraph capture / replay of the solve and HiFT (dit_fast.py:392-422,
 *                        hift_graph.py:35-47)
 *   t2w_flow_encode      BatchedToken2Wav._encoder + _encoder_core + the encoder_proj of _flow_encode
 *                        (engine/runtime/token2wav_batch.py:42-79, 365-386, 402-444) and _setup_encoder_one /
 *                        _setup_encoder_batched (:556-616): UpsampleConformerEncoderV2.forward_chunk over many streams
 *   t2w_flow_speaker     spk_embed_affine_layer(F.normalize(spk)) (engine/runtime/token2wav_batch.py:375)
 */
#ifndef T2W_H
#define T2W_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int t2w_abi_version(void);
const char* t2w_last_error(void);

/* ---------------------------------------------------------------- DiT estimator and CFG Euler solve */

typedef struct t2w_dit t2w_dit;

typedef struct {
  int mel, hidden, depth, heads, head_dim, ffn, freq, steps;
  float eps_block, eps_qk, eps_conv, eps_final, cfg_rate;
} t2w_dit_dims;

typedef struct {
  const void* qkv_w; const float* qkv_b;     /* [3H, H]: to_q | to_k | to_v */
  const float* qn_w; const float* qn_b;       /* q_norm [64] */
  const float* kn_w; const float* kn_b;       /* k_norm [64] */
  const void* proj_w; const float* proj_b;    /* [H, H] */
  const void* c1_w; const float* c1_b;        /* [H, 3H] frame-major: tap 0 multiplies frame t-2 */
  const float* cln_w; const float* cln_b;     /* conv block LayerNorm [H] */
  const void* c2_w; const float* c2_b;        /* [H, 3H] */
  const void* fc1_w; const float* fc1_b;      /* [F, H] */
  const void* fc2_w; const float* fc2_b;      /* [H, F] */
} t2w_dit_block;

typedef struct {
  const void* in_w; const float* in_b;        /* [H, 4 mel]: x | mu | spk | cond */
  const void* out_w; const float* out_b;      /* [mel, H] */
  const float* mods;                          /* [steps, depth, 9, H]: shift, 1 + scale, gate of msa, mlp, conv */
  const float* final_mods;                    /* [steps, 2, H]: shift, 1 + scale */
  const float* dts;                           /* HOST pointer [steps]: Euler step sizes */
  const float* rope_freq;                     /* [head_dim / 2] or null.  No counterpart in the reference (its DiT has no
                                               * positional encoding): rotary embedding of q and k after their
                                               * LayerNorm, channel pair (2i, 2i + 1) of a head turned by the angle
                                               * tok_abs * rope_freq[i] (RoFormer); null = none, the reference's DiT */
} t2w_dit_globals;

/* fp8 copies of a block's six GEMM weights (no counterpart in the reference; its fp8 convention of
 * engine/runtime/fp8.py:15-37): OCP e4m3 codes with the same layouts as t2w_dit_block, and fp32 per-output-channel
 * scales max|w_n| / 448. */
typedef struct {
  const void* qkv_w8; const float* qkv_ws;
  const void* proj_w8; const float* proj_ws;
  const void* c1_w8; const float* c1_ws;
  const void* c2_w8; const float* c2_ws;
  const void* fc1_w8; const float* fc1_ws;
  const void* fc2_w8; const float* fc2_ws;
} t2w_dit_block_fp8;

int t2w_dit_create(const t2w_dit_dims* dims, t2w_dit** out);
int t2w_dit_set_block(t2w_dit* m, int block, const t2w_dit_block* w);
/* fp8 weights of a block; once every block has them, solves may set t2w_solve_args.fp8 */
int t2w_dit_set_block_fp8(t2w_dit* m, int block, const t2w_dit_block_fp8* w);
int t2w_dit_set_globals(t2w_dit* m, const t2w_dit_globals* g);
void t2w_dit_destroy(t2w_dit* m);

/* Timestep conditioning tables for S <= 16 t values (fp32 weights):
 * emb = [cos(1000 t f) | sin(1000 t f)]; temb = W2 silu(W0 emb + b0) + b2;
 * mods_out[s] = Wada silu(temb) + bada (depth * 9H values, then 1 added to the scale columns);
 * final_out[s] = Wfin silu(temb) + bfin (2H values, 1 added to the scale half). */
typedef struct {
  const float* freqs;                         /* [freq / 2] */
  const float* te0_w; const float* te0_b;     /* [H, freq] */
  const float* te2_w; const float* te2_b;     /* [H, H] */
  const float* ada_w; const float* ada_b;     /* [depth * 9H, H] */
  const float* fin_w; const float* fin_b;     /* [2H, H] */
} t2w_mod_weights;

size_t t2w_dit_mods_workspace_bytes(const t2w_dit* m, int S);
int t2w_dit_build_mods(const t2w_dit* m, const t2w_mod_weights* w, const float* ts, int S, float* mods_out,
                       float* final_out, void* workspace, void* stream);

/* One packed ragged call.  Rows 0..R/2-1 are the conditional rows of the requests, R/2..R-1 the unconditional rows in
 * the same order; a row's tokens are contiguous, the first half of the tokens belong to the conditional rows. */
typedef struct {
  int n_tok, n_rows, half, n_tiles, chunk;
  const float* x0;          /* [half, mel] initial noise of the conditional tokens */
  const float* stat;        /* [half, 3 mel]: mu | spk | cond of the conditional tokens (unconditional: zeros) */
  const float* in_rows;     /* t2w_dit_forward only: [n_tok, 4 mel] full estimator input rows */
  float* out;               /* solve: [half, mel] final x; forward: [n_tok, mel] dphi */
  const int* tok_row;       /* [n_tok] row of each token */
  const int* tok_pos;       /* [n_tok] position inside its row */
  const int* a_src;         /* [n_tok] tok + 2 * row: first frame of its conv window in the padded frame buffer */
  const int* new_slot;      /* [n_tok] key slot receiving the token's key / value */
  const int* row_start;     /* [R] */
  const int* row_len;       /* [R] */
  const int* row_kv_off;    /* [R] offset of the row's key list in kv_idx */
  const int* row_kv_len;    /* [R] length of the row's key list (its tokens first, then its cached keys) */
  const int* conv_rd;       /* [R] conv cache row slot read */
  const int* conv_wr;       /* [R] conv cache row slot written (never one that any row reads in this call) */
  const int* kv_idx;
  const int* tiles;         /* [n_tiles, 2] (row, first position) of each 64-query attention tile */
  void* k_pool;             /* [steps * depth, n_slots, H] bf16 */
  void* v_pool;
  long long pool_layer_stride;  /* n_slots * H */
  void* conv_pool;          /* [row slots, steps, depth, 2, 2, H] bf16 */
  void* workspace;
  size_t workspace_bytes;
  int fp8;                  /* 0: bf16 block GEMMs; 1: fp8 MFMA (e4m3 weights, MX fp8 activations); 2: e4m3 weights
                             * with per-output-channel scales dequantized to bf16 before each block GEMM, bf16
                             * activations and MFMA (1 and 2 need fp8 weights) */
  const int* tok_abs;       /* [n_tok] position of the token in its stream (frames of kept windows before it); read
                             * only with globals.rope_freq */
  int kv_max;               /* 0, or a bound on every row's key-list length (row_kv_len) in this call and in every replay
                             * of a graph captured from it; bounds up to 512 let the attention hold each row's keys in
                             * LDS (up to 256: two rows per CU).  A row longer than a stated bound gets NaN attention
                             * outputs. */
} t2w_solve_args;

/* includes the fp8 activation buffers once the model has fp8 weights */
size_t t2w_dit_workspace_bytes(const t2w_dit* m, int n_tok, int n_rows);
int t2w_dit_solve(const t2w_dit* m, const t2w_solve_args* a, void* stream);
/* t2w_dit_solve without a workspace, allocating nothing: for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops).  No counterpart in the reference.  The workspace is a static device array of
 * 32 MiB that the library holds on each device it runs on until the process ends; a->workspace and
 * a->workspace_bytes are ignored.  Calls needing more (t2w_dit_workspace_bytes() > 32 MiB: at hidden 1024 about 800
 * tokens) fail with a message.  Every call on a device shares that device's array, so calls that overlap on one
 * device (concurrent streams or threads) race; serialise them.  Nothing in it needs clearing between calls. */
int t2w_dit_solve_noalloc(const t2w_dit* m, const t2w_solve_args* a, void* stream);
/* Launch timer, a measurement aid (no counterpart in the reference).  t2w_timer_arm(cap) arms it on the calling
 * thread; the eager (not capturing) calls that follow bracket each instrumented kernel launch with a pair of HIP events
 * on its stream, up to cap launches.  t2w_timer_read waits for `stream`, writes the launches' kinds, durations (ms)
 * and algorithmic HBM bytes (the least its operands make it move) in launch order, up to cap, their count to *n,
 * and disarms.  Instrumented: the DiT's dense gated-residual tile GEMMs (proj and fc2 of every block, calls of more
 * than 128 tokens) and HiFT's elementwise kernels. */
enum {
  T2W_TIMER_RESID_GEMM = 1,
  T2W_TIMER_HIFT_PHASE = 2,
  T2W_TIMER_HIFT_SOURCE = 3,
  T2W_TIMER_HIFT_STFT = 4,
  T2W_TIMER_HIFT_ISTFT = 5,
  T2W_TIMER_HIFT_REFLECT = 6,
  T2W_TIMER_HIFT_SNAKE = 7,
  T2W_TIMER_HIFT_F0_HEAD = 8
};
int t2w_timer_arm(int cap);
int t2w_timer_read(void* stream, int* kinds, float* ms, double* bytes, int cap, int* n);
/* One estimator evaluation at Euler step `step`'s key/value and conv-cache layers with the given tables
 * (mods [depth, 9, H], final_mods [2, H]) on in_rows; writes dphi [n_tok, mel] to a->out. */
int t2w_dit_forward(const t2w_dit* m, const t2w_solve_args* a, int step, const float* mods, const float* final_mods,
                    void* stream);

/* ---------------------------------------------------------------- flow encoder (codec tokens -> mu) */

typedef struct t2w_flow t2w_flow;

/* dim % 512 == 0 with heads of 64; stride 2; relative positions |r| <= rmax - 1 are tabulated, so a stream may hold
 * at most rmax keys per stack in a call */
typedef struct {
  int vocab, dim, heads, ffn, depth1, depth2, look, stride, mel, spk, rmax;
  float eps_layer, eps_embed, eps_after;
} t2w_flow_dims;

/* one conformer layer: layers 0 .. depth1 - 1 before the upsampling, depth1 .. depth1 + depth2 - 1 after it */
typedef struct {
  const void* qkv_w; const float* qkv_b;      /* [3C, C]: linear_q | linear_k | linear_v */
  const float* pos_u; const float* pos_v;      /* pos_bias_u / pos_bias_v [C] (head h at h * 64) */
  const void* ptab;                            /* fp16 [2 rmax - 1, C]: linear_pos(sinusoid(r)) at row r + rmax - 1 */
  const void* out_w; const float* out_b;       /* linear_out [C, C] */
  const float* ln1_w; const float* ln1_b;      /* norm_mha */
  const float* ln2_w; const float* ln2_b;      /* norm_ff */
  const void* w1; const float* b1;             /* feed_forward.w_1 [ffn, C] (SiLU) */
  const void* w2; const float* b2;             /* feed_forward.w_2 [C, ffn] */
} t2w_flow_layer;

typedef struct {
  const float* embed_table;                    /* fp32 [vocab, C]: input_embedding rows through the embed Linear */
  const float* embed_ln_w; const float* embed_ln_b;
  const void* conv1_w; const float* conv1_b;   /* pre-lookahead conv1 [C, (look + 1) C] frame-major */
  const void* conv2_w; const float* conv2_b;   /* pre-lookahead conv2 [C, 3C] frame-major (tap 0: frame t - 2) */
  const void* up_w; const float* up_b;         /* [C, (2 stride + 1) C]: the up_layer conv followed by up_embed's Linear */
  const float* up_ln_w; const float* up_ln_b;  /* up_embed LayerNorm */
  const float* after_w; const float* after_b;  /* after_norm */
  const void* proj_w; const float* proj_b;     /* encoder_proj [mel, C] */
  const float* spk_w; const float* spk_b;      /* fp32 spk_embed_affine_layer [mel, spk] */
  const float* ones;                           /* [C] of 1.0 (the residual adds use the gated-residual epilogue) */
} t2w_flow_globals;

/* One packed ragged call over R streams (see flow_capi.hip for the row layout).  Stream s: T1 = t1[s] frames (its
 * window's tokens less the lookahead, or all of a final window's), T2 = stride T1. */
typedef struct {
  int n_rows, n_in, n_gap, n1, n_up, n2, n_tiles1, n_tiles2;  /* n_in = n1 + look R, n_gap = n1 + 2R, n2 = 2 n1, n_up = n2 + 4R */
  const int* tok;        /* [n_in] token of each conv1 input row, -1: zero row (a final window's lookahead) */
  const int* res;        /* [n_in] h1 row that the embedded row also starts, -1: none (lookahead rows) */
  const int* c1_src;     /* [n_gap] conv1 taps: first input row (any valid row for the two cache rows of a stream) */
  const int* gofs;       /* [R] first row of the stream in the conv1 output (its two cached frames) */
  const int* t1;         /* [R] */
  const int* c2_src;     /* [n1] conv2 taps: first row in the conv1 output (gofs + t) */
  const int* up_dst;     /* [n1] row of the first upsampled copy of stack-1 row m (uofs + 4 + 2t) */
  const int* uofs;       /* [R] first row of the stream in the upsampling input (its four cached frames) */
  const int* o1;         /* [R] first stack-1 row */
  const int* up_src;     /* [n2] upsampling conv taps: uofs + f */
  const int* o2;         /* [R] first stack-2 row */
  const int* t2;         /* [R] */
  const int* cnn_rd;     /* [R] conv-cache slot read (a zero slot for an empty cache) */
  const int* cnn_wr;     /* [R] conv-cache slot written (never one any stream of the call reads) */
  const int* new1;       /* [n1] pool slot receiving each stack-1 row's keys / values */
  const int* new2;       /* [n2] */
  const int* kv1_idx; const int* kv1_off; const int* kv1_len; const int* tiles1;  /* stack-1 key lists, [n_tiles1, 2] */
  const int* kv2_idx; const int* kv2_off; const int* kv2_len; const int* tiles2;
  void* pool1; long long pool1_layer_stride;  /* fp16 [depth1][slots][2C] (k | v), stride in elements */
  void* pool2; long long pool2_layer_stride;  /* fp16 [depth2][slots][2C] */
  void* cnn_pool;        /* bf16 [slots][(2 + 2 stride) C]: two pre-lookahead frames, then 2 stride upsampled frames */
  float* mu_out;         /* [n2, mel] */
  void* workspace;
  size_t workspace_bytes;
} t2w_flow_args;

int t2w_flow_create(const t2w_flow_dims* dims, t2w_flow** out);
int t2w_flow_set_layer(t2w_flow* m, int layer, const t2w_flow_layer* w);
int t2w_flow_set_globals(t2w_flow* m, const t2w_flow_globals* g);
void t2w_flow_destroy(t2w_flow* m);
size_t t2w_flow_workspace_bytes(const t2w_flow* m, int n_in, int n_gap, int n1, int n_up, int n2);
int t2w_flow_encode(const t2w_flow* m, const t2w_flow_args* a, void* stream);
/* out [R, mel] = spk_w F.normalize(spk [R, spk]) + spk_b */
int t2w_flow_speaker(const t2w_flow* m, const float* spk, float* out, int R, void* stream);

/* ---------------------------------------------------------------- kernel-level entry points (tests, benchmarks) */

/* C = A . W^T + bias; epi 0: bf16 out, 1: GELU-tanh bf16 out, 2: C(fp16) = fp16(C + gate * (.)) (the gated residual
 * stream, fp16 as the reference's activations, fp32 arithmetic), 3: fp32 out, 7: fp16 out.
 * a_src non-null: conv taps mode, A row m = frames a_src[m] .. a_src[m] + K / lda - 1 of A (rows lda wide).
 * Calls of at most 128 rows (K <= 3072, ldc % 4 == 0) run as one kernel that splits K over the waves of a workgroup;
 * larger ones on the tile GEMM (16-bit outputs: ldc % 8 == 0 and C 16-byte aligned there). */
int t2w_gemm_bf16(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate,
                  void* C, int ldc, int M, int N, int K, int epi, void* stream);
/* t2w_gemm_bf16 with an explicit tile configuration (-1: chosen by shape; 0: 128x128 of 4 waves, 1: 256x256 of
 * 8 waves, 2: 256x128 of 8 waves, 3: 208x256 of 8 waves) for tile sweeps.
 * K % 64 == 0, lda % 8 == 0 (taps mode: lda % 64 == 0). */
int t2w_gemm_bf16_tile(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate,
                       void* C, int ldc, int M, int N, int K, int epi, int tile, void* stream);
/* t2w_gemm_bf16 with a workspace for split-K partials (256-byte aligned; up to splits x M x N fp32): a call whose tile
 * grid would leave most CUs idle (few rows) splits K over ~512 waves and reduces the partials in a fixed order. */
int t2w_gemm_bf16_ws(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate,
                     void* C, int ldc, int M, int N, int K, int epi, void* workspace, size_t workspace_bytes,
                     void* stream);
/* MX fp8 quantization (no counterpart in the reference; the fp8 weight convention of engine/runtime/fp8.py:15-37 with
 * activations in 32-value K blocks): x [M, K] bf16 -> q [M, K] OCP e4m3 and scales [M, K / 32] E8M0, each block scaled
 * by the smallest power of two that keeps its largest magnitude within 448.  K % 32 == 0. */
int t2w_quant_mx8(const void* x, int ldx, int M, int K, void* q, int ldq, void* scales, void* stream);
/* C = epilogue(dequant(A) . dequant(W)^T + bias) on fp8 MFMA: A [M, K] e4m3 with MX scales a_scale[row * a_sld + k / 32]
 * (taps mode as t2w_gemm_bf16, rows = frames), W [N, K] e4m3 scaled per output channel by w_scale[N].  K % 128 == 0. */
int t2w_gemm_fp8(const void* A, int lda, const int* a_src, const void* a_scale, int a_sld, const void* W, const float* w_scale,
                 const float* bias, const float* gate, void* C, int ldc, int M, int N, int K, int epi, void* stream);
/* LayerNorm (no affine) of the fp16 residual rows h [N, H], then * scale1 + shift (fp32), out bf16 [N, H] */
int t2w_ln_mod(const void* h, const float* shift, const float* scale1, float eps, void* out, int N, int H,
               void* stream);
int t2w_qk_norm_scatter(const void* qkv, const float* qw, const float* qb, const float* kw, const float* kb, float eps,
                        void* q_out, void* k_pool, void* v_pool, const int* slots, int N, int heads, void* stream);
/* Block-causal attention of packed rows over paged key slots: q [N, heads * 64]; row r's queries are tokens
 * row_start[r] .. + row_len[r], its keys the slots kv_idx[row_kv_off[r] ..][0 .. row_kv_len[r]) (its new tokens first,
 * then cached keys); tiles [n_tiles, 2] lists (row, first query) of every 64-query tile.  chunk > 0: a new token sees
 * the new tokens of its own and earlier chunks only; cached keys are always visible.  n_rows: rows of the call;
 * kv_max: 0, or a bound on every row_kv_len[r] (as t2w_solve_args.kv_max; bounds up to 512 select the row-resident
 * kernel on calls of 256 or more (row, head) pairs whose rows average three or more 64-query tiles). */
int t2w_attention(const void* q, const void* k_pool, const void* v_pool, void* out, const int* kv_idx,
                  const int* row_start, const int* row_len, const int* row_kv_off, const int* row_kv_len,
                  const int* tiles, int n_tiles, int heads, int chunk, float scale, int n_rows, int kv_max,
                  void* stream);

/* ---------------------------------------------------------------- HiFT vocoder (fp32) */

typedef struct t2w_hift t2w_hift;

typedef struct {
  int mel, base, n_up, harmonics, f0_channels, f0_layers, sr, n_fft, hop;
  int up_rates[3], up_kernels[3], res_kernels[3], res_dilations[3], src_kernels[3];
  float sine_amp, noise_std, voiced_threshold, lrelu_slope, audio_limit;
} t2w_hift_dims;

typedef struct {
  const float* w; const float* b;  /* w [Cout, taps, Cin]; transposed convs: [u, Cout, ceil(k / u), Cin] polyphase */
  const void* wbf;                 /* optional bf16 copy [phases, Cout padded to 64, taps, Cin padded to 64] (zeros in
                                      the padding) for the bf16-MFMA decoder; null: the conv always runs fp32 */
} t2w_conv;
typedef struct {
  t2w_conv c1[3], c2[3];
  const float* a1[3]; const float* inv1[3];  /* Snake alpha and 1 / (alpha + 1e-9) before convs1[j] */
  const float* a2[3]; const float* inv2[3];
} t2w_resblock;

typedef struct {
  t2w_conv f0[5]; const float* f0_head_w; const float* f0_head_b;  /* f0 predictor: 5 x (conv k3 + ELU), Linear(C -> 1) */
  const float* src_w; const float* src_b;                           /* NSF merge Linear(harmonics + 1 -> 1) */
  t2w_conv conv_pre, ups[3], src_down[3], conv_post;
  t2w_resblock src_res[3], res[9];
  const float* window;                                              /* [n_fft] periodic Hann */
} t2w_hift_weights;

/* The handle keeps the weight pointers (the caller keeps the weights alive) and, for every conv with a bf16 copy, makes a
 * device copy of it in the MFMA operand order its kernels read (the same size; freed by t2w_hift_destroy); the copies
 * are made on the null stream and are complete when create returns.  The bf16 weights are read only there: writes to
 * them after create are not seen by the bf16 convs (create a new handle).  So are the fp32 weights of the three source
 * downsampling convs (src_down[i].w, required), copied with their 18 input channels padded to 32; the other fp32
 * weights are read at every call. */
int t2w_hift_create(const t2w_hift_dims* dims, const t2w_hift_weights* w, t2w_hift** out);
void t2w_hift_destroy(t2w_hift* h);
/* Plan of a call over n_items rows with frames[i] mel frames (host array): ints for t2w_hift_plan to fill, which the
 * caller copies to device memory; workspace bytes. */
int t2w_hift_plan_ints(int n_items);
int t2w_hift_plan(const t2w_hift* h, int n_items, const int* frames, int* plan_host);
size_t t2w_hift_workspace_bytes(const t2w_hift* h, int n_items, const int* frames);
/* hift_forward_noise for rows of different lengths, time-major and packed: mel [sum T, mel]; noise [sum 480 T, harmonics
 * + 1]; cache_source [n_items, S] replaces each row's first S source samples; speech / source out [sum 480 T].
 * f0_override / source_override (optional, device): use these instead of the f0 predictor / the NSF source. f0_out
 * (optional): the f0 used [sum T]. */
int t2w_hift_forward(const t2w_hift* h, int n_items, const int* frames, const int* plan_dev, const float* mel,
                     const float* noise, const float* cache_source, int S, const float* f0_override,
                     const float* source_override, float* speech, float* source, float* f0_out, void* workspace,
                     size_t workspace_bytes, int decode_bf16, void* stream);
/* decode_bf16: nonzero puts the decoder's stride-1 and transposed convs (conv_pre, upsampling, ResBlocks, conv_post) on
 * bf16 MFMA with fp32 activations and accumulation; the f0 predictor, the NSF source, the source downsampling convs, STFT
 * and ISTFT stay fp32.  Its value picks how a ResBlock dilation's two convs run: 1 as one kernel that keeps the first
 * conv's output on chip where the call's grid fills the chip (else as two convs), 2 always as two convs, 3 as one kernel
 * wherever the channel count allows (64, 128 or 256).  The modes give the same result up to the order of fp32 sums. */

/* ---------------------------------------------------------------- co-scheduling on one GPU (CU-masked streams)
 * The reference runs Token2Wav in a worker process of its own beside the Thinker/Talker and shares the GPU through CUDA
 * MPS (engine/runtime/t2w_worker.py:858-924, scripts/serve_engine.sh:1-45).  Here the module can run in the engine's
 * own process on a stream of its own, optionally restricted to a set of CUs, so the two share the GPU without a
 * separate process: t2w_stream_create_cu_mask makes a stream of the current device whose kernels (graph replays
 * included) run only on the CUs whose bits are set in mask[0 .. n_words) (bit i of word w = CU 32 w + i), at the
 * default priority.  Each word must hold one run of at least 8 consecutive bits, or none: the runtime fails to create
 * queues whose masks interleave single CUs or leave a group fewer than 8, and such masks are refused here.
 * t2w_device_cus gives the current device's CU count.  Release the stream with
 * t2w_stream_destroy (after its work is done). */
int t2w_device_cus(int* n);
int t2w_stream_create_cu_mask(const uint32_t* mask, int n_words, void** out);
int t2w_stream_destroy(void* stream);

/* ---------------------------------------------------------------- graphs (hipGraph capture of a stream) */

typedef struct t2w_graph t2w_graph;
int t2w_graph_begin(void* stream);
int t2w_graph_end(void* stream, t2w_graph** out);
int t2w_graph_launch(t2w_graph* g, void* stream);
void t2w_graph_destroy(t2w_graph* g);

#ifdef __cplusplus
}
#endif

#endif /* T2W_H */
