// C-ABI of the flow encoder: the model object and one packed ragged encoder call over many streams' windows
// (engine/runtime/token2wav_batch.py:365-444 with _encoder_core :42-79), plus the speaker affine layer (:375).
//
// Layout of a call (R streams; stream s has T1 frames after its pre-lookahead conv and T2 = stride * T1 after the
// upsampling): the conv1 input x0 has T1 + look rows per stream (tokens, then the zero lookahead of a final window); the
// conv1 output G has 2 + T1 rows per stream (its two cached frames first, so conv2 is a taps GEMM); the stack-1
// residual stream h1 T1 rows; the upsampling input U 4 + 2 T1 rows (cached frames, then each stack-1 frame twice); the
// stack-2 residual stream h2 T2 rows.  Keys and values of every layer live in fp16 slot pools; each stream's key list
// (cached frames, then its new frames) is given per call.  Nothing here allocates: the caller passes a workspace of
// t2w_flow_workspace_bytes().
#include <hip/hip_runtime.h>

#include <cmath>
#include <vector>

#include "../../include/t2w.h"
#include "flow_internal.h"
#include "t2w_internal.h"

using namespace t2w;

namespace t2w {
int set_error(const char* what, hipError_t e);
}

namespace {

int ferr(const char* what, hipError_t e = hipSuccess) { return set_error(what, e); }

#define T2W_FCHECK(expr, what)                    \
  do {                                            \
    hipError_t e_ = (expr);                       \
    if (e_ != hipSuccess) return ferr(what, e_);  \
  } while (0)

size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

constexpr size_t FLOW_SPLITK_BYTES = (size_t)16 << 20;

struct FWork {
  bf16_t* x0; bf16_t* G; f16_t* h1; bf16_t* U; float* Y; f16_t* h2; bf16_t* A; f16_t* qkv; bf16_t* ao; bf16_t* F;
  float* part;
};

size_t fcarve(const t2w_flow_dims& d, int n_in, int n_gap, int n1, int n_up, int n2, char* base, FWork* w) {
  const size_t C = d.dim, nm = (size_t)(n1 > n2 ? n1 : n2);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return base ? (void*)(base + o) : nullptr; };
  FWork t;
  t.x0 = (bf16_t*)take((size_t)n_in * C * 2);
  t.G = (bf16_t*)take((size_t)n_gap * C * 2);
  t.h1 = (f16_t*)take((size_t)n1 * C * 2);
  t.U = (bf16_t*)take((size_t)n_up * C * 2);
  t.Y = (float*)take((size_t)n2 * C * 4);
  t.h2 = (f16_t*)take((size_t)n2 * C * 2);
  t.A = (bf16_t*)take(nm * C * 2);
  t.qkv = (f16_t*)take(nm * 3 * C * 2);
  t.ao = (bf16_t*)take(nm * C * 2);
  t.F = (bf16_t*)take(nm * (size_t)d.ffn * 2);
  t.part = (float*)take(FLOW_SPLITK_BYTES);
  if (w) *w = t;
  return off;
}

GemmArgs fgemm(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate, void* C, int ldc,
               int M, int N, int K, const FWork& w, int act = ACT_NONE) {
  GemmArgs g{};
  g.ws = w.part;
  g.ws_bytes = FLOW_SPLITK_BYTES;
  g.A = (const bf16_t*)A;
  g.lda = lda;
  g.a_src = a_src;
  g.tapC = lda;
  g.B = (const bf16_t*)W;
  g.ldb = K;
  g.bias = bias;
  g.gate = gate;
  g.C = C;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  g.act = act;
  return g;
}

}  // namespace

struct t2w_flow {
  t2w_flow_dims d;
  std::vector<t2w_flow_layer> layers;
  std::vector<bool> layer_set;
  t2w_flow_globals g;
  bool globals_set = false;
};

int t2w_flow_create(const t2w_flow_dims* dims, t2w_flow** out) {
  if (!dims || !out) return ferr("null argument");
  const t2w_flow_dims& d = *dims;
  if (d.dim % 512 || d.heads * 64 != d.dim) return ferr("flow encoder: width must be a multiple of 512 with heads of 64");
  if (d.ffn % 64 || d.ffn <= 0) return ferr("flow encoder: ffn must be a positive multiple of 64");
  if (d.depth1 < 1 || d.depth2 < 1 || d.look < 1 || d.stride != 2 || d.mel <= 0 || d.spk <= 0 || d.rmax < 2)
    return ferr("flow encoder: bad dimensions (stride must be 2)");
  t2w_flow* m = new t2w_flow();
  m->d = d;
  m->layers.resize(d.depth1 + d.depth2);
  m->layer_set.assign(d.depth1 + d.depth2, false);
  *out = m;
  return 0;
}

int t2w_flow_set_layer(t2w_flow* m, int layer, const t2w_flow_layer* w) {
  if (!m || !w) return ferr("null argument");
  if (layer < 0 || layer >= (int)m->layers.size()) return ferr("flow encoder: layer index out of range");
  m->layers[layer] = *w;
  m->layer_set[layer] = true;
  return 0;
}

int t2w_flow_set_globals(t2w_flow* m, const t2w_flow_globals* g) {
  if (!m || !g) return ferr("null argument");
  m->g = *g;
  m->globals_set = true;
  return 0;
}

void t2w_flow_destroy(t2w_flow* m) { delete m; }

size_t t2w_flow_workspace_bytes(const t2w_flow* m, int n_in, int n_gap, int n1, int n_up, int n2) {
  if (!m) return 0;
  return fcarve(m->d, n_in, n_gap, n1, n_up, n2, nullptr, nullptr);
}

namespace {

int check_flow(const t2w_flow* m) {
  if (!m) return ferr("null model");
  if (!m->globals_set) return ferr("flow encoder globals not set");
  for (bool b : m->layer_set)
    if (!b) return ferr("flow encoder layer weights not set");
  return 0;
}

// one conformer layer on the residual stream h (n rows): pre-norm relative-position attention, then the SiLU FFN
int run_layer(const t2w_flow* m, const t2w_flow_layer& k, f16_t* h, int n, bool normed, f16_t* pool, const int* new_slot,
              const int* kv_idx, const int* kv_off, const int* kv_len, const int* row_start, const int* row_len, const int* tiles,
              int n_tiles, const FWork& w, hipStream_t st) {
  const t2w_flow_dims& d = m->d;
  const int C = d.dim;
  if (!normed) T2W_FCHECK(ln_mod(h, k.ln1_b, k.ln1_w, d.eps_layer, w.A, n, C, st), "flow norm_mha");
  T2W_FCHECK(gemm_bf16(fgemm(w.A, C, nullptr, k.qkv_w, k.qkv_b, nullptr, w.qkv, 3 * C, n, 3 * C, C, w), EPI_F16, st), "flow qkv");
  T2W_FCHECK(flow_kv_store(w.qkv, 3 * C, pool, new_slot, n, C, st), "flow key/value store");
  RelAttnArgs a{};
  a.qkv = w.qkv;
  a.ldq = 3 * C;
  a.pool = pool;
  a.ptab = (const f16_t*)k.ptab;
  a.rmax = d.rmax;
  a.bias_u = k.pos_u;
  a.bias_v = k.pos_v;
  a.out = w.ao;
  a.kv_idx = kv_idx;
  a.kv_off = kv_off;
  a.kv_len = kv_len;
  a.row_start = row_start;
  a.row_len = row_len;
  a.tiles = tiles;
  a.n_tiles = n_tiles;
  a.heads = d.heads;
  a.scale = 1.0f / sqrtf(64.0f);
  T2W_FCHECK(flow_rel_attention(a, st), "flow attention");
  T2W_FCHECK(gemm_bf16(fgemm(w.ao, C, nullptr, k.out_w, k.out_b, m->g.ones, h, C, n, C, C, w), EPI_RESID_F16, st), "flow linear_out");
  T2W_FCHECK(ln_mod(h, k.ln2_b, k.ln2_w, d.eps_layer, w.A, n, C, st), "flow norm_ff");
  T2W_FCHECK(gemm_bf16(fgemm(w.A, C, nullptr, k.w1, k.b1, nullptr, w.F, d.ffn, n, d.ffn, C, w, ACT_SILU), EPI_BF16, st), "flow w_1");
  T2W_FCHECK(gemm_bf16(fgemm(w.F, d.ffn, nullptr, k.w2, k.b2, m->g.ones, h, C, n, C, d.ffn, w), EPI_RESID_F16, st), "flow w_2");
  return 0;
}

}  // namespace

int t2w_flow_encode(const t2w_flow* m, const t2w_flow_args* a, void* stream) {
  if (check_flow(m)) return 1;
  if (!a) return ferr("null arguments");
  const t2w_flow_dims& d = m->d;
  const t2w_flow_globals& g = m->g;
  const int C = d.dim, R = a->n_rows;
  if (R <= 0) return 0;
  if (a->n1 <= 0 || a->n2 != d.stride * a->n1 || a->n_in != a->n1 + R * d.look || a->n_gap != a->n1 + 2 * R ||
      a->n_up != a->n2 + 2 * d.stride * R)
    return ferr("flow encoder: inconsistent row counts (n_in = n1 + look R, n_gap = n1 + 2 R, n2 = stride n1, n_up = n2 + 2 stride R)");
  if (!a->tok || !a->res || !a->c1_src || !a->gofs || !a->t1 || !a->c2_src || !a->up_dst || !a->uofs || !a->o1 || !a->up_src ||
      !a->cnn_rd || !a->cnn_wr || !a->new1 || !a->new2 || !a->kv1_idx || !a->kv1_off || !a->kv1_len || !a->tiles1 || !a->o2 ||
      !a->t2 || !a->kv2_idx || !a->kv2_off || !a->kv2_len || !a->tiles2 || !a->pool1 || !a->pool2 || !a->cnn_pool || !a->mu_out)
    return ferr("flow encoder: null argument pointer");
  if (!a->workspace || ((uintptr_t)a->workspace & 255)) return ferr("flow encoder: workspace missing or not 256-byte aligned");
  FWork w;
  const size_t need = fcarve(d, a->n_in, a->n_gap, a->n1, a->n_up, a->n2, (char*)a->workspace, &w);
  if (a->workspace_bytes < need) return ferr("flow encoder: workspace too small");
  const hipStream_t st = (hipStream_t)stream;
  const float xscale = sqrtf((float)C);
  const long long cstride = (long long)(2 + 2 * d.stride) * C;
  bf16_t* cnn = (bf16_t*)a->cnn_pool;

  // embedding (table row, LayerNorm, x sqrt(C)) of every token; the first T1 of each stream start h1
  T2W_FCHECK(flow_embed(g.embed_table, a->tok, a->res, g.embed_ln_w, g.embed_ln_b, d.eps_embed, xscale, w.x0, w.h1, a->n_in, C, st),
             "flow embed");
  // pre-lookahead layer: conv1 over each frame and its lookahead (leaky ReLU), its cached frames, conv2 + residual
  T2W_FCHECK(gemm_bf16(fgemm(w.x0, C, a->c1_src, g.conv1_w, g.conv1_b, nullptr, w.G, C, a->n_gap, C, (d.look + 1) * C, w, ACT_LRELU),
                       EPI_BF16, st), "flow pre-lookahead conv1");
  T2W_FCHECK(flow_look_place(w.G, cnn, a->gofs, a->t1, a->cnn_rd, a->cnn_wr, R, C, cstride, st), "flow pre-lookahead cache");
  T2W_FCHECK(gemm_bf16(fgemm(w.G, C, a->c2_src, g.conv2_w, g.conv2_b, g.ones, w.h1, C, a->n1, C, 3 * C, w), EPI_RESID_F16, st),
             "flow pre-lookahead conv2");
  f16_t* pool1 = (f16_t*)a->pool1;
  for (int l = 0; l < d.depth1; ++l)
    if (run_layer(m, m->layers[l], w.h1, a->n1, false, pool1 + (size_t)l * a->pool1_layer_stride, a->new1, a->kv1_idx, a->kv1_off,
                  a->kv1_len, a->o1, a->t1, a->tiles1, a->n_tiles1, w, st))
      return 1;
  // 2x upsampling (nearest, then the conv over 4 cached frames) composed with the up_embed Linear, its LayerNorm and
  // x sqrt(C), and the first up layer's norm
  T2W_FCHECK(flow_up_place(w.h1, w.U, a->up_dst, a->n1, a->uofs, a->o1, a->t1, cnn, a->cnn_rd, a->cnn_wr, R, C, cstride, st),
             "flow upsample frames");
  T2W_FCHECK(gemm_bf16(fgemm(w.U, C, a->up_src, g.up_w, g.up_b, nullptr, w.Y, C, a->n2, C, (2 * d.stride + 1) * C, w), EPI_F32, st),
             "flow upsample conv");
  const t2w_flow_layer& u0 = m->layers[d.depth1];
  T2W_FCHECK(flow_ln_scale_ln(w.Y, g.up_ln_w, g.up_ln_b, d.eps_embed, xscale, w.h2, u0.ln1_w, u0.ln1_b, d.eps_layer, w.A, a->n2, C, st),
             "flow up_embed norm");
  f16_t* pool2 = (f16_t*)a->pool2;
  for (int l = 0; l < d.depth2; ++l)
    if (run_layer(m, m->layers[d.depth1 + l], w.h2, a->n2, l == 0, pool2 + (size_t)l * a->pool2_layer_stride, a->new2, a->kv2_idx,
                  a->kv2_off, a->kv2_len, a->o2, a->t2, a->tiles2, a->n_tiles2, w, st))
      return 1;
  T2W_FCHECK(ln_mod(w.h2, g.after_b, g.after_w, d.eps_after, w.A, a->n2, C, st), "flow after_norm");
  T2W_FCHECK(gemm_bf16(fgemm(w.A, C, nullptr, g.proj_w, g.proj_b, nullptr, a->mu_out, d.mel, a->n2, d.mel, C, w), EPI_F32, st),
             "flow encoder_proj");
  return 0;
}

int t2w_flow_speaker(const t2w_flow* m, const float* spk, float* out, int R, void* stream) {
  if (check_flow(m)) return 1;
  if (!spk || !out) return ferr("null argument");
  T2W_FCHECK(flow_speaker(spk, m->g.spk_w, m->g.spk_b, out, R, m->d.spk, m->d.mel, (hipStream_t)stream), "flow speaker affine");
  return 0;
}
