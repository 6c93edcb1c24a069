// C-ABI layer: the DiT model object, the whole CFG Euler solve as one call, kernel-level entry points and hipGraph
// capture.  No allocation happens in any compute call: the caller passes a workspace of t2w_dit_workspace_bytes().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/t2w.h"
#include "t2w_internal.h"

using namespace t2w;

namespace {

thread_local std::string g_err;

int fail(const char* what, hipError_t e = hipSuccess) {
  char buf[512];
  if (e != hipSuccess)
    snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
  else
    snprintf(buf, sizeof buf, "%s", what);
  g_err = buf;
  return 1;
}

#define T2W_CHECK(expr, what)                 \
  do {                                        \
    hipError_t e_ = (expr);                   \
    if (e_ != hipSuccess) return fail(what, e_); \
  } while (0)

size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

namespace t2w {
int set_error(const char* what, hipError_t e) { return fail(what, e); }
LaunchTimer& launch_timer() {
  thread_local LaunchTimer t;
  return t;
}
}  // namespace t2w

namespace {
// HBM bytes a gated-residual GEMM of M rows must move at least: A [M, K] bf16, W [N, K] bf16, the fp16 residual
// read and written, bias and gate
double resid_bytes(int M, int N, int K) { return 2.0 * M * K + 2.0 * N * K + 4.0 * M * N + 8.0 * N; }
}  // namespace

// Scratch of t2w_dit_solve_noalloc: the solve's whole workspace (activations, split-K partials) for calls that fit,
// in device memory the library owns.  Each device holds its own copy from module load until the process ends; host
// code only ever uses the per-device address hipGetSymbolAddress returns (the symbol itself names a host stand-in).
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_dev;  // device ordinal -> address of that device's scratch (null until looked up)

// The current device's scratch address, looked up once per device (the current device must be the one asked about).
int scratch_address(void** out) {
  int dev = 0;
  T2W_CHECK(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if ((size_t)dev >= g_scratch_dev.size()) g_scratch_dev.resize(dev + 1, nullptr);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    T2W_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return fail("hipGetSymbolAddress(scratch) returned null");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}

}  // namespace

struct t2w_dit {
  t2w_dit_dims d;
  std::vector<t2w_dit_block> blocks;
  std::vector<bool> block_set;
  std::vector<t2w_dit_block_fp8> blocks8;
  std::vector<bool> block8_set;
  bool fp8_ready() const {
    for (bool b : block8_set)
      if (!b) return false;
    return !block8_set.empty();
  }
  t2w_dit_globals g;
  std::vector<float> dts;
  bool globals_set = false;
};

namespace {

struct Work {  // carve of the caller's workspace for n tokens, R rows
  bf16_t* a_in; float* x; f16_t* h; bf16_t* abuf; bf16_t* big; bf16_t* q; bf16_t* ao; bf16_t* P; float* dphi;
  float* part; size_t part_bytes;  // split-K partials of the GEMMs of calls with few tokens
  // fp8 mode: MX fp8 activations (codes, block scales) of the qkv / fc1 inputs, the attention output, the conv frame
  // buffer and the fc1 output
  uint8_t *a8, *a8s, *o8, *o8s, *P8, *P8s, *b8, *b8s;
  bf16_t* wdq;  // fp8 weight-only mode: the current GEMM's weights dequantized to bf16
};

// calls of up to this many tokens get a split-K partial area of SPLITK_BYTES
constexpr int SPLITK_MAX_TOK = 1024;
constexpr size_t SPLITK_BYTES = (size_t)16 << 20;

size_t carve(const t2w_dit_dims& d, int N, int R, bool fp8, char* base, Work* w) {
  const int H = d.hidden, M = d.mel;
  const size_t bigc = (size_t)N * (size_t)(3 * H > d.ffn ? 3 * H : d.ffn);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align_up(off + bytes); return base ? (void*)(base + o) : nullptr; };
  Work t;
  t.a_in = (bf16_t*)take((size_t)N * 4 * M * 2);
  t.x = (float*)take((size_t)N * M * 4);
  t.h = (f16_t*)take((size_t)N * H * 2);  // the residual stream, fp16
  t.abuf = (bf16_t*)take((size_t)N * H * 2);
  t.big = (bf16_t*)take(bigc * 2);
  t.q = (bf16_t*)take((size_t)N * H * 2);
  t.ao = (bf16_t*)take((size_t)N * H * 2);
  t.P = (bf16_t*)take((size_t)(N + 2 * R) * H * 2);
  t.dphi = (float*)take((size_t)N * M * 4);
  t.part_bytes = N <= SPLITK_MAX_TOK ? SPLITK_BYTES : 0;
  t.part = t.part_bytes ? (float*)take(t.part_bytes) : nullptr;
  t.a8 = t.a8s = t.o8 = t.o8s = t.P8 = t.P8s = t.b8 = t.b8s = nullptr;
  t.wdq = nullptr;
  if (fp8) {
    const size_t wmax = std::max((size_t)3 * H * H, (size_t)H * d.ffn);
    t.wdq = (bf16_t*)take(wmax * 2);
    const size_t F = (size_t)d.ffn, NP = (size_t)N + 2 * R;
    t.a8 = (uint8_t*)take((size_t)N * H); t.a8s = (uint8_t*)take((size_t)N * H / 32);
    t.o8 = (uint8_t*)take((size_t)N * H); t.o8s = (uint8_t*)take((size_t)N * H / 32);
    t.P8 = (uint8_t*)take(NP * H); t.P8s = (uint8_t*)take(NP * H / 32);
    t.b8 = (uint8_t*)take((size_t)N * F); t.b8s = (uint8_t*)take((size_t)N * F / 32);
  }
  if (w) *w = t;
  return off;
}

int check_model(const t2w_dit* m) {
  if (!m) return fail("null model");
  if (!m->globals_set) return fail("model globals not set");
  for (size_t b = 0; b < m->block_set.size(); ++b)
    if (!m->block_set[b]) return fail("model block weights not set");
  return 0;
}

GemmArgs gemm_args(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate, void* C,
                   int ldc, int M, int N, int K, const Work* w = nullptr) {
  GemmArgs g{};
  g.ws = w ? w->part : nullptr;
  g.ws_bytes = w ? w->part_bytes : 0;
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
  return g;
}

// fp8 GEMM: A as MX fp8 codes with block scales (rows a_sld apart), W as e4m3 codes with per-channel scales
GemmArgs gemm8(const uint8_t* A, int lda, const int* a_src, const uint8_t* as, const void* W8, const float* ws,
               const float* bias, const float* gate, void* C, int ldc, int M, int N, int K) {
  GemmArgs g = gemm_args(A, lda, a_src, W8, bias, gate, C, ldc, M, N, K);
  g.a_scale = as;
  g.a_sld = lda / 32;
  g.w_scale = ws;
  return g;
}

// K splits of the deferred GEMMs of a call of N tokens (0: no deferral): enough workgroups to occupy the 256 CUs, at
// most 4 (the row kernels' limit), and the sums must fit the partial area; 0 unless the deferred GEMMs of the kind fit
// the small-row kernel.  The conv GEMMs (taps) run on 64-row tiles above 32 tokens (gemm_small_part64), proj and fc2
// on 32-row tiles (measured faster for them: K = 1024 / 2048 leaves 64-row tiles too few steps per workgroup).
int defer_splits(const t2w_dit_dims& d, int N, const Work& w, bool taps) {
  const int H = d.hidden;
  if (N > GEMM_SMALL_MAX_M || !w.part) return 0;
  const int rows = taps && N > 32 ? 64 : 32;
  const int tiles = ((N + rows - 1) / rows) * ((H + 31) / 32);
  const int S = std::min(4, 256 / tiles);
  if (S < 2 || (size_t)S * N * H * 4 > w.part_bytes) return 0;
  static const int taps_marker = 0;  // gemm_small_fits checks only the presence of a frame id list
  GemmArgs g{};
  g.M = N; g.N = H; g.ldc = H; g.splits = S; g.tapC = H;
  for (int K : taps ? std::initializer_list<int>{3 * H} : std::initializer_list<int>{H, d.ffn}) {
    g.K = K;
    g.ldb = K;
    g.lda = taps ? H : K;
    g.a_src = taps ? &taps_marker : nullptr;
    if (!gemm_small_fits(g, EPI_PART)) return 0;
  }
  return S;
}

// g (its bias and gate excepted) as a K-split GEMM into the partial area; the returned Pend finishes it
Pend gemm_deferred(GemmArgs g, int S, const Work& w, hipStream_t st, hipError_t* err) {
  Pend p;
  p.part = w.part; p.S = S; p.stride = (size_t)g.M * g.N; p.ld = g.N; p.bias = g.bias; p.gate = g.gate;
  g.C = w.part;
  g.ldc = g.N;
  g.splits = S;
  g.c_split = p.stride;
  *err = gemm_small(g, EPI_PART, st);
  return p;
}

// One estimator evaluation from w.a_in (bf16 [N, 4 mel]) to w.dphi (fp32 [N, mel]) at Euler step `step`.
int run_estimator(const t2w_dit* m, const t2w_solve_args* a, const Work& w, int step, const float* mods,
                  const float* fmods, float* dphi, hipStream_t st) {
  const t2w_dit_dims& d = m->d;
  const int N = a->n_tok, R = a->n_rows, H = d.hidden, F = d.ffn, M = d.mel, D = d.depth;
  T2W_CHECK(gemm_bf16(gemm_args(w.a_in, 4 * M, nullptr, m->g.in_w, m->g.in_b, nullptr, w.h, H, N, H, 4 * M, &w), EPI_F16, st), "in_proj");
  const long long cstride = (long long)d.steps * D * 4 * H;
  const bool f8 = a->fp8 == 1;  // fp8 MFMA, MX fp8 activations
  const bool w8 = a->fp8 == 2;  // e4m3 weights dequantized per GEMM, bf16 activations and MFMA
  hipError_t derr = hipSuccess;
  // the block GEMM's bf16 weights: its own, or (w8) its e4m3 weights dequantized into w.wdq just before it
  // calls of more than 1024 tokens: the row kernel before each block GEMM also reads that GEMM's weights (and the one
  // after it, where no row kernel comes between), so they are cached when the GEMM starts (w8: its dequantization
  // already leaves them there).  Streaming chunks do not: their row kernels are short, and reading the weights there
  // puts the reads on the critical path (chunk DiT 14.8 -> 19.1 ms measured)
  const bool pf_on = !w8 && N > 1024;
  auto pf_of = [&](const void* a0, size_t b0, const void* a1 = nullptr, size_t b1 = 0) {
    Prefetch pf;
    if (pf_on) {
      pf.p[0] = a0; pf.bytes[0] = b0;
      pf.p[1] = a1; pf.bytes[1] = b1;
    }
    return pf;
  };
  const size_t eb = f8 ? 1 : 2;  // bytes per weight
  auto wt = [&](const void* bf, const void* q8, const float* s8, int N, int K) -> const void* {
    if (!w8) return bf;
    if (derr == hipSuccess) derr = dequant_w8((const uint8_t*)q8, s8, N, K, w.wdq, st);
    return w.wdq;
  };
  // Calls of few tokens: the gated-residual GEMMs and conv1 split K over several workgroups per tile and the row
  // kernel that reads their result next finishes their epilogue (pend: the result it has to finish).
  const int Sd = f8 ? 0 : defer_splits(d, N, w, false), St = f8 ? 0 : defer_splits(d, N, w, true);
  const bool S = Sd > 0 && St > 0;  // deferral on: proj / fc2 split Sd ways, conv1 / conv2 St ways
  Pend pend;
  hipError_t perr = hipSuccess;
  for (int b = 0; b < D; ++b) {
    const t2w_dit_block& k = m->blocks[b];
    const t2w_dit_block_fp8* k8 = (f8 || w8) ? &m->blocks8[b] : nullptr;
    const float* md = mods + (size_t)b * 9 * H;
    const float *sh_a = md, *sc_a = md + H, *g_a = md + 2 * H, *sh_m = md + 3 * H, *sc_m = md + 4 * H, *g_m = md + 5 * H;
    const float *sh_c = md + 6 * H, *sc_c = md + 7 * H, *g_c = md + 8 * H;
    const size_t layer = (size_t)(step * D + b) * (size_t)a->pool_layer_stride;
    bf16_t* kp = (bf16_t*)a->k_pool + layer;
    bf16_t* vp = (bf16_t*)a->v_pool + layer;
    GemmArgs gq;
    if (f8) {
      T2W_CHECK(ln_mod_mx8(w.h, sh_a, sc_a, d.eps_block, w.a8, w.a8s, N, H, st,
                           pf_of(k8->qkv_w8, eb * 3 * H * H, k8->proj_w8, eb * H * H)), "ln_mod msa");
      gq = gemm8(w.a8, H, nullptr, w.a8s, k8->qkv_w8, k8->qkv_ws, k.qkv_b, nullptr, w.big, 3 * H, N, 3 * H, H);
    } else {
      T2W_CHECK(ln_mod(w.h, sh_a, sc_a, d.eps_block, w.abuf, N, H, st, pend, pf_of(k.qkv_w, eb * 3 * H * H, k.proj_w, eb * H * H)),
                "ln_mod msa");
      pend = Pend();
      gq = gemm_args(w.abuf, H, nullptr, wt(k.qkv_w, k8 ? k8->qkv_w8 : nullptr, k8 ? k8->qkv_ws : nullptr, 3 * H, H), k.qkv_b, nullptr,
                     w.big, 3 * H, N, 3 * H, H, &w);
      T2W_CHECK(derr, "dequant qkv");
    }
    gq.qk = QkvOut{w.q, kp, vp, a->new_slot, k.qn_w, k.qn_b, k.kn_w, k.kn_b, d.eps_qk, H, m->g.rope_freq, a->tok_abs};
    const bool small_qkv = gemm_small_fits(gq, EPI_QKV);
    if (small_qkv || (!gemm_splits(gq) && H % 256 == 0)) {
      // per-head q / k LayerNorm and the key / value scatter in the projection's epilogue; the small-row kernel also
      // rotates q and k, the tile kernel leaves that to rope_qk (the sine and cosine would spill its registers)
      if (!small_qkv) gq.qk.rfreq = nullptr;
      T2W_CHECK(gemm_bf16(gq, EPI_QKV, st), "qkv");
      if (!small_qkv && m->g.rope_freq) T2W_CHECK(rope_qk(w.q, kp, a->new_slot, a->tok_abs, m->g.rope_freq, N, H, st), "rope");
    } else {
      T2W_CHECK(gemm_bf16(gq, EPI_BF16, st), "qkv");
      T2W_CHECK(qk_norm_scatter(w.big, k.qn_w, k.qn_b, k.kn_w, k.kn_b, d.eps_qk, w.q, kp, vp, a->new_slot, N, d.heads, st,
                                m->g.rope_freq, a->tok_abs),
                "qk_norm");
    }
    AttnArgs at;
    at.q = w.q; at.k_pool = kp; at.v_pool = vp; at.out = w.ao; at.kv_idx = a->kv_idx; at.row_start = a->row_start;
    at.row_len = a->row_len; at.row_kv_off = a->row_kv_off; at.row_kv_len = a->row_kv_len; at.tiles = a->tiles;
    at.n_tiles = a->n_tiles; at.heads = d.heads; at.chunk = a->chunk; at.scale = 1.0f / sqrtf((float)d.head_dim);
    at.n_rows = a->n_rows; at.kv_max = a->kv_max;
    if (f8) { at.out8 = w.o8; at.out8s = w.o8s; }
    T2W_CHECK(attention(at, st), "attention");
    if (f8)
      T2W_CHECK(gemm_bf16(gemm8(w.o8, H, nullptr, w.o8s, k8->proj_w8, k8->proj_ws, k.proj_b, g_a, w.h, H, N, H, H), EPI_RESID_F16, st), "proj");
    else if (S) {
      const void* pw = wt(k.proj_w, k8 ? k8->proj_w8 : nullptr, k8 ? k8->proj_ws : nullptr, H, H);
      T2W_CHECK(derr, "dequant proj");
      pend = gemm_deferred(gemm_args(w.ao, H, nullptr, pw, k.proj_b, g_a, w.h, H, N, H, H, &w), Sd, w, st, &perr);
      T2W_CHECK(perr, "proj");
    } else {
      const void* pw = wt(k.proj_w, k8 ? k8->proj_w8 : nullptr, k8 ? k8->proj_ws : nullptr, H, H);
      T2W_CHECK(derr, "dequant proj");
      T2W_CHECK(timed_launch(T2W_TIMER_RESID_GEMM, resid_bytes(N, H, H), st, [&] { return gemm_bf16(gemm_args(w.ao, H, nullptr, pw, k.proj_b, g_a, w.h, H, N, H, H, &w), EPI_RESID_F16, st); }), "proj");
    }
    ConvPlace cp;
    cp.P = w.P; cp.tok_row = a->tok_row; cp.tok_pos = a->tok_pos; cp.row_start = a->row_start; cp.row_len = a->row_len;
    cp.rd = a->conv_rd; cp.wr = a->conv_wr; cp.cache_stride = cstride; cp.N = N; cp.R = R;
    if (f8) { cp.P8 = w.P8; cp.P8s = w.P8s; }
    bf16_t* cbase = (bf16_t*)a->conv_pool + ((size_t)(step * D + b) * 2) * 2 * H;
    cp.cache_base = cbase;
    cp.cache_out_base = cbase;
    T2W_CHECK(ln_mod_conv(w.h, sh_c, sc_c, d.eps_block, cp, H, st, pend, pf_of(f8 ? k8->c1_w8 : k.c1_w, eb * 3 * H * H)),
              "ln_mod_conv");
    pend = Pend();
    if (f8) {
      T2W_CHECK(gemm_bf16(gemm8(w.P8, H, a->a_src, w.P8s, k8->c1_w8, k8->c1_ws, k.c1_b, nullptr, w.ao, H, N, H, 3 * H), EPI_BF16, st), "conv1");
    } else {
      const void* cw = wt(k.c1_w, k8 ? k8->c1_w8 : nullptr, k8 ? k8->c1_ws : nullptr, H, 3 * H);
      T2W_CHECK(derr, "dequant conv1");
      if (S) {
        pend = gemm_deferred(gemm_args(w.P, H, a->a_src, cw, k.c1_b, nullptr, w.ao, H, N, H, 3 * H, &w), St, w, st, &perr);
        T2W_CHECK(perr, "conv1");
      } else {
        T2W_CHECK(gemm_bf16(gemm_args(w.P, H, a->a_src, cw, k.c1_b, nullptr, w.ao, H, N, H, 3 * H, &w), EPI_BF16, st), "conv1");
      }
    }
    cp.cache_base = cbase + 2 * H;
    cp.cache_out_base = cbase + 2 * H;
    T2W_CHECK(ln_mish_conv(w.ao, k.cln_w, k.cln_b, d.eps_conv, cp, H, st, pend, pf_of(f8 ? k8->c2_w8 : k.c2_w, eb * 3 * H * H)),
              "ln_mish_conv");
    pend = Pend();
    if (f8) {
      T2W_CHECK(gemm_bf16(gemm8(w.P8, H, a->a_src, w.P8s, k8->c2_w8, k8->c2_ws, k.c2_b, g_c, w.h, H, N, H, 3 * H), EPI_RESID_F16, st), "conv2");
    } else {
      const void* cw = wt(k.c2_w, k8 ? k8->c2_w8 : nullptr, k8 ? k8->c2_ws : nullptr, H, 3 * H);
      T2W_CHECK(derr, "dequant conv2");
      if (S) {
        pend = gemm_deferred(gemm_args(w.P, H, a->a_src, cw, k.c2_b, g_c, w.h, H, N, H, 3 * H, &w), St, w, st, &perr);
        T2W_CHECK(perr, "conv2");
      } else {
        T2W_CHECK(gemm_bf16(gemm_args(w.P, H, a->a_src, cw, k.c2_b, g_c, w.h, H, N, H, 3 * H, &w), EPI_RESID_F16, st), "conv2");
      }
    }
    if (f8) {
      T2W_CHECK(ln_mod_mx8(w.h, sh_m, sc_m, d.eps_block, w.a8, w.a8s, N, H, st,
                           pf_of(k8->fc1_w8, eb * F * H, k8->fc2_w8, eb * H * F)), "ln_mod mlp");
      GemmArgs g1 = gemm8(w.a8, H, nullptr, w.a8s, k8->fc1_w8, k8->fc1_ws, k.fc1_b, nullptr, w.b8, F, N, F, H);
      g1.c_scale = w.b8s;
      g1.c_sld = F / 32;
      T2W_CHECK(gemm_bf16(g1, EPI_GELU_MX8, st), "fc1");
      T2W_CHECK(gemm_bf16(gemm8(w.b8, F, nullptr, w.b8s, k8->fc2_w8, k8->fc2_ws, k.fc2_b, g_m, w.h, H, N, H, F), EPI_RESID_F16, st), "fc2");
    } else {
      T2W_CHECK(ln_mod(w.h, sh_m, sc_m, d.eps_block, w.abuf, N, H, st, pend, pf_of(k.fc1_w, eb * F * H, k.fc2_w, eb * H * F)),
                "ln_mod mlp");
      pend = Pend();
      const void* f1w = wt(k.fc1_w, k8 ? k8->fc1_w8 : nullptr, k8 ? k8->fc1_ws : nullptr, F, H);
      T2W_CHECK(derr, "dequant fc1");
      T2W_CHECK(gemm_bf16(gemm_args(w.abuf, H, nullptr, f1w, k.fc1_b, nullptr, w.big, F, N, F, H, &w), EPI_GELU_BF16, st), "fc1");
      const void* f2w = wt(k.fc2_w, k8 ? k8->fc2_w8 : nullptr, k8 ? k8->fc2_ws : nullptr, H, F);
      T2W_CHECK(derr, "dequant fc2");
      if (S) {
        pend = gemm_deferred(gemm_args(w.big, F, nullptr, f2w, k.fc2_b, g_m, w.h, H, N, H, F, &w), Sd, w, st, &perr);
        T2W_CHECK(perr, "fc2");
      } else {
        T2W_CHECK(timed_launch(T2W_TIMER_RESID_GEMM, resid_bytes(N, H, F), st, [&] { return gemm_bf16(gemm_args(w.big, F, nullptr, f2w, k.fc2_b, g_m, w.h, H, N, H, F, &w), EPI_RESID_F16, st); }), "fc2");
      }
    }
  }
  T2W_CHECK(ln_mod(w.h, fmods, fmods + H, d.eps_final, w.abuf, N, H, st, pend), "final norm");
  T2W_CHECK(gemm_bf16(gemm_args(w.abuf, H, nullptr, m->g.out_w, m->g.out_b, nullptr, dphi, M, N, M, H, &w), EPI_F32, st), "final linear");
  return 0;
}

int check_args(const t2w_dit* m, const t2w_solve_args* a) {
  if (check_model(m)) return 1;
  if (!a) return fail("null args");
  if (a->n_tok <= 0 || a->n_rows <= 0) return fail("empty call");
  if (a->fp8 < 0 || a->fp8 > 2) return fail("fp8 must be 0 (bf16), 1 (fp8 MFMA) or 2 (e4m3 weights, bf16 MFMA)");
  if (a->fp8 && !m->fp8_ready()) return fail("fp8 solve needs fp8 weights for every block");
  if (a->fp8 == 1 && (m->d.hidden % 128 || m->d.ffn % 128)) return fail("fp8 solve needs hidden and ffn multiples of 128");
  if (a->workspace_bytes < carve(m->d, a->n_tok, a->n_rows, m->fp8_ready(), nullptr, nullptr)) return fail("workspace too small");
  if (a->chunk < 0) return fail("negative chunk");
  if (a->kv_max < 0) return fail("negative kv_max");
  if (m->g.rope_freq && !a->tok_abs) return fail("rotary embedding needs tok_abs (stream positions)");
  return 0;
}

}  // namespace

extern "C" {

int t2w_abi_version(void) { return 1; }

const char* t2w_last_error(void) { return g_err.c_str(); }

int t2w_dit_create(const t2w_dit_dims* dims, t2w_dit** out) {
  if (!dims || !out) return fail("null argument");
  const t2w_dit_dims& d = *dims;
  if (d.head_dim != 64) return fail("head_dim must be 64");
  if (d.hidden != d.heads * 64) return fail("hidden must be heads * 64");
  if (d.hidden != 256 && d.hidden != 512 && d.hidden != 1024) return fail("hidden must be 256, 512 or 1024");
  if ((4 * d.mel) % 64 || d.ffn % 64) return fail("4 * mel and ffn must be multiples of 64");
  if (d.depth <= 0 || d.steps <= 0 || d.steps > 16) return fail("bad depth / steps");
  void* scr = nullptr;
  if (scratch_address(&scr)) return 1;  // the no-allocation solve's scratch on the current device, looked up at set-up
  t2w_dit* m = new t2w_dit();
  m->d = d;
  m->blocks.resize(d.depth);
  m->block_set.assign(d.depth, false);
  *out = m;
  return 0;
}

int t2w_dit_set_block(t2w_dit* m, int block, const t2w_dit_block* w) {
  if (!m || !w || block < 0 || block >= m->d.depth) return fail("bad block");
  m->blocks[block] = *w;
  m->block_set[block] = true;
  return 0;
}

int t2w_dit_set_block_fp8(t2w_dit* m, int block, const t2w_dit_block_fp8* w) {
  if (!m || !w || block < 0 || block >= m->d.depth) return fail("bad block");
  if (!w->qkv_w8 || !w->qkv_ws || !w->proj_w8 || !w->proj_ws || !w->c1_w8 || !w->c1_ws || !w->c2_w8 || !w->c2_ws ||
      !w->fc1_w8 || !w->fc1_ws || !w->fc2_w8 || !w->fc2_ws)
    return fail("fp8 block weights incomplete");
  if (m->blocks8.empty()) {
    m->blocks8.resize(m->d.depth);
    m->block8_set.assign(m->d.depth, false);
  }
  m->blocks8[block] = *w;
  m->block8_set[block] = true;
  return 0;
}

int t2w_dit_set_globals(t2w_dit* m, const t2w_dit_globals* g) {
  if (!m || !g || !g->dts) return fail("bad globals");
  m->g = *g;
  m->dts.assign(g->dts, g->dts + m->d.steps);
  m->g.dts = m->dts.data();
  m->globals_set = true;
  return 0;
}

void t2w_dit_destroy(t2w_dit* m) { delete m; }

size_t t2w_dit_mods_workspace_bytes(const t2w_dit* m, int S) {
  if (!m) return 0;
  return align_up((size_t)S * m->d.freq * 4) + 2 * align_up((size_t)S * m->d.hidden * 4);
}

int t2w_dit_build_mods(const t2w_dit* m, const t2w_mod_weights* w, const float* ts, int S, float* mods_out, float* final_out,
                       void* workspace, void* stream) {
  if (!m || !w || S <= 0 || S > 16) return fail("bad build_mods arguments");
  hipStream_t st = (hipStream_t)stream;
  const int H = m->d.hidden, Fq = m->d.freq, D = m->d.depth;
  char* base = (char*)workspace;
  float* emb = (float*)base;
  float* h1 = (float*)(base + align_up((size_t)S * Fq * 4));
  float* temb = (float*)(base + align_up((size_t)S * Fq * 4) + align_up((size_t)S * H * 4));
  T2W_CHECK(temb_sinusoid(ts, w->freqs, emb, S, Fq / 2, st), "sinusoid");
  T2W_CHECK(gemv_rows_f32(emb, Fq, 0, w->te0_w, w->te0_b, h1, H, S, H, Fq, 1, st), "t_embedder.0");
  T2W_CHECK(gemv_rows_f32(h1, H, 0, w->te2_w, w->te2_b, temb, H, S, H, H, 0, st), "t_embedder.2");
  T2W_CHECK(gemv_rows_f32(temb, H, 1, w->ada_w, w->ada_b, mods_out, D * 9 * H, S, D * 9 * H, H, 0, st), "adaLN");
  T2W_CHECK(gemv_rows_f32(temb, H, 1, w->fin_w, w->fin_b, final_out, 2 * H, S, 2 * H, H, 0, st), "final adaLN");
  for (int j = 1; j < 9; j += 3) T2W_CHECK(add_one_cols(mods_out, S * D, 9 * H, j * H, H, st), "1 + scale");
  T2W_CHECK(add_one_cols(final_out, S, 2 * H, H, H, st), "1 + scale");
  return 0;
}

size_t t2w_dit_workspace_bytes(const t2w_dit* m, int n_tok, int n_rows) {
  if (!m) return 0;
  return carve(m->d, n_tok, n_rows, m->fp8_ready(), nullptr, nullptr);
}

int t2w_dit_solve(const t2w_dit* m, const t2w_solve_args* a, void* stream) {
  if (check_args(m, a)) return 1;
  if (2 * a->half != a->n_tok) return fail("n_tok must be 2 * half");
  hipStream_t st = (hipStream_t)stream;
  const t2w_dit_dims& d = m->d;
  Work w;
  carve(d, a->n_tok, a->n_rows, m->fp8_ready(), (char*)a->workspace, &w);
  T2W_CHECK(pack_inputs(a->x0, a->stat, w.a_in, w.x, a->half, d.mel, st), "pack_inputs");
  for (int s = 0; s < d.steps; ++s) {
    if (run_estimator(m, a, w, s, m->g.mods + (size_t)s * d.depth * 9 * d.hidden, m->g.final_mods + (size_t)s * 2 * d.hidden, w.dphi, st))
      return 1;
    T2W_CHECK(euler_update(w.x, w.dphi, w.a_in, s + 1 == d.steps ? a->out : nullptr, a->half, d.mel, m->dts[s], d.cfg_rate, st),
              "euler");
  }
  return 0;
}

int t2w_dit_solve_noalloc(const t2w_dit* m, const t2w_solve_args* a, void* stream) {
  if (check_model(m)) return 1;
  if (!a) return fail("null args");
  const size_t need = carve(m->d, a->n_tok, a->n_rows, m->fp8_ready(), nullptr, nullptr);
  if (need > NOALLOC_SCRATCH_BYTES) {
    char buf[256];
    snprintf(buf, sizeof buf, "t2w_dit_solve_noalloc: a call of %d tokens and %d rows needs %zu bytes of scratch, the static "
             "scratch holds %zu (use t2w_dit_solve with a workspace)", a->n_tok, a->n_rows, need, NOALLOC_SCRATCH_BYTES);
    return fail(buf);
  }
  void* scr = nullptr;
  if (scratch_address(&scr)) return 1;
  t2w_solve_args b = *a;
  b.workspace = scr;
  b.workspace_bytes = NOALLOC_SCRATCH_BYTES;
  return t2w_dit_solve(m, &b, stream);
}

int t2w_timer_arm(int cap) {
  if (cap <= 0) return fail("timer_arm: capacity must be positive");
  LaunchTimer& t = launch_timer();
  for (const TimedLaunch& x : t.v) {
    (void)hipEventDestroy(x.e0);
    (void)hipEventDestroy(x.e1);
  }
  t.v.clear();
  t.cap = cap;
  t.armed = true;
  return 0;
}

int t2w_timer_read(void* stream, int* kinds, float* ms, double* bytes, int cap, int* n) {
  if (!n) return fail("timer_read: null count");
  *n = 0;
  LaunchTimer& t = launch_timer();
  t.armed = false;
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  int k = 0;
  for (const TimedLaunch& x : t.v) {
    if (e == hipSuccess && k < cap) {
      float v = 0.f;
      e = hipEventElapsedTime(&v, x.e0, x.e1);
      if (kinds) kinds[k] = x.kind;
      if (ms) ms[k] = v;
      if (bytes) bytes[k] = x.bytes;
      ++k;
    }
    (void)hipEventDestroy(x.e0);
    (void)hipEventDestroy(x.e1);
  }
  t.v.clear();
  T2W_CHECK(e, "timer_read");
  *n = k;
  return 0;
}

int t2w_dit_forward(const t2w_dit* m, const t2w_solve_args* a, int step, const float* mods, const float* final_mods, void* stream) {
  if (check_args(m, a)) return 1;
  if (!a->in_rows) return fail("in_rows required");
  if (step < 0 || step >= m->d.steps) return fail("bad step");
  hipStream_t st = (hipStream_t)stream;
  Work w;
  carve(m->d, a->n_tok, a->n_rows, m->fp8_ready(), (char*)a->workspace, &w);
  T2W_CHECK(convert_rows_bf16(a->in_rows, w.a_in, (long long)a->n_tok * 4 * m->d.mel, st), "convert");
  if (run_estimator(m, a, w, step, mods, final_mods, a->out, st)) return 1;
  return 0;
}

int t2w_gemm_bf16(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate, void* C, int ldc,
                  int M, int N, int K, int epi, void* stream) {
  return t2w_gemm_bf16_tile(A, lda, a_src, W, bias, gate, C, ldc, M, N, K, epi, -1, stream);
}

int t2w_gemm_bf16_tile(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate, void* C, int ldc,
                       int M, int N, int K, int epi, int tile, void* stream) {
  if (K % 64) return fail("K must be a multiple of 64");
  if (lda % 8) return fail("lda must be a multiple of 8 (16-byte rows)");
  if (epi < 0 || (epi > 3 && epi != EPI_F16)) return fail("bad epilogue");
  if (a_src && (K % lda || lda % 64)) return fail("taps mode: K must be a multiple of lda, lda of 64");
  if (tile > 3) return fail("bad tile configuration");
  T2W_CHECK(gemm_bf16(gemm_args(A, lda, a_src, W, bias, gate, C, ldc, M, N, K), epi, (hipStream_t)stream, tile), "gemm");
  return 0;
}

int t2w_gemm_bf16_ws(const void* A, int lda, const int* a_src, const void* W, const float* bias, const float* gate, void* C,
                     int ldc, int M, int N, int K, int epi, void* workspace, size_t workspace_bytes, void* stream) {
  if (K % 64) return fail("K must be a multiple of 64");
  if (lda % 8) return fail("lda must be a multiple of 8 (16-byte rows)");
  if (epi < 0 || (epi > 3 && epi != EPI_F16)) return fail("bad epilogue");
  if (a_src && (K % lda || lda % 64)) return fail("taps mode: K must be a multiple of lda, lda of 64");
  if (((uintptr_t)workspace & 255) != 0) return fail("workspace must be 256-byte aligned");
  GemmArgs g = gemm_args(A, lda, a_src, W, bias, gate, C, ldc, M, N, K);
  g.ws = (float*)workspace;
  g.ws_bytes = workspace ? workspace_bytes : 0;
  T2W_CHECK(gemm_bf16(g, epi, (hipStream_t)stream, -1), "gemm");
  return 0;
}

int t2w_quant_mx8(const void* x, int ldx, int M, int K, void* q, int ldq, void* scales, void* stream) {
  if (K % 32 || ldx % 8 || ldq % 8) return fail("quant_mx8: K % 32, ldx % 8 and ldq % 8 must be 0");
  T2W_CHECK(quant_mx8((const bf16_t*)x, ldx, M, K, (uint8_t*)q, ldq, (uint8_t*)scales, (hipStream_t)stream), "quant_mx8");
  return 0;
}

int t2w_gemm_fp8(const void* A, int lda, const int* a_src, const void* a_scale, int a_sld, const void* W, const float* w_scale,
                 const float* bias, const float* gate, void* C, int ldc, int M, int N, int K, int epi, void* stream) {
  if (K % 128) return fail("fp8 gemm: K must be a multiple of 128");
  if (lda % 16 || a_sld % 4) return fail("fp8 gemm: lda % 16 and a_sld % 4 must be 0");
  if (epi < 0 || epi > 3) return fail("bad epilogue");
  if (a_src && (K % lda || lda % 128)) return fail("fp8 taps mode: K must be a multiple of lda, lda of 128");
  if (!a_scale || !w_scale) return fail("fp8 gemm: scales required");
  GemmArgs g = gemm_args(A, lda, a_src, W, bias, gate, C, ldc, M, N, K);
  g.a_scale = (const uint8_t*)a_scale;
  g.a_sld = a_sld;
  g.w_scale = w_scale;
  T2W_CHECK(gemm_bf16(g, epi, (hipStream_t)stream, -1), "gemm fp8");
  return 0;
}

int t2w_ln_mod(const void* h, const float* shift, const float* scale1, float eps, void* out, int N, int H, void* stream) {
  T2W_CHECK(ln_mod((f16_t*)const_cast<void*>(h), shift, scale1, eps, (bf16_t*)out, N, H, (hipStream_t)stream), "ln_mod");  // h only read
  return 0;
}

int t2w_qk_norm_scatter(const void* qkv, const float* qw, const float* qb, const float* kw, const float* kb, float eps, void* q_out,
                        void* k_pool, void* v_pool, const int* slots, int N, int heads, void* stream) {
  T2W_CHECK(qk_norm_scatter((const bf16_t*)qkv, qw, qb, kw, kb, eps, (bf16_t*)q_out, (bf16_t*)k_pool, (bf16_t*)v_pool, slots, N, heads,
                            (hipStream_t)stream),
            "qk_norm");
  return 0;
}

int t2w_attention(const void* q, const void* k_pool, const void* v_pool, void* out, const int* kv_idx, const int* row_start,
                  const int* row_len, const int* row_kv_off, const int* row_kv_len, const int* tiles, int n_tiles, int heads, int chunk,
                  float scale, int n_rows, int kv_max, void* stream) {
  if (n_rows < 0 || kv_max < 0) return fail("attention: negative n_rows or kv_max");
  AttnArgs at;
  at.q = (const bf16_t*)q; at.k_pool = (const bf16_t*)k_pool; at.v_pool = (const bf16_t*)v_pool; at.out = (bf16_t*)out;
  at.kv_idx = kv_idx; at.row_start = row_start; at.row_len = row_len; at.row_kv_off = row_kv_off; at.row_kv_len = row_kv_len;
  at.tiles = tiles; at.n_tiles = n_tiles; at.heads = heads; at.chunk = chunk; at.scale = scale;
  at.n_rows = n_rows; at.kv_max = kv_max;
  T2W_CHECK(attention(at, (hipStream_t)stream), "attention");
  return 0;
}

struct t2w_graph {
  hipGraph_t graph;
  hipGraphExec_t exec;
};

int t2w_device_cus(int* n) {
  if (!n) return fail("device_cus: null output");
  int dev = 0;
  T2W_CHECK(hipGetDevice(&dev), "hipGetDevice");
  T2W_CHECK(hipDeviceGetAttribute(n, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
  return 0;
}

int t2w_stream_create_cu_mask(const uint32_t* mask, int n_words, void** out) {
  if (!mask || !out || n_words <= 0) return fail("stream_create_cu_mask: null mask or output");
  int cus = 0;
  if (t2w_device_cus(&cus)) return 1;
  int set = 0;
  for (int w = 0; w < n_words; ++w) {
    for (int b = 0; b < 32; ++b)
      if ((mask[w] >> b) & 1u) set += 32 * w + b < cus ? 1 : 0;
    // each 32-CU word one run of at least 8 consecutive CUs, or none: the runtime's queue creation fails on masks
    // that interleave single CUs or give a group fewer than 8 (measured: 2 and 4 fail, 8 and more pass), and the
    // failure then sticks to the process's later calls
    const uint32_t low = mask[w] ? (mask[w] >> __builtin_ctz(mask[w])) : 0u;
    if ((low & (low + 1u)) || (low && __builtin_popcount(low) < 8))
      return fail("stream_create_cu_mask: each 32-bit word of the mask must be one run of at least 8 consecutive CUs, or empty");
  }
  if (set == 0) return fail("stream_create_cu_mask: the mask names none of the device's CUs");
  hipStream_t s = nullptr;
  T2W_CHECK(hipExtStreamCreateWithCUMask(&s, (uint32_t)n_words, mask), "hipExtStreamCreateWithCUMask");
  *out = (void*)s;
  return 0;
}

int t2w_stream_destroy(void* stream) {
  if (!stream) return 0;
  T2W_CHECK(hipStreamDestroy((hipStream_t)stream), "stream destroy");
  return 0;
}

int t2w_graph_begin(void* stream) {
  T2W_CHECK(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal), "begin capture");
  return 0;
}

int t2w_graph_end(void* stream, t2w_graph** out) {
  hipGraph_t g;
  T2W_CHECK(hipStreamEndCapture((hipStream_t)stream, &g), "end capture");
  hipGraphExec_t ex;
  hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return fail("instantiate", e);
  }
  *out = new t2w_graph{g, ex};
  return 0;
}

int t2w_graph_launch(t2w_graph* g, void* stream) {
  if (!g) return fail("null graph");
  T2W_CHECK(hipGraphLaunch(g->exec, (hipStream_t)stream), "graph launch");
  return 0;
}

void t2w_graph_destroy(t2w_graph* g) {
  if (!g) return;
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  delete g;
}

}  // extern "C"
