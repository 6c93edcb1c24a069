// C-ABI of the HiFT vocoder: the model object and the whole forward (f0 predictor, NSF source, STFT, decoder, ISTFT)
// as one call over rows of different lengths.  No allocation in the forward: the caller passes the workspace and a
// device copy of the plan.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/t2w.h"
#include "hift_internal.h"
#include "launch_timer.h"

using namespace t2w;

namespace {

#define H_CHECK(expr, what)                               \
  do {                                                    \
    hipError_t e_ = (expr);                               \
    if (e_ != hipSuccess) return t2w::set_error(what, e_); \
  } while (0)

size_t al(size_t x) { return (x + 63) & ~(size_t)63; }  // floats, 256-byte aligned

enum Cls { C_T = 0, C_S0 = 1, C_S1 = 2, C_S2 = 3, C_SMP = 4, C_S2P = 5, N_CLS = 6 };

struct Lens {  // per-class totals and maxima of a call
  long long tot[N_CLS];
  int mx[N_CLS];
};

}  // namespace

struct t2w_hift {
  t2w_hift_dims d;
  t2w_hift_weights w;
  int chans[4];
  // each bf16 conv's weights in MFMA fragment order (made by t2w_hift_create, freed by t2w_hift_destroy), by wbf
  std::vector<std::pair<const void*, uint16_t*>> frag;
  const uint16_t* frag_of(const void* wbf) const {
    for (const auto& f : frag)
      if (f.first == wbf) return f.second;
    return nullptr;
  }
  // the source downsampling convs' fp32 weights with their 18 input channels padded to STFT_LD ([Cout][taps][32], made
  // by t2w_hift_create), read with the padded STFT rows
  float* src_w32[3] = {nullptr, nullptr, nullptr};
};

namespace {

int class_len(const t2w_hift_dims& d, int cls, int T) {
  const int L1 = T * d.up_rates[0], L2 = L1 * d.up_rates[1], L3 = L2 * d.up_rates[2] + 1;
  switch (cls) {
    case C_T: return T;
    case C_S0: return L1;
    case C_S1: return L2;
    case C_S2: return L3;
    case C_SMP: return (L3 - 1) * d.hop;
    case C_S2P: return L3 - 1;
  }
  return 0;
}

Lens lens_of(const t2w_hift_dims& d, int n, const int* frames) {
  Lens L;
  for (int c = 0; c < N_CLS; ++c) {
    L.tot[c] = 0;
    L.mx[c] = 0;
    for (int i = 0; i < n; ++i) {
      const int v = class_len(d, c, frames[i]);
      L.tot[c] += v;
      L.mx[c] = std::max(L.mx[c], v);
    }
  }
  return L;
}

struct Bufs {
  float *f0a, *f0b, *f0, *phase, *stft, *X, *XN, *Z, *TMP, *S, *Z2, *post;
};

size_t carve(const t2w_hift* h, const Lens& L, char* base, Bufs* b) {
  const t2w_hift_dims& d = h->d;
  size_t big = 0;
  big = std::max(big, (size_t)L.tot[C_T] * d.base);
  big = std::max(big, (size_t)L.tot[C_S0] * h->chans[1]);
  big = std::max(big, (size_t)L.tot[C_S1] * h->chans[2]);
  big = std::max(big, (size_t)L.tot[C_S2] * h->chans[3]);
  size_t off = 0;
  auto take = [&](size_t n) { float* p = base ? (float*)base + off : nullptr; off += al(n); return p; };
  Bufs t;
  t.f0a = take((size_t)L.tot[C_T] * d.f0_channels);
  t.f0b = take((size_t)L.tot[C_T] * d.f0_channels);
  t.f0 = take(L.tot[C_T]);
  t.phase = take((size_t)L.tot[C_T] * (d.harmonics + 1));
  t.stft = take((size_t)L.tot[C_S2] * STFT_LD);
  t.X = take(big);
  t.XN = take(big);
  t.Z = take(big);
  t.TMP = take(big);
  t.S = take(big);
  t.Z2 = take(big);
  t.post = take((size_t)L.tot[C_S2] * (d.n_fft + 2));
  if (b) *b = t;
  return off * sizeof(float);
}

struct Ctx {
  const t2w_hift* h;
  bool bf16;       // bf16 MFMA decoder convs
  int fuse;        // ResBlock dilations as one kernel each: 0 never, 1 where the grid fills the chip, 2 always
  const int* plan;  // device: [class][off | len][n]
  int n;
  Lens L;
  hipStream_t st;
  const int* off(int c) const { return plan + (size_t)(2 * c) * n; }
  const int* len(int c) const { return plan + (size_t)(2 * c + 1) * n; }
};

// a plain conv: kernel k, dilation dil, stride s, padding p; input class ci_cls, output class co_cls
ConvDesc conv_desc(const Ctx& x, const t2w_conv& w, const float* in, int Cin, int in_cls, float* out, int Cout, int out_cls, int k, int dil,
                   int s, int p) {
  ConvDesc c{};
  c.x = in; c.ldx = Cin; c.in_off = x.off(in_cls); c.in_len = x.len(in_cls);
  c.y = out; c.ldy = Cout; c.out_off = x.off(out_cls); c.out_len = x.len(out_cls);
  c.w = w.w; c.wbf = (const uint16_t*)w.wbf; c.wfr = x.h->frag_of(w.wbf); c.bias = w.b; c.Cin = Cin; c.Cout = Cout; c.taps = k;
  c.s_in = s; c.d_in = dil; c.s_out = 1; c.n_phase = 1; c.off_in[0] = -p; c.off_out[0] = 0;
  c.pre = PRE_NONE; c.epi = EPI_STORE; c.n_items = x.n;
  return c;
}

// fused ResBlock dilations below this many workgroups leave the chip half idle: two convs with smaller tiles instead
constexpr long kPairMinBlocks = 128;

// whether run() takes c to the bf16 MFMA convolution (else the fp32 one)
bool on_bf16(const Ctx& x, const ConvDesc& c) {
  const int span = (c.taps - 1) * (c.d_in < 0 ? -c.d_in : c.d_in);
  return x.bf16 && c.wbf && c.s_in == 1 && span <= 64 && c.ldx % 4 == 0 && c.ldy % 4 == 0;
}

int run(const Ctx& x, const ConvDesc& c, int out_cls, const char* what) {
  const int mr = x.L.mx[out_cls] / c.s_out + 2;
  if (on_bf16(x, c))
    H_CHECK(conv_bf16(c, c.wbf, mr, x.st), what);
  else
    H_CHECK(conv_f32(c, mr, x.st), what);
  return 0;
}

// ResBlock on `in` (class cls, C channels): per dilation z = c2(snake(c1(snake(z)))) + z.  The last dilation's output
// goes to `sum` (mean of the stage's ResBlocks, sum_mode 0 / 1 / 2) or, with add_into, is added into add_into.  z and tmp
// are scratch (z may be `in`, which is then overwritten).  A dilation runs as one fused kernel (conv1's output kept in
// LDS, written to a scratch buffer other than its input) when the bf16 path fuses and the grid fills the chip, else as
// two convs through a scratch buffer (the second in place when its input is scratch).  Two fp32 convs take their
// Snakes out of the tap loop (where an element's Snake would be evaluated once per tap): snake1 of the input into
// `act` (a scratch buffer no other argument names) and snake2 in conv1's epilogue; the values are the same.
int resblock(const Ctx& x, const t2w_resblock& rb, int k, const float* in, float* z, float* tmp, float* act, int C, int cls, float* sum,
             int sum_mode, float* add_into) {
  const t2w_hift_dims& d = x.h->d;
  const int mr = x.L.mx[cls] + 2;
  auto other = [&](const float* p) { return p == z ? tmp : z; };  // a scratch buffer that is not p
  const float* cur = in;
  for (int j = 0; j < 3; ++j) {
    const int dil = d.res_dilations[j];
    const bool fused = x.bf16 && x.fuse && rb.c1[j].wbf && rb.c2[j].wbf && resblock_pair_fits(C, k, dil) &&
                       (x.fuse == 2 || (long)((mr + resblock_pair_rows(C, k) - 1) / resblock_pair_rows(C, k)) * x.n >= kPairMinBlocks);
    float* mid = other(cur);  // conv1's output (two-kernel path)
    float* out = fused ? other(cur) : (cur == z || cur == tmp ? (float*)cur : other(mid));
    ConvDesc c1 = conv_desc(x, rb.c1[j], cur, C, cls, mid, C, cls, k, dil, 1, dil * (k - 1) / 2);
    c1.pre = PRE_SNAKE; c1.alpha = rb.a1[j]; c1.inv = rb.inv1[j];
    ConvDesc c2 = conv_desc(x, rb.c2[j], fused ? cur : mid, C, cls, out, C, cls, k, 1, 1, (k - 1) / 2);
    c2.pre = PRE_SNAKE; c2.alpha = rb.a2[j]; c2.inv = rb.inv2[j];
    c2.res = cur;
    if (j < 2) {
      c2.epi = EPI_RES;  // out = conv + res (in place when out == cur: each element is read and written by one thread)
    } else if (add_into) {
      c2.epi = EPI_ADD_RES;
      c2.y = add_into;
    } else {
      c2.epi = EPI_RES_MEAN;
      c2.sum = sum;
      c2.sum_mode = sum_mode;
      c2.sum_div = 3;
    }
    if (fused) {
      H_CHECK(resblock_pair_bf16(c1, c2, mr, x.st), "resblock pair");
    } else {
      if (!on_bf16(x, c1) && !on_bf16(x, c2) && C % 4 == 0) {
        H_CHECK(timed_launch(T2W_TIMER_HIFT_SNAKE, 8.0 * C * x.L.tot[cls], x.st,
                             [&] { return snake_rows(cur, C, x.L.tot[cls], c1.alpha, c1.inv, act, x.st); }),
                "resblock snake1");
        c1.x = act;
        c1.pre = PRE_NONE;
        c1.epi = EPI_SNAKE;
        c1.alpha = c2.alpha;
        c1.inv = c2.inv;
        c2.pre = PRE_NONE;
      }
      if (run(x, c1, cls, "resblock conv1")) return 1;
      if (run(x, c2, cls, "resblock conv2")) return 1;
    }
    cur = out;
  }
  return 0;
}

}  // namespace

extern "C" {

int t2w_hift_create(const t2w_hift_dims* dims, const t2w_hift_weights* w, t2w_hift** out) {
  if (!dims || !w || !out) return t2w::set_error("null argument", hipSuccess);
  const t2w_hift_dims& d = *dims;
  if (d.n_up != 3 || d.n_fft != 16 || d.hop != 4 || d.f0_layers != 5 || d.harmonics + 1 > 16)
    return t2w::set_error("unsupported HiFT geometry (3 upsampling stages, n_fft 16, hop 4, 5 f0 convs)", hipSuccess);
  for (int i = 0; i < 3; ++i)
    if (d.up_rates[i] > 8) return t2w::set_error("upsampling rate above 8", hipSuccess);
  t2w_hift* h = new t2w_hift();
  h->d = d;
  h->w = *w;
  h->chans[0] = d.base;
  for (int i = 0; i < 3; ++i) h->chans[i + 1] = d.base >> (i + 1);
  // fragment-ordered copies of the bf16 weights, one per distinct wbf, in the shapes the forward gives each conv
  auto add = [&](const t2w_conv& cv, int n_phase, int Cout, int taps, int Cin) -> hipError_t {
    if (!cv.wbf || h->frag_of(cv.wbf)) return hipSuccess;
    uint16_t* p = nullptr;
    const size_t bytes = (size_t)n_phase * ((Cout + 63) & ~63) * taps * ((Cin + 63) & ~63) * sizeof(uint16_t);
    hipError_t e = hipMalloc((void**)&p, bytes);
    if (e != hipSuccess) return e;
    h->frag.push_back({cv.wbf, p});
    return conv_weight_fragments((const uint16_t*)cv.wbf, p, n_phase, Cout, taps, Cin, nullptr);
  };
  const int nsrc = d.n_fft + 2;
  hipError_t e = add(w->conv_pre, 1, d.base, 7, d.mel);
  for (int i = 0; i < 3 && e == hipSuccess; ++i) {
    const int u = d.up_rates[i], cout = h->chans[i + 1];
    e = add(w->ups[i], u, cout, (d.up_kernels[i] + u - 1) / u, h->chans[i]);
    const int r = i == 0 ? d.up_rates[2] * d.up_rates[1] : (i == 1 ? d.up_rates[2] : 1);
    if (e == hipSuccess) e = add(w->src_down[i], 1, cout, r == 1 ? 1 : 2 * r, nsrc);
    for (int j = 0; j < 3 && e == hipSuccess; ++j) {
      e = add(w->src_res[i].c1[j], 1, cout, d.src_kernels[i], cout);
      if (e == hipSuccess) e = add(w->src_res[i].c2[j], 1, cout, d.src_kernels[i], cout);
      for (int q = 0; q < 3 && e == hipSuccess; ++q) {
        e = add(w->res[i * 3 + q].c1[j], 1, cout, d.res_kernels[q], cout);
        if (e == hipSuccess) e = add(w->res[i * 3 + q].c2[j], 1, cout, d.res_kernels[q], cout);
      }
    }
  }
  if (e == hipSuccess) e = add(w->conv_post, 1, nsrc, 7, h->chans[3]);
  for (int i = 0; i < 3 && e == hipSuccess; ++i) {  // the source downsampling weights, input channels padded with zeros
    const int r = i == 0 ? d.up_rates[2] * d.up_rates[1] : (i == 1 ? d.up_rates[2] : 1), taps = r == 1 ? 1 : 2 * r;
    const size_t rows = (size_t)h->chans[i + 1] * taps;
    if (!w->src_down[i].w) {
      e = hipErrorInvalidValue;
      break;
    }
    e = hipMalloc((void**)&h->src_w32[i], rows * STFT_LD * sizeof(float));
    if (e == hipSuccess) e = hipMemsetAsync(h->src_w32[i], 0, rows * STFT_LD * sizeof(float), nullptr);
    if (e == hipSuccess)
      e = hipMemcpy2DAsync(h->src_w32[i], STFT_LD * sizeof(float), w->src_down[i].w, nsrc * sizeof(float), nsrc * sizeof(float), rows,
                           hipMemcpyDeviceToDevice, nullptr);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e != hipSuccess) {
    t2w_hift_destroy(h);
    return t2w::set_error("hift_create: bf16 weight copies", e);
  }
  *out = h;
  return 0;
}

void t2w_hift_destroy(t2w_hift* h) {
  if (!h) return;
  for (auto& f : h->frag) (void)hipFree(f.second);
  for (float* p : h->src_w32)
    if (p) (void)hipFree(p);
  delete h;
}

int t2w_hift_plan_ints(int n_items) { return 2 * N_CLS * n_items; }

int t2w_hift_plan(const t2w_hift* h, int n, const int* frames, int* plan) {
  if (!h || n <= 0 || !frames || !plan) return t2w::set_error("bad plan arguments", hipSuccess);
  for (int c = 0; c < N_CLS; ++c) {
    long long o = 0;
    for (int i = 0; i < n; ++i) {
      if (frames[i] <= 0) return t2w::set_error("rows need at least one mel frame", hipSuccess);
      const int L = class_len(h->d, c, frames[i]);
      plan[(2 * c) * n + i] = (int)o;
      plan[(2 * c + 1) * n + i] = L;
      o += L;
    }
  }
  // the last stage's transposed conv writes rows 1.. of each row's stage-2 buffer (row 0 is its reflection pad)
  for (int i = 0; i < n; ++i) plan[(2 * C_S2P) * n + i] = plan[(2 * C_S2) * n + i] + 1;
  return 0;
}

size_t t2w_hift_workspace_bytes(const t2w_hift* h, int n, const int* frames) {
  if (!h || n <= 0) return 0;
  return carve(h, lens_of(h->d, n, frames), nullptr, nullptr);
}

int t2w_hift_forward(const t2w_hift* h, int n, const int* frames, const int* plan_dev, const float* mel, const float* noise,
                     const float* cache_source, int S, const float* f0_override, const float* source_override, float* speech,
                     float* source, float* f0_out, void* workspace, size_t workspace_bytes, int decode_bf16, void* stream) {
  if (!h || n <= 0 || !frames || !plan_dev || !mel || !speech || !source) return t2w::set_error("bad hift arguments", hipSuccess);
  const t2w_hift_dims& d = h->d;
  Ctx x{h, decode_bf16 != 0, decode_bf16 == 1 ? 1 : (decode_bf16 == 3 ? 2 : 0), plan_dev, n, lens_of(d, n, frames), (hipStream_t)stream};
  for (int i = 0; i < n; ++i)
    if (S > class_len(d, C_SMP, frames[i])) return t2w::set_error("source cache longer than a row", hipSuccess);
  if (S > 0 && !cache_source) return t2w::set_error("missing source cache", hipSuccess);
  if (workspace_bytes < carve(h, x.L, nullptr, nullptr)) return t2w::set_error("hift workspace too small", hipSuccess);
  Bufs B;
  carve(h, x.L, (char*)workspace, &B);
  const t2w_hift_weights& w = h->w;
  const int harm = d.harmonics + 1, nsrc = d.n_fft + 2;

  // f0 predictor: five kernel-3 convs with ELU, then |Linear(C -> 1)|
  const float* f0 = f0_override;
  if (!f0) {
    const float* cur = mel;
    int cin = d.mel;
    for (int l = 0; l < d.f0_layers; ++l) {
      float* o = (l & 1) ? B.f0b : B.f0a;
      ConvDesc c = conv_desc(x, w.f0[l], cur, cin, C_T, o, d.f0_channels, C_T, 3, 1, 1, 1);
      c.epi = EPI_ELU;
      c.wbf = nullptr;  // the f0 predictor stays fp32: its rounding integrates into the source phase
      if (run(x, c, C_T, "f0 conv")) return 1;
      cur = o;
      cin = d.f0_channels;
    }
    H_CHECK(timed_launch(T2W_TIMER_HIFT_F0_HEAD, 4.0 * (d.f0_channels + 1) * (x.L.tot[C_T] + 1), x.st,
                         [&] { return f0_head(cur, d.f0_channels, w.f0_head_w, w.f0_head_b, B.f0, (int)x.L.tot[C_T], x.st); }),
            "f0 head");
    f0 = B.f0;
  }
  if (f0_out) H_CHECK(hipMemcpyAsync(f0_out, f0, x.L.tot[C_T] * sizeof(float), hipMemcpyDeviceToDevice, x.st), "f0 out");

  // NSF source
  const int up = d.up_rates[0] * d.up_rates[1] * d.up_rates[2] * d.hop;
  const float* s = source_override;
  if (!s) {
    const double fr = (double)x.L.tot[C_T], smp = (double)x.L.tot[C_SMP], cached = (double)n * S;
    H_CHECK(timed_launch(T2W_TIMER_HIFT_PHASE, 4.0 * fr * (1 + harm), x.st,
                         [&] { return nsf_phase(f0, x.off(C_T), x.len(C_T), n, harm, (float)d.sr, (float)up, B.phase, x.st); }),
            "nsf phase");
    // noise in and the sample out per generated sample, the cache copied for the first S of a row, f0 and the frame
    // phases read once
    H_CHECK(timed_launch(T2W_TIMER_HIFT_SOURCE, (smp - cached) * 4.0 * (harm + 1) + cached * 8.0 + 4.0 * fr * (1 + harm), x.st,
                         [&] {
                           return nsf_source(B.phase, f0, x.off(C_T), x.len(C_T), x.off(C_SMP), n, x.L.mx[C_T], harm, (float)(1.0 / up), up,
                                             d.sine_amp, d.noise_std, (float)((double)d.sine_amp / 3.0), d.voiced_threshold, noise,
                                             w.src_w, w.src_b, cache_source, S, source, x.st);
                         }),
            "nsf source");
    s = source;
  } else if (s != source) {
    H_CHECK(hipMemcpyAsync(source, s, x.L.tot[C_SMP] * sizeof(float), hipMemcpyDeviceToDevice, x.st), "source copy");
  }
  H_CHECK(timed_launch(T2W_TIMER_HIFT_STFT, 4.0 * x.L.tot[C_SMP] + 4.0 * STFT_LD * x.L.tot[C_S2], x.st,
                       [&] { return stft16(s, x.off(C_SMP), x.len(C_SMP), x.off(C_S2), x.len(C_S2), n, x.L.mx[C_S2], w.window, B.stft, x.st); }),
          "stft");

  // decoder
  {
    ConvDesc c = conv_desc(x, w.conv_pre, mel, d.mel, C_T, B.X, d.base, C_T, 7, 1, 1, 3);
    if (run(x, c, C_T, "conv_pre")) return 1;
  }
  float* X = B.X;  // stage input (leaky ReLU applied on load)
  float* Sb = B.S;
  const int scls[3] = {C_S0, C_S1, C_S2};
  for (int i = 0; i < 3; ++i) {
    const int u = d.up_rates[i], k = d.up_kernels[i], p = (k - u) / 2;
    const int cin = h->chans[i], cout = h->chans[i + 1];
    const int in_cls = i == 0 ? C_T : scls[i - 1];
    const int cls = scls[i];
    {  // transposed conv as u polyphase convs: output t = q u + ph - p reads inputs q - m with kernel taps ph + m u
      ConvDesc c{};
      c.x = X; c.ldx = cin; c.in_off = x.off(in_cls); c.in_len = x.len(in_cls);
      c.y = B.XN; c.ldy = cout;
      c.out_off = x.off(i == 2 ? C_S2P : cls);
      c.out_len = x.len(i == 2 ? C_S2P : cls);
      c.w = w.ups[i].w; c.wbf = (const uint16_t*)w.ups[i].wbf; c.wfr = h->frag_of(w.ups[i].wbf); c.bias = w.ups[i].b; c.Cin = cin; c.Cout = cout; c.taps = (k + u - 1) / u;
      c.s_in = 1; c.d_in = -1; c.s_out = u; c.n_phase = u;
      for (int ph = 0; ph < u; ++ph) { c.off_in[ph] = 0; c.off_out[ph] = ph - p; }
      c.pre = PRE_LEAKY; c.slope = d.lrelu_slope; c.epi = EPI_STORE; c.n_items = n;
      if (run(x, c, i == 2 ? C_S2P : cls, "ups")) return 1;
      if (i == 2)
        H_CHECK(timed_launch(T2W_TIMER_HIFT_REFLECT, 8.0 * cout * n, x.st, [&] { return reflect_rows(B.XN, cout, x.off(C_S2), n, x.st); }),
                "reflection pad");
    }
    {  // source branch: downsampling conv of the source STFT, a ResBlock, added into the stage input
      const int r = i == 0 ? d.up_rates[2] * d.up_rates[1] : (i == 1 ? d.up_rates[2] : 1);
      ConvDesc c = r == 1 ? conv_desc(x, w.src_down[i], B.stft, STFT_LD, C_S2, B.Z2, cout, cls, 1, 1, 1, 0)
                          : conv_desc(x, w.src_down[i], B.stft, STFT_LD, C_S2, B.Z2, cout, cls, 2 * r, 1, r, r / 2);
      c.w = x.h->src_w32[i];  // padded like the STFT rows
      if (run(x, c, cls, "source down")) return 1;
      // X (the stage input) is dead once the transposed conv has read it: the ResBlocks' Snake scratch
      if (resblock(x, w.src_res[i], d.src_kernels[i], B.Z2, B.Z2, B.TMP, X, cout, cls, nullptr, 0, B.XN)) return 1;
    }
    for (int j = 0; j < 3; ++j)
      if (resblock(x, w.res[i * 3 + j], d.res_kernels[j], B.XN, B.Z, B.TMP, X, cout, cls, Sb, j, nullptr)) return 1;
    std::swap(X, Sb);  // the mean is the next stage's input
  }
  {
    ConvDesc c = conv_desc(x, w.conv_post, X, h->chans[3], C_S2, B.post, nsrc, C_S2, 7, 1, 1, 3);
    c.pre = PRE_LEAKY;
    c.slope = 0.01f;
    if (run(x, c, C_S2, "conv_post")) return 1;
  }
  H_CHECK(timed_launch(T2W_TIMER_HIFT_ISTFT, 4.0 * nsrc * x.L.tot[C_S2] + 4.0 * x.L.tot[C_SMP], x.st,
                       [&] { return istft16(B.post, x.off(C_S2), x.len(C_S2), x.off(C_SMP), n, x.L.mx[C_SMP], w.window, d.audio_limit, speech, x.st); }),
          "istft");
  return 0;
}

}  // extern "C"
