// HiFT vocoder kernels (fp32): implicit-GEMM 1-D convolutions on fp32 MFMA, the NSF harmonic source, STFT and ISTFT.
//
// Activations are time-major ([rows, channels], one item's frames contiguous), so for every tap a conv's K slice over
// input channels is contiguous and the GEMM is rows x Cout x (taps * Cin).  Transposed convolutions run as `u`
// polyphase convolutions (phase p of the output sees taps p, p + u, .. of the kernel over inputs q, q - 1, ..).  The
// activation before a conv (leaky ReLU, Snake) is applied while its input tile is staged in LDS; the epilogue adds the
// bias and, for ResBlocks, the residual and the running mean over the stage's three ResBlocks.
#include "common.h"
#include "hift_internal.h"

namespace t2w {

namespace {


// exact twiddles of the 16-point DFT: cos / sin(2 pi m / 16)
__constant__ float kCos16[16] = {1.0f, 0.923879533f, 0.707106781f, 0.382683432f, 0.0f, -0.382683432f, -0.707106781f, -0.923879533f,
                                 -1.0f, -0.923879533f, -0.707106781f, -0.382683432f, 0.0f, 0.382683432f, 0.707106781f, 0.923879533f};
__constant__ float kSin16[16] = {0.0f, 0.382683432f, 0.707106781f, 0.923879533f, 1.0f, 0.923879533f, 0.707106781f, 0.382683432f,
                                 0.0f, -0.382683432f, -0.707106781f, -0.923879533f, -1.0f, -0.923879533f, -0.707106781f, -0.382683432f};

__device__ __forceinline__ float pre_act(float v, int pre, float slope, float a, float inv) {
  if (pre == PRE_LEAKY) return v > 0.f ? v : v * slope;
  if (pre == PRE_SNAKE) {
    const float s = sinf(__fmul_rn(v, a));
    return __fadd_rn(v, __fmul_rn(inv, __fmul_rn(s, s)));
  }
  return v;
}

// epilogue of a 32-row x 32-channel MFMA block: this lane's output row and channels co + q*8 + (lane/32)*4 + e
__device__ __forceinline__ void conv_epilogue(const ConvDesc& c, int b, int out_row, int co_base, int lane, const f32x16& acc) {
  const size_t row = (size_t)c.out_off[b] + (size_t)out_row;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int co = co_base + q * 8 + (lane >> 5) * 4 + e;
      if (co >= c.Cout) continue;
      float v = __fadd_rn(acc[q * 4 + e], c.bias[co]);
      float* yp = c.y + row * c.ldy + co;
      switch (c.epi) {
        case EPI_STORE: *yp = v; break;
        case EPI_ELU: *yp = v > 0.f ? v : expm1f(v); break;
        case EPI_SNAKE: *yp = pre_act(v, PRE_SNAKE, 0.f, c.alpha[co], c.inv[co]); break;
        case EPI_RES: *yp = __fadd_rn(v, c.res[row * c.ldy + co]); break;
        case EPI_ADD_RES: *yp = __fadd_rn(*yp, __fadd_rn(v, c.res[row * c.ldy + co])); break;
        case EPI_RES_MEAN: {
          v = __fadd_rn(v, c.res[row * c.ldy + co]);
          float* sp = c.sum + row * c.ldy + co;
          if (c.sum_mode == 0) *sp = v;
          else if (c.sum_mode == 1) *sp = __fadd_rn(*sp, v);
          else *sp = __fdiv_rn(__fadd_rn(*sp, v), (float)c.sum_div);
        } break;
      }
    }
  }
}

// the tensors the epilogue of four channels reads before it writes: the residual (r) and the output or the running
// sum it accumulates into (t); loaded ahead so that a batch of rows has all its loads in flight
__device__ __forceinline__ void conv_epilogue4_loads(const ConvDesc& c, size_t row, int co, float4& r, float4& t) {
  if (c.epi == EPI_RES || c.epi == EPI_ADD_RES || c.epi == EPI_RES_MEAN) r = *(const float4*)(c.res + row * c.ldy + co);
  if (c.epi == EPI_ADD_RES) t = *(const float4*)(c.y + row * c.ldy + co);
  if (c.epi == EPI_RES_MEAN && c.sum_mode != 0) t = *(const float4*)(c.sum + row * c.ldy + co);
}

// epilogue of four consecutive channels co .. co + 3 of one output row (all inside Cout), with its loads already done
// (r, t as conv_epilogue4_loads left them)
// SNK: the caller may pass EPI_SNAKE (the fp32 kernels; kept out of the bf16 kernels, whose registers are full)
template <bool SNK = false>
__device__ __forceinline__ void conv_epilogue4_pre(const ConvDesc& c, size_t row, int co, float4 a, float4 r, float4 t) {
  const float4 bb = *(const float4*)(c.bias + co);
  float v[4] = {__fadd_rn(a.x, bb.x), __fadd_rn(a.y, bb.y), __fadd_rn(a.z, bb.z), __fadd_rn(a.w, bb.w)};
  float* yp = c.y + row * c.ldy + co;
  if (c.epi == EPI_STORE) {
    *(float4*)yp = make_float4(v[0], v[1], v[2], v[3]);
  } else if (c.epi == EPI_ELU) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v[e] > 0.f ? v[e] : expm1f(v[e]);
    *(float4*)yp = make_float4(v[0], v[1], v[2], v[3]);
  } else if (SNK && c.epi == EPI_SNAKE) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = pre_act(v[e], PRE_SNAKE, 0.f, c.alpha[co + e], c.inv[co + e]);
    *(float4*)yp = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    v[0] = __fadd_rn(v[0], r.x); v[1] = __fadd_rn(v[1], r.y); v[2] = __fadd_rn(v[2], r.z); v[3] = __fadd_rn(v[3], r.w);
    if (c.epi == EPI_RES) {
      *(float4*)yp = make_float4(v[0], v[1], v[2], v[3]);
    } else if (c.epi == EPI_ADD_RES) {
      *(float4*)yp = make_float4(__fadd_rn(t.x, v[0]), __fadd_rn(t.y, v[1]), __fadd_rn(t.z, v[2]), __fadd_rn(t.w, v[3]));
    } else {  // EPI_RES_MEAN
      float* sp = c.sum + row * c.ldy + co;
      if (c.sum_mode == 0) {
        *(float4*)sp = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        float o[4] = {__fadd_rn(t.x, v[0]), __fadd_rn(t.y, v[1]), __fadd_rn(t.z, v[2]), __fadd_rn(t.w, v[3])};
        if (c.sum_mode == 2) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = __fdiv_rn(o[e], (float)c.sum_div);
        }
        *(float4*)sp = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// conv_epilogue4 with its own loads
template <bool SNK = false>
__device__ __forceinline__ void conv_epilogue4(const ConvDesc& c, size_t row, int co, float4 a) {
  float4 r, t;
  conv_epilogue4_loads(c, row, co, r, t);
  conv_epilogue4_pre<SNK>(c, row, co, a, r, t);
}

// the last n < 4 channels co .. co + n - 1 of a Cout that is not a multiple of 4, element by element
template <bool SNK = false>
__device__ __forceinline__ void conv_epilogue_part(const ConvDesc& c, size_t orow, int co0, int n, float4 v) {
  const float vv[4] = {v.x, v.y, v.z, v.w};
  for (int e = 0; e < 4 && e < n; ++e) {
    const int co = co0 + e;
    float x = __fadd_rn(vv[e], c.bias[co]);
    float* yp = c.y + orow * c.ldy + co;
    if (c.epi == EPI_STORE) *yp = x;
    else if (c.epi == EPI_ELU) *yp = x > 0.f ? x : expm1f(x);
    else if (SNK && c.epi == EPI_SNAKE) *yp = pre_act(x, PRE_SNAKE, 0.f, c.alpha[co], c.inv[co]);
    else {
      x = __fadd_rn(x, c.res[orow * c.ldy + co]);
      if (c.epi == EPI_RES) *yp = x;
      else if (c.epi == EPI_ADD_RES) *yp = __fadd_rn(*yp, x);
      else {
        float* sp = c.sum + orow * c.ldy + co;
        if (c.sum_mode == 0) *sp = x;
        else if (c.sum_mode == 1) *sp = __fadd_rn(*sp, x);
        else *sp = __fdiv_rn(__fadd_rn(*sp, x), (float)c.sum_div);
      }
    }
  }
}

// fp32 implicit-GEMM convolution (v_mfma_f32_32x32x2f32) for the convs the reference keeps in strict fp32 (f0
// predictor, conv_pre, the first upsampling stage, conv_post, the source downsampling convs).  A workgroup of 4 waves
// owns 128 output rows x 32 WN output channels (waves WM x WN, WM = 4 / WN: 32 WN channels and 128 / WM rows each).
// K runs in stages of 32 values: the activation rows of the stage (activation applied) and its weights are
// loaded into registers one stage ahead (16-byte loads where rows and channels allow: eight lanes per 128-byte row
// segment), stored k-major to one of two LDS buffers, one barrier per stage.  MFMA roles as in the bf16 kernels: the
// weights are the A operand (32 output channels), the activations the B operand (32 output rows).
constexpr int F_BM = 128, F_BK = 32, F_AS = F_BM + 4;  // LDS row strides padded by 4 floats (2-way bank conflicts at most)

template <int WN, bool FLAT>
__global__ void __launch_bounds__(256) conv_f32_kernel(ConvDesc c) {
  constexpr int BN = 32 * WN, WM = 4 / WN, WTM = F_BM / WM, TM = WTM / 32, BS = BN + 4;
  constexpr int AV = F_BM * F_BK / 4 / 256, BV = BN * F_BK / 4 / 256;  // float4 loads per thread and stage
  static_assert(AV >= 1 && BV >= 1, "load layout");
  __shared__ float As[2][F_BK * F_AS];  // [k][row]
  __shared__ float Bs[2][F_BK * BS];    // [k][co]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int b = blockIdx.z / c.n_phase, ph = blockIdx.z % c.n_phase;
  const int Tin = c.in_len[b], Tout = c.out_len[b];
  const int oo = c.off_out[ph];
  // output rows r with 0 <= r * s_out + oo < Tout
  const int r_lo = oo >= 0 ? 0 : (-oo + c.s_out - 1) / c.s_out;
  const int r_hi = Tout - 1 - oo < 0 ? -1 : (Tout - 1 - oo) / c.s_out;
  const int r0 = r_lo + blockIdx.x * F_BM;
  if (r0 > r_hi) return;
  const int co0 = blockIdx.y * BN;
  // the fields the loaders use, as locals (indexing the argument struct inside the lambdas put it in scratch memory)
  const int Cin = c.Cin, Cout = c.Cout, taps = c.taps, s_in = c.s_in, d_in = c.d_in, ldx = c.ldx, off = c.off_in[ph], pre = c.pre;
  const float slope = c.slope;
  const float* alpha = c.alpha;
  const float* inv = c.inv;
  const float* xb = c.x + (size_t)c.in_off[b] * ldx;
  const float* wph = c.w + (size_t)ph * Cout * taps * Cin;
  // K index k = j Cin + ci.  Undilated convs whose Cin is not a multiple of 32 run it flat in chunks of 32 across tap
  // boundaries (tap j + 1's rows follow tap j's, so a chunk is contiguous per output row and a narrow Cin wastes no K);
  // the others by (tap, 32-channel chunk).
  constexpr bool flat = FLAT;
  const int nck = (Cin + F_BK - 1) / F_BK, KT = taps * Cin;
  const int S = flat ? (KT + F_BK - 1) / F_BK : taps * nck;
  const bool vec_x = ldx % 4 == 0, vec_w = Cin % 4 == 0;
  // loader role: row / channel lr + 32 i, K values 4 lf .. 4 lf + 3 of the stage
  const int lr = tid >> 3, lf = tid & 7;
  // flat mode: (tap, channel) of this thread's four K values of stage s (one division per stage); ci = Cin marks a value
  // past K
  auto kdec = [&](int s, int (&jj)[4], int (&cc)[4]) {
    const int k0 = s * F_BK, j0 = k0 / Cin, ci0 = k0 - j0 * Cin + 4 * lf;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int j = j0, ci = ci0 + e;
      while (ci >= Cin) { ci -= Cin; ++j; }  // at most 32 / Cin + 1 steps
      if (j >= taps) { j = 0; ci = Cin; }
      jj[e] = j;
      cc[e] = ci;
    }
  };

  float4 ra[AV], rb[BV];
  // regular K order (tap, 32-channel chunk): one tap and a run of channels per thread and stage
  auto load_chunk = [&](int s) __attribute__((always_inline)) {
    const int j = s / nck, ci = (s - j * nck) * F_BK + 4 * lf;
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int row = r0 + lr + 32 * i;
      const int in_row = row * s_in + j * d_in + off;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row <= r_hi && in_row >= 0 && in_row < Tin) {
        const float* p = xb + (size_t)in_row * ldx + ci;
        if (vec_x && ci + 4 <= Cin) {
          v = *(const float4*)p;
        } else {
          if (ci < Cin) v.x = p[0];
          if (ci + 1 < Cin) v.y = p[1];
          if (ci + 2 < Cin) v.z = p[2];
          if (ci + 3 < Cin) v.w = p[3];
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int co = co0 + lr + 32 * i;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (co < Cout) {
        const float* p = wph + ((size_t)co * taps + j) * Cin + ci;
        if (vec_w && ci + 4 <= Cin) {
          v = *(const float4*)p;
        } else {
          if (ci < Cin) v.x = p[0];
          if (ci + 1 < Cin) v.y = p[1];
          if (ci + 2 < Cin) v.z = p[2];
          if (ci + 3 < Cin) v.w = p[3];
        }
      }
      rb[i] = v;
    }
  };
  auto store_chunk = [&](int s, int buf) __attribute__((always_inline)) {
    const int j = s / nck, ci = (s - j * nck) * F_BK + 4 * lf;
    float al[4] = {0.f, 0.f, 0.f, 0.f}, iv[4] = {0.f, 0.f, 0.f, 0.f};
    if (pre == PRE_SNAKE) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (ci + e < Cin) { al[e] = alpha[ci + e]; iv[e] = inv[ci + e]; }
    }
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int rl = lr + 32 * i;
      const int row = r0 + rl, in_row = row * s_in + j * d_in + off;
      const bool ok = row <= r_hi && in_row >= 0 && in_row < Tin;
      const float v[4] = {ra[i].x, ra[i].y, ra[i].z, ra[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = (pre && ok && ci + e < Cin) ? pre_act(v[e], pre, slope, al[e], iv[e]) : v[e];
        As[buf][(4 * lf + e) * F_AS + rl] = x;
      }
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int cl = lr + 32 * i;
      Bs[buf][(4 * lf + 0) * BS + cl] = rb[i].x;
      Bs[buf][(4 * lf + 1) * BS + cl] = rb[i].y;
      Bs[buf][(4 * lf + 2) * BS + cl] = rb[i].z;
      Bs[buf][(4 * lf + 3) * BS + cl] = rb[i].w;
    }
  };
  // flat K order: each of a thread's four K values has its own (tap, channel)
  auto load_flat = [&](int s) __attribute__((always_inline)) {
    int jj[4], cc[4];
    kdec(s, jj, cc);
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int row = r0 + lr + 32 * i;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (row <= r_hi) {
        const int base = row * s_in + off;
        if (vec_x && vec_w && cc[0] + 4 <= Cin) {  // Cin % 4 == 0: the four values share a tap
          const int in_row = base + jj[0];
          if (in_row >= 0 && in_row < Tin) {
            const float4 q = *(const float4*)(xb + (size_t)in_row * ldx + cc[0]);
            v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int in_row = base + jj[e];
            if (cc[e] < Cin && in_row >= 0 && in_row < Tin) v[e] = xb[(size_t)in_row * ldx + cc[e]];
          }
        }
      }
      ra[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int co = co0 + lr + 32 * i;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (co < Cout) {
        const float* p = wph + (size_t)co * KT;
        if (vec_w && cc[0] + 4 <= Cin) {
          const float4 q = *(const float4*)(p + jj[0] * Cin + cc[0]);
          v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (cc[e] < Cin) v[e] = p[jj[e] * Cin + cc[e]];
        }
      }
      rb[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
  };
  auto store_flat = [&](int s, int buf) __attribute__((always_inline)) {
    int jj[4], cc[4];
    kdec(s, jj, cc);
    float al[4] = {0.f, 0.f, 0.f, 0.f}, iv[4] = {0.f, 0.f, 0.f, 0.f};
    if (pre == PRE_SNAKE) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (cc[e] < Cin) { al[e] = alpha[cc[e]]; iv[e] = inv[cc[e]]; }
    }
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int rl = lr + 32 * i;
      const int row = r0 + rl, base = row * s_in + off;
      const float v[4] = {ra[i].x, ra[i].y, ra[i].z, ra[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int in_row = base + jj[e];
        const bool ok = row <= r_hi && in_row >= 0 && in_row < Tin && cc[e] < Cin;
        As[buf][(4 * lf + e) * F_AS + rl] = (pre && ok) ? pre_act(v[e], pre, slope, al[e], iv[e]) : v[e];
      }
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int cl = lr + 32 * i;
      Bs[buf][(4 * lf + 0) * BS + cl] = rb[i].x;
      Bs[buf][(4 * lf + 1) * BS + cl] = rb[i].y;
      Bs[buf][(4 * lf + 2) * BS + cl] = rb[i].z;
      Bs[buf][(4 * lf + 3) * BS + cl] = rb[i].w;
    }
  };
  auto load = [&](int s) __attribute__((always_inline)) {
    if constexpr (FLAT) load_flat(s);
    else load_chunk(s);
  };
  auto store = [&](int s, int buf) __attribute__((always_inline)) {
    if constexpr (FLAT) store_flat(s, buf);
    else store_chunk(s, buf);
  };

  f32x16 acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  load(0);
  store(0, 0);
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    const int buf = s & 1;
    if (s + 1 < S) load(s + 1);
    const float* A = As[buf];
    const float* B = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < F_BK / 2; ++kk) {
      const int k = 2 * kk + (lane >> 5);
      const float w = B[k * BS + wn * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(w, A[k * F_AS + wm * WTM + i * 32 + (lane & 31)], acc[i], 0, 0, 0);
    }
    if (s + 1 < S) store(s + 1, buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = r0 + wm * WTM + i * 32 + (lane & 31);
    if (r <= r_hi) conv_epilogue(c, b, r * c.s_out + oo, co0 + wn * 32, lane, acc[i]);
  }
}

// The same fp32 convolution with its operands copied straight into LDS (global_load_lds_dwordx4, no register staging
// and no LDS stores), for Cin a multiple of 32 and 16-byte rows.  A stage is one tap and 32 input channels: 128
// activation rows and 32 WN weight rows of 128 bytes, 16-byte chunks XOR-swizzled by (row / 2) % 8; the lanes of an
// instruction name the logical chunk that lands in their physical slot.  Rows outside the item (zero padding) and
// output channels past Cout fetch a 16-byte zero block instead.  A fragment read of 16 bytes gives a lane four K
// values of its row, which feed four v_mfma_f32_32x32x2f32: lane half h of read q holds K values 4 (2 q + h) .. + 3,
// so MFMA (q, m) sums the K pair (8 q + m, 8 q + 4 + m) on both operands.  A leaky-ReLU pre-activation is applied to the
// fragment after the read (zero rows stay zero); Snake convs take conv_f32_kernel (evaluated once per element and stage
// there, not once per element, tap and wave).  Two LDS stages, separate objects, the K loop unrolled by two: the loads
// of stage s + 1 are issued before the MFMAs of stage s.
__device__ __align__(16) float conv_zero16[4];  // never written: the load source of padding rows

__device__ __forceinline__ int fswz(int row, int chunk) { return row * 8 + (chunk ^ ((row >> 1) & 7)); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int WN, int PRE>
__global__ void __launch_bounds__(256, 2) conv_f32_dma_kernel(ConvDesc c) {
  constexpr int BN = 32 * WN, WM = 4 / WN, WTM = F_BM / WM, TM = WTM / 32;
  constexpr int RA = F_BM / 8, NB = RA + BN / 8, PW = NB / 4;  // 8-row load blocks: activations, all, per wave
  static_assert(NB % 4 == 0, "load blocks per wave");
  static_assert(PRE == PRE_NONE || PRE == PRE_LEAKY, "Snake convs take the register-staged kernel (or Snake out of the conv)");
  __shared__ uint4 sA0[F_BM * 8], sA1[F_BM * 8], sB0[BN * 8], sB1[BN * 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int b = blockIdx.z / c.n_phase, ph = blockIdx.z % c.n_phase;
  const int Tin = c.in_len[b], Tout = c.out_len[b];
  const int oo = c.off_out[ph];
  const int r_lo = oo >= 0 ? 0 : (-oo + c.s_out - 1) / c.s_out;
  const int r_hi = Tout - 1 - oo < 0 ? -1 : (Tout - 1 - oo) / c.s_out;
  const int r0 = r_lo + blockIdx.x * F_BM;
  if (r0 > r_hi) return;
  const int co0 = blockIdx.y * BN;
  const int Cin = c.Cin, Cout = c.Cout, taps = c.taps, ldx = c.ldx, d_in = c.d_in;
  const int nck = Cin / 32, S = taps * nck;
  const float* xb = c.x + (size_t)c.in_off[b] * ldx;
  const float* wph = c.w + (size_t)ph * Cout * taps * Cin;
  // this lane's rows of its load blocks: activation row base (tap 0) or weight row, and its logical chunk
  int rbase[PW], lch[PW];
  bool rok[PW];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int blk = wave + 4 * p, trow = (blk < RA ? blk : blk - RA) * 8 + (lane >> 3);
    lch[p] = (lane & 7) ^ ((trow >> 1) & 7);
    if (blk < RA) {
      const int row = r0 + trow;
      rok[p] = row <= r_hi;
      rbase[p] = row * c.s_in + c.off_in[ph];
    } else {
      rok[p] = co0 + trow < Cout;
      rbase[p] = co0 + trow;
    }
  }
  auto issue = [&](uint4* dA, uint4* dB, int s) __attribute__((always_inline)) {
    const int j = s / nck, ci = (s - j * nck) * 32;
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int blk = wave + 4 * p;
      const float* src = conv_zero16;
      uint4* dst;
      if (blk < RA) {
        const int in_row = rbase[p] + j * d_in;
        if (rok[p] && in_row >= 0 && in_row < Tin) src = xb + (size_t)in_row * ldx + ci + lch[p] * 4;
        dst = dA + blk * 64;
      } else {
        if (rok[p]) src = wph + ((size_t)rbase[p] * taps + j) * Cin + ci + lch[p] * 4;
        dst = dB + (blk - RA) * 64;
      }
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)dst, 16, 0, 0);
    }
  };
  f32x16 acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  const float slope = c.slope;
  auto compute = [&](const uint4* A, const uint4* B) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ch = 2 * q + (lane >> 5);
      const float4 wv = *(const float4*)&B[fswz(wn * 32 + (lane & 31), ch)];
      float a[TM][4];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const float4 v = *(const float4*)&A[fswz(wm * WTM + i * 32 + (lane & 31), ch)];
        a[i][0] = v.x; a[i][1] = v.y; a[i][2] = v.z; a[i][3] = v.w;
        if constexpr (PRE == PRE_LEAKY) {
#pragma unroll
          for (int m = 0; m < 4; ++m) a[i][m] = pre_act(a[i][m], PRE_LEAKY, slope, 0.f, 0.f);
        }
      }
      const float w[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(w[m], a[i][m], acc[i], 0, 0, 0);
    }
  };
  issue(sA0, sB0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  for (int s = 0; s < S; s += 2) {
    if (s + 1 < S) issue(sA1, sB1, s + 1);
    compute(sA0, sB0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (s + 1 < S) {
      if (s + 2 < S) issue(sA0, sB0, s + 2);
      compute(sA1, sB1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    }
  }
  // epilogue through a 4 KB LDS slab per wave (the stage buffers are free after the last barrier): each 32 x 32 block
  // goes in as the accumulators lie (lane: row lane % 32, channels q 8 + (lane / 32) 4 ..) and comes back as whole row
  // segments, eight lanes per row of 32 channels, so the output and residual accesses are 16 bytes per lane
  float4* st = (float4*)sA0 + wave * 256;
  const int ncols = min(32, Cout - (co0 + wn * 32));
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    {
      const int t = lane & 31;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c4 = q * 2 + (lane >> 5);
        st[t * 8 + (c4 ^ (t & 7))] = make_float4(acc[i][q * 4], acc[i][q * 4 + 1], acc[i][q * 4 + 2], acc[i][q * 4 + 3]);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int c4 = lane & 7;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int row = rr * 8 + (lane >> 3);
      const int r = r0 + wm * WTM + i * 32 + row;
      const float4 v = st[row * 8 + (c4 ^ (row & 7))];
      if (r > r_hi || c4 * 4 >= ncols) continue;
      const size_t orow = (size_t)c.out_off[b] + (size_t)(r * c.s_out + oo);
      if (c4 * 4 + 3 < ncols) conv_epilogue4<true>(c, orow, co0 + wn * 32 + c4 * 4, v);
      else conv_epilogue_part<true>(c, orow, co0 + wn * 32 + c4 * 4, ncols - c4 * 4, v);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// bf16-MFMA convolution (fp32 activations in HBM, bf16 operands, fp32 accumulation) for stride-1 convs and the
// polyphase transposed convs.  A workgroup owns BM output rows x 64 output channels; its four waves own BM / 4 rows
// each.  For every 64-channel input chunk the input rows of all taps form one slab of BM + (taps - 1) |d| rows, staged
// once in LDS (two 16-byte fp32 loads per thread and row segment, activation applied with the hardware sine, rounded
// to bf16, 16-byte chunks XOR-swizzled by row); each tap then reads the slab rows shifted by its offset, so the tap loop
// has no barrier.  Weight fragments come straight from L2 into registers, the next tap's loaded while this tap's MFMAs
// run.  The epilogue stages each wave's 32-row blocks through LDS and works on whole rows (16-byte accesses).
constexpr int HB_BN = 64, HB_MAXSPAN = 64;

__device__ __forceinline__ int hswz(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

__device__ __forceinline__ float pre_fast(float v, int pre, float slope, float a, float inv) {
  if (pre == PRE_LEAKY) return v > 0.f ? v : v * slope;
  if (pre == PRE_SNAKE) {
    const float s = __sinf(v * a);
    return v + inv * (s * s);
  }
  return v;
}

template <int BM>
__global__ void __launch_bounds__(256, 2) conv_bf16_kernel(ConvDesc c, const bf16_t* __restrict__ wbf) {
  constexpr int NWV = 4, RPP = 32;              // waves; slab rows per pass of the block (8 threads per row)
  constexpr int WTM = BM / NWV, TM = WTM / 32;  // NWV waves along time, each all 64 channels
  // loads batched across rows (slab fill, epilogue) in the 512-row tile (2 waves per SIMD, registers to spare); the
  // 128-row tile keeps 4 waves per SIMD.  Measured: 256-row tiles at 3 waves per SIMD were 10% slower in all.
  constexpr bool BATCH = BM >= 512;
  extern __shared__ uint4 hl[];               // slab [BM + span][8 chunks]; later the epilogue's fp32 blocks
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.z / c.n_phase, ph = blockIdx.z % c.n_phase;
  const int Tin = c.in_len[b], Tout = c.out_len[b];
  const int oo = c.off_out[ph];
  const int r_lo = oo >= 0 ? 0 : (-oo + c.s_out - 1) / c.s_out;
  const int r_hi = Tout - 1 - oo < 0 ? -1 : (Tout - 1 - oo) / c.s_out;
  const int r0 = r_lo + blockIdx.x * BM;
  if (r0 > r_hi) return;
  const int co0 = blockIdx.y * HB_BN;
  const float* xb = c.x + (size_t)c.in_off[b] * c.ldx;
  // tap j reads input row r + j d + off: the slab starts at r0 + min_j(j d) + off
  const int dmin = c.d_in < 0 ? (c.taps - 1) * c.d_in : 0;
  const int slab0 = r0 + dmin + c.off_in[ph];
  const int span = (c.taps - 1) * (c.d_in < 0 ? -c.d_in : c.d_in);
  const int srows = BM + span;
  const int cin_pad = (c.Cin + 63) & ~63;
  // this tile's weights in fragment order: 1 KB blocks (32 output channels, one tap, 16 input channels) in the order
  // (output block, tap, input block), the tile's first block at the row-major offset of its first weight
  const bf16_t* wph = (const bf16_t*)c.wfr + ((size_t)ph * ((c.Cout + 63) & ~63) + co0) * c.taps * cin_pad;
  const int nib = cin_pad / 16;
  // wave-uniform count of this wave's 32-row blocks that hold output rows
  const int live = min(TM, max(0, (r_hi - (r0 + wave * WTM)) / 32 + 1));

  f32x16 acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // this lane's weight fragments of tap j: channel rows co0 + jj * 32 + lane % 32, K chunk kk * 2 + lane / 32 (one
  // contiguous kilobyte per (kk, jj) for the wave)
  auto load_w = [&](int j, int c0, bf16x8 (&w)[4][2]) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        w[kk][jj] = as_bf16x8(*(const uint4*)(wph + ((size_t)((jj * c.taps + j) * nib + (c0 >> 4) + kk) * 512 + lane * 8)));
  };
  const int sch = tid & 7;  // this thread's 8-channel chunk of the slab rows
  for (int c0 = 0; c0 < c.Cin; c0 += 64) {
    __syncthreads();  // the previous chunk's slab is no longer read
    const int ci = c0 + sch * 8;
    float al[8], iv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      al[e] = (c.pre == PRE_SNAKE && ci + e < c.Cin) ? c.alpha[ci + e] : 0.f;
      iv[e] = (c.pre == PRE_SNAKE && ci + e < c.Cin) ? c.inv[ci + e] : 0.f;
    }
    // slab row sr from its two loaded float4 (row inside the input, all 8 channels inside Cin), or element by element
    auto put_fast = [&](int sr, float4 u0, float4 u1) {
      float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = pre_fast(v[e], c.pre, c.slope, al[e], iv[e]);
      hl[hswz(sr, sch)] = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
    };
    auto put_edge = [&](int sr, int in_row) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float xv = 0.f;
        if (in_row >= 0 && in_row < Tin && ci + e < c.Cin) xv = pre_fast(xb[(size_t)in_row * c.ldx + ci + e], c.pre, c.slope, al[e], iv[e]);
        v[e] = xv;
      }
      hl[hswz(sr, sch)] = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
    };
    if constexpr (!BATCH) {  // one slab row at a time: keeps the register budget of 4 waves per SIMD
      for (int sr = tid >> 3; sr < srows; sr += RPP) {
        const int in_row = slab0 + sr;
        if (in_row >= 0 && in_row < Tin && ci + 8 <= c.Cin)
          put_fast(sr, *(const float4*)(xb + (size_t)in_row * c.ldx + ci), *(const float4*)(xb + (size_t)in_row * c.ldx + ci + 4));
        else
          put_edge(sr, in_row);
      }
    } else {  // SU slab rows per thread and pass, all their loads in flight before the first one is used
      constexpr int SU = 4;
      for (int sr0 = tid >> 3; sr0 < srows; sr0 += RPP * SU) {
        float4 u[SU][2];
        bool fast[SU];
#pragma unroll
        for (int x = 0; x < SU; ++x) {
          const int sr = sr0 + RPP * x, in_row = slab0 + sr;
          fast[x] = sr < srows && in_row >= 0 && in_row < Tin && ci + 8 <= c.Cin;
          if (fast[x]) {
            u[x][0] = *(const float4*)(xb + (size_t)in_row * c.ldx + ci);
            u[x][1] = *(const float4*)(xb + (size_t)in_row * c.ldx + ci + 4);
          }
        }
#pragma unroll
        for (int x = 0; x < SU; ++x) {
          const int sr = sr0 + RPP * x;
          if (sr >= srows) break;
          if (fast[x]) put_fast(sr, u[x][0], u[x][1]);
          else put_edge(sr, slab0 + sr);
        }
      }
    }
    bf16x8 wa[4][2], wb[4][2];
    load_w(0, c0, wa);
    __syncthreads();
    for (int j = 0; j < c.taps; ++j) {
      if (j + 1 < c.taps) load_w(j + 1, c0, wb);
      const int shift = j * c.d_in - dmin;  // slab row of output row r0 + i for this tap: i + shift
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int chunk = kk * 2 + (lane >> 5);
        bf16x8 af[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = as_bf16x8(hl[hswz(wave * WTM + i * 32 + (lane & 31) + shift, chunk)]);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          if (i >= live) break;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[kk][jj], af[i], acc[i][jj], 0, 0, 0);
        }
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) wa[kk][jj] = wb[kk][jj];
    }
  }

  // epilogue: each wave stages one 32-row x 64-channel block at a time (fp32, 16 chunks of 4 channels per row,
  // chunk c at c ^ (row & 15)), then reads it back four rows per instruction
  __syncthreads();
  float4* st = (float4*)hl + wave * (32 * 16);
  const int ncols = min(HB_BN, c.Cout - co0);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    if (i >= live) break;
    const int t = lane & 31;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c4 = jj * 8 + q * 2 + (lane >> 5);
        st[t * 16 + (c4 ^ (t & 15))] = make_float4(acc[i][jj][q * 4], acc[i][jj][q * 4 + 1], acc[i][jj][q * 4 + 2], acc[i][jj][q * 4 + 3]);
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int c4 = lane & 15;
    if constexpr (!BATCH) {
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const int row = rr * 4 + (lane >> 4);
        const int r = r0 + wave * WTM + i * 32 + row;
        const float4 v = st[row * 16 + (c4 ^ (row & 15))];
        if (r > r_hi || c4 * 4 >= ncols) continue;
        const size_t orow = (size_t)c.out_off[b] + (size_t)(r * c.s_out + oo);
        if (c4 * 4 + 3 < ncols) conv_epilogue4(c, orow, co0 + c4 * 4, v);
        else conv_epilogue_part(c, orow, co0 + c4 * 4, ncols - c4 * 4, v);
      }
    } else {
      // the eight rows of this lane: every residual / accumulator load in flight before the first store
      float4 vv4[8], rr4[8], tt4[8];
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const int row = rr * 4 + (lane >> 4);
        const int r = r0 + wave * WTM + i * 32 + row;
        vv4[rr] = st[row * 16 + (c4 ^ (row & 15))];
        rr4[rr] = tt4[rr] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r <= r_hi && c4 * 4 + 3 < ncols)
          conv_epilogue4_loads(c, (size_t)c.out_off[b] + (size_t)(r * c.s_out + oo), co0 + c4 * 4, rr4[rr], tt4[rr]);
      }
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const int row = rr * 4 + (lane >> 4);
        const int r = r0 + wave * WTM + i * 32 + row;
        if (r > r_hi || c4 * 4 >= ncols) continue;
        const size_t orow = (size_t)c.out_off[b] + (size_t)(r * c.s_out + oo);
        if (c4 * 4 + 3 < ncols) conv_epilogue4_pre(c, orow, co0 + c4 * 4, vv4[rr], rr4[rr], tt4[rr]);
        else conv_epilogue_part(c, orow, co0 + c4 * 4, ncols - c4 * 4, vv4[rr]);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// One ResBlock dilation in one pass on bf16 MFMA: y = conv2(snake2(conv1(snake1(x)))) + x, both convs C -> C channels
// with kernel k and zero padding at each item's ends, conv1 dilated by dil (padding dil (k - 1) / 2), conv2 undilated
// (padding (k - 1) / 2).  A workgroup owns BO = BM1 - (k - 1) output rows and all C channels.  conv1 runs over the BM1
// rows conv2 reads (its halo included) in 64-channel input chunks staged in LDS as in conv_bf16_kernel; its result,
// bias and Snake applied, rounded to bf16 and zero outside the item, is written to LDS over the dead input slab (all C
// channels) and is conv2's input, read with no barrier in conv2's tap loop.  So conv1's output never goes through HBM
// and the residual is the block's own input rows (L2 hits).  Four waves split the BM1 x C tile into blocks of 128 rows x
// 64 channels; BM1 = 32768 / C keeps the conv2 slab at 64 KB.  Each output sums its products in the order
// conv_bf16_kernel does (64-channel chunks, taps, 16-channel steps), and the roundings are the same (conv1 + bias in fp32,
// Snake, bf16), so the result equals the two-kernel path's.
constexpr int RP_SPAN = 64;  // conv1's largest tap span (k - 1) dil

template <int C>
__global__ void __launch_bounds__(256, 2) resblock_pair_kernel(ConvDesc c1, ConvDesc c2) {
  constexpr int BM1 = 32768 / C, WN = C / 64, WM = 4 / WN, WTM = BM1 / WM, TM = WTM / 32;
  constexpr int CH = C / 8, MSK = (CH < 16 ? CH : 16) - 1;  // conv2 slab: 16-byte chunks per row; XOR swizzle mask
  static_assert(WTM == 128 && TM == 4, "waves own 128 rows x 64 channels");
  constexpr int SU = C == 64 ? 4 : 2;  // slab rows per thread in flight while staging (registers: acc is live in later chunks)
  extern __shared__ uint4 hl[];  // conv1's input slab [BM1 + span][8 chunks]; then conv2's [BM1 + 16][CH]; then the epilogue's
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int b = blockIdx.y;
  const int T = c1.in_len[b];
  const int k = c1.taps, dil = c1.d_in;
  const int h2 = (k - 1) >> 1, BO = BM1 - 2 * h2;
  const int r0 = blockIdx.x * BO;
  if (r0 >= T) return;
  const int t0 = r0 - h2;        // item time of conv2 slab row 0 (conv1 output row)
  const int u0 = t0 - h2 * dil;  // item time of conv1 slab row 0
  const int srows = BM1 + (k - 1) * dil;
  const float* xb = c1.x + (size_t)c1.in_off[b] * C;
  const bf16_t* w1 = (const bf16_t*)c1.wfr + (size_t)wn * 64 * k * C;  // fragment order, this wave's 64 output channels
  const bf16_t* w2 = (const bf16_t*)c2.wfr + (size_t)wn * 64 * k * C;
  const float* a1 = c1.alpha;
  const float* iv1 = c1.inv;
  const int ws = wm * WTM;  // this wave's first tile row
  // wave-uniform counts of this wave's live 32-row blocks: conv1 rows that conv2 reads for an output row inside the
  // item, conv2 rows inside the item and the workgroup's BO
  const int n1 = T - r0 + 2 * h2 - ws, n2 = min(BO, T - r0) - ws;
  const int live1 = n1 <= 0 ? 0 : min(TM, (n1 + 31) >> 5);
  const int live2 = n2 <= 0 ? 0 : min(TM, (n2 + 31) >> 5);

  f32x16 acc[TM][2];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // this lane's fragments of tap j, input channels c0 .. c0 + 63: channel rows jj * 32 + lane % 32 of the wave's 64
  // (one contiguous kilobyte per (kk, jj) for the wave)
  auto load_w = [&](const bf16_t* w, int j, int c0, bf16x8 (&f)[4][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        f[kk][jj] = as_bf16x8(*(const uint4*)(w + ((size_t)((jj * k + j) * (C / 16) + (c0 >> 4) + kk)) * 512 + lane * 8));
  };

  // conv1 over the BM1 rows, one 64-channel input chunk at a time
  const int sch = tid & 7;
  for (int c0 = 0; c0 < C; c0 += 64) {
    __syncthreads();  // the previous chunk's slab is no longer read
    const int ci = c0 + sch * 8;
    float al[8], iv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { al[e] = a1[ci + e]; iv[e] = iv1[ci + e]; }
    for (int sr0 = tid >> 3; sr0 < srows; sr0 += 32 * SU) {
      float4 u[SU][2];
      bool in[SU];
#pragma unroll
      for (int x = 0; x < SU; ++x) {
        const int sr = sr0 + 32 * x, t = u0 + sr;
        in[x] = sr < srows && t >= 0 && t < T;
        if (in[x]) {
          u[x][0] = *(const float4*)(xb + (size_t)t * C + ci);
          u[x][1] = *(const float4*)(xb + (size_t)t * C + ci + 4);
        }
      }
#pragma unroll
      for (int x = 0; x < SU; ++x) {
        const int sr = sr0 + 32 * x;
        if (sr >= srows) break;
        uint4 o = make_uint4(0u, 0u, 0u, 0u);
        if (in[x]) {
          float v[8] = {u[x][0].x, u[x][0].y, u[x][0].z, u[x][0].w, u[x][1].x, u[x][1].y, u[x][1].z, u[x][1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = pre_fast(v[e], PRE_SNAKE, 0.f, al[e], iv[e]);
          o = make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
        }
        hl[hswz(sr, sch)] = o;
      }
    }
    // taps in pairs with the two weight sets in fixed roles: the loads of tap j + 1 (into wb) and j + 2 (into wa) are
    // issued before the MFMAs of taps j and j + 1
    bf16x8 wa[4][2], wb[4][2];
    auto tap1 = [&](const bf16x8 (&w)[4][2], int j) __attribute__((always_inline)) {
      const int shift = j * dil;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int chunk = kk * 2 + (lane >> 5);
        bf16x8 af[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = as_bf16x8(hl[hswz(ws + i * 32 + (lane & 31) + shift, chunk)]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w[kk][jj], af[i], acc[i][jj], 0, 0, 0);
      }
    };
    load_w(w1, 0, c0, wa);
    __syncthreads();
    for (int j = 0; j < k; j += 2) {
      if (j + 1 < k) load_w(w1, j + 1, c0, wb);
      tap1(wa, j);
      if (j + 1 < k) {
        if (j + 2 < k) load_w(w1, j + 2, c0, wa);
        tap1(wb, j + 1);
      }
    }
  }

  // conv1's output to the conv2 slab: row s, 16-byte chunk c at s * CH + (c ^ (s & MSK)); this lane holds row
  // ws + i * 32 + lane % 32 and, per (jj, q), the four channels wn * 64 + jj * 32 + q * 8 + (lane / 32) * 4 ..
  __syncthreads();  // every wave is done with conv1's slab
  {
    uint2* s2 = (uint2*)hl;
    const float* b1 = c1.bias;
    const float* a2 = c2.alpha;
    const float* iv2 = c2.inv;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int ch = wn * 64 + jj * 32 + q * 8 + (lane >> 5) * 4;
        const float4 bb = *(const float4*)(b1 + ch), aa = *(const float4*)(a2 + ch), ii = *(const float4*)(iv2 + ch);
        const int chunk = wn * 8 + jj * 4 + q;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          if (i >= live1) break;
          const int s = ws + i * 32 + (lane & 31), t = t0 + s;
          float v[4] = {__fadd_rn(acc[i][jj][q * 4], bb.x), __fadd_rn(acc[i][jj][q * 4 + 1], bb.y),
                        __fadd_rn(acc[i][jj][q * 4 + 2], bb.z), __fadd_rn(acc[i][jj][q * 4 + 3], bb.w)};
          v[0] = pre_fast(v[0], PRE_SNAKE, 0.f, aa.x, ii.x);
          v[1] = pre_fast(v[1], PRE_SNAKE, 0.f, aa.y, ii.y);
          v[2] = pre_fast(v[2], PRE_SNAKE, 0.f, aa.z, ii.z);
          v[3] = pre_fast(v[3], PRE_SNAKE, 0.f, aa.w, ii.w);
          const bool inside = t >= 0 && t < T;
          s2[(s * CH + (chunk ^ (s & MSK))) * 2 + (lane >> 5)] = inside ? make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3])) : make_uint2(0u, 0u);
        }
      }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  __syncthreads();

  // conv2: output row o reads conv2 slab rows o .. o + k - 1; the (chunk, tap) steps in conv_bf16_kernel's order, the
  // next step's weights loaded while this step's MFMAs run
  {
    bf16x8 wa[4][2], wb[4][2];
    auto tap2 = [&](const bf16x8 (&w)[4][2], int j, int c0) __attribute__((always_inline)) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int chunk = (c0 >> 3) + kk * 2 + (lane >> 5);
        bf16x8 af[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int s = ws + i * 32 + (lane & 31) + j;
          af[i] = as_bf16x8(hl[s * CH + (chunk ^ (s & MSK))]);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w[kk][jj], af[i], acc[i][jj], 0, 0, 0);
      }
    };
    // the (chunk, tap) step after (j, c0)
    auto next = [&](int& j, int& c0) __attribute__((always_inline)) {
      if (j + 1 == k) { j = 0; c0 += 64; } else { ++j; }
    };
    load_w(w2, 0, 0, wa);
    const int steps = (C / 64) * k;
    int j = 0, c0 = 0;
    for (int sidx = 0; sidx < steps; sidx += 2) {  // steps in pairs, weight sets in fixed roles as in conv1
      int j1 = j, c1 = c0;
      next(j1, c1);
      if (sidx + 1 < steps) load_w(w2, j1, c1, wb);
      tap2(wa, j, c0);
      if (sidx + 1 < steps) {
        int j2 = j1, c2 = c1;
        next(j2, c2);
        if (sidx + 2 < steps) load_w(w2, j2, c2, wa);
        tap2(wb, j1, c1);
        j = j2;
        c0 = c2;
      }
    }
  }

  // epilogue as in conv_bf16_kernel: bias, residual (the input rows), and the output / running-mean update.  Each
  // block's residual rows are loaded one block ahead (block 0's before the barrier), so their latency overlaps the
  // previous block's stores instead of being paid once per block.
  const int co0 = wn * 64;
  const int r_end = min(r0 + BO, T);
  const int c4 = lane & 15;
  const size_t row0 = (size_t)c2.out_off[b];
  const float* resb = c2.res + row0 * C;
  auto res_loads = [&](int i, float4 (&rv)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int r = r0 + ws + i * 32 + rr * 4 + (lane >> 4);
      rv[rr] = r < r_end ? *(const float4*)(resb + (uint32_t)(r * C + co0 + c4 * 4)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  float4 rn[8];
  if (live2 > 0) res_loads(0, rn);
  __syncthreads();  // every wave is done with the conv2 slab
  float4* st = (float4*)hl + wave * (32 * 16);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    if (i >= live2) break;
    float4 rr4[8];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) rr4[rr] = rn[rr];
    const int t = lane & 31;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cc = jj * 8 + q * 2 + (lane >> 5);
        st[t * 16 + (cc ^ (t & 15))] = make_float4(acc[i][jj][q * 4], acc[i][jj][q * 4 + 1], acc[i][jj][q * 4 + 2], acc[i][jj][q * 4 + 3]);
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float4 vv4[8];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int row = rr * 4 + (lane >> 4);
      vv4[rr] = st[row * 16 + (c4 ^ (row & 15))];
    }
    if (i + 1 < live2) res_loads(i + 1, rn);
    // the running sum / accumulated output (the stage's last dilation only) per row, next to its store
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int row = rr * 4 + (lane >> 4);
      const int r = r0 + ws + i * 32 + row;
      if (r < r_end) {
        const uint32_t o = (uint32_t)(r * C + co0 + c4 * 4);
        float4 t4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c2.epi == EPI_ADD_RES) t4 = *(const float4*)(c2.y + row0 * C + o);
        else if (c2.epi == EPI_RES_MEAN && c2.sum_mode != 0) t4 = *(const float4*)(c2.sum + row0 * C + o);
        conv_epilogue4_pre(c2, row0 + (size_t)r, co0 + c4 * 4, vv4[rr], rr4[rr], t4);
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// Small grids (a streaming window: one item of a few thousand samples) leave most CUs idle with whole-slab tiles, and
// each tile's tap loop is a chain of weight-load latencies.  Here a workgroup of CS_WAVES waves owns 32 output rows x
// NB * 32 output channels and splits the (tap, 64-channel input chunk) steps over its waves, the next step's loads
// issued before this step's MFMAs; the waves' fp32 blocks are summed through LDS in wave order (deterministic) and the
// epilogue writes four channels per thread.  A CU's load throughput bounds these calls, so (as in the small-row GEMM)
// the loads cover whole lines: a step's weights are NB * 32 rows of 128 bytes, eight lanes per row; its activations 32
// rows of 64 fp32 channels, sixteen lanes per row (activation applied, rounded to bf16).  Both go through the wave's
// LDS slab (16-byte chunks XOR-swizzled by (row / 2) % 8) and come back as MFMA fragments.  NB = 1 halves the weight
// bytes each workgroup reads where the grid stays within the chip.  MFMA roles as in the small-row GEMM: the weights
// are the A operand (32 output channels), the activations the B operand (32 output rows).
constexpr int CS_WAVES = 8;

template <int NB>
__global__ void __launch_bounds__(64 * CS_WAVES) conv_bf16_split_kernel(ConvDesc c, const bf16_t* __restrict__ wbf) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  __shared__ u32x4 slab[CS_WAVES][(NB + 1) * 256];  // per wave: W rows then activation rows of a step; then its blocks
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, cl = lane & 31;
  const int b = blockIdx.z / c.n_phase, ph = blockIdx.z % c.n_phase;
  const int Tin = c.in_len[b], Tout = c.out_len[b];
  const int oo = c.off_out[ph];
  const int r_lo = oo >= 0 ? 0 : (-oo + c.s_out - 1) / c.s_out;
  const int r_hi = Tout - 1 - oo < 0 ? -1 : (Tout - 1 - oo) / c.s_out;
  const int r0 = r_lo + blockIdx.x * 32;
  if (r0 > r_hi) return;  // the whole workgroup leaves together
  const int co0 = blockIdx.y * (NB * 32);
  const float* xb = c.x + (size_t)c.in_off[b] * c.ldx;
  const int cin_pad = (c.Cin + 63) & ~63, nch = cin_pad / 64;
  // rows co0 .. co0 + NB * 32 - 1 exist: the weights are padded to 64 output channels
  const bf16_t* wph = wbf + ((size_t)ph * ((c.Cout + 63) & ~63) + co0) * c.taps * cin_pad;
  const int NS = c.taps * nch;
  const int s0 = w * NS / CS_WAVES, s1 = (w + 1) * NS / CS_WAVES;  // this wave's steps (possibly none)
  const int wr = lane >> 3, wc = lane & 7;    // weight loads: row i * 8 + wr, 16-byte chunk wc
  const int xr = lane >> 4, xc = lane & 15;   // activation loads: row i * 4 + xr, channels xc * 4 .. + 3

  // step st: tap j = st / nch, input channels cc .. cc + 63 with cc = (st % nch) * 64
  auto load = [&](int st, float4 (&xv)[8], u32x4 (&wv)[4 * NB]) {
    const int j = st / nch, cc = (st - j * nch) * 64;
#pragma unroll
    for (int i = 0; i < 4 * NB; ++i)
      wv[i] = *(const u32x4*)(wph + ((size_t)(i * 8 + wr) * c.taps + j) * cin_pad + cc + wc * 8);
    const int ch = cc + xc * 4;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = r0 + i * 4 + xr, in_row = r + j * c.d_in + c.off_in[ph];
      const bool rok = r <= r_hi && in_row >= 0 && in_row < Tin;
      const float* xp = xb + (size_t)(rok ? in_row : 0) * c.ldx + ch;
      if (rok && ch + 3 < c.Cin) xv[i] = *(const float4*)xp;
      else {
        float t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = (rok && ch + u < c.Cin) ? xp[u] : 0.f;
        xv[i] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
  };
  // activation (zero inputs stay zero: the padding rows and channels of the reference's zero-padded conv), bf16, slab,
  // fragments, MFMAs
  auto mma = [&](int st, const float4 (&xv)[8], const u32x4 (&wv)[4 * NB], f32x16 (&acc)[NB]) {
    const int j = st / nch, cc = (st - j * nch) * 64, ch = cc + xc * 4;
    float al[4] = {0.f, 0.f, 0.f, 0.f}, iv[4] = {0.f, 0.f, 0.f, 0.f};
    if (c.pre == PRE_SNAKE) {
      if (ch + 3 < c.Cin) {
        const float4 a4 = *(const float4*)(c.alpha + ch), i4 = *(const float4*)(c.inv + ch);
        al[0] = a4.x; al[1] = a4.y; al[2] = a4.z; al[3] = a4.w;
        iv[0] = i4.x; iv[1] = i4.y; iv[2] = i4.z; iv[3] = i4.w;
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          al[u] = ch + u < c.Cin ? c.alpha[ch + u] : 0.f;
          iv[u] = ch + u < c.Cin ? c.inv[ch + u] : 0.f;
        }
      }
    }
    u32x4* sl = slab[w];
#pragma unroll
    for (int i = 0; i < 4 * NB; ++i) {
      const int r = i * 8 + wr;
      sl[r * 8 + (wc ^ ((r >> 1) & 7))] = wv[i];
    }
    u32x2* sx = (u32x2*)(sl + NB * 256);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = i * 4 + xr, r = r0 + rr, in_row = r + j * c.d_in + c.off_in[ph];
      const bool rok = r <= r_hi && in_row >= 0 && in_row < Tin;
      const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
      float o[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) o[u] = (rok && ch + u < c.Cin) ? pre_fast(v[u], c.pre, c.slope, al[u], iv[u]) : 0.f;
      u32x2 pk;
      pk.x = pack2(o[0], o[1]);
      pk.y = pack2(o[2], o[3]);
      sx[(rr * 8 + ((xc >> 1) ^ ((rr >> 1) & 7))) * 2 + (xc & 1)] = pk;
    }
    u32x4 xf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) xf[kk] = sl[NB * 256 + cl * 8 + ((h * 4 + kk) ^ ((cl >> 1) & 7))];
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) {
      u32x4 wf[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) wf[kk] = sl[(jj * 32 + cl) * 8 + ((h * 4 + kk) ^ ((cl >> 1) & 7))];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        acc[jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wf[kk]), __builtin_bit_cast(bf16x8, xf[kk]), acc[jj], 0, 0, 0);
    }
  };

  f32x16 acc[NB];
#pragma unroll
  for (int jj = 0; jj < NB; ++jj)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[jj][i] = 0.f;
  float4 xa[8], xb2[8];
  u32x4 wa[4 * NB], wb2[4 * NB];
  // two register sets named at compile time: the loop runs two steps per pass
  if (s0 < s1) load(s0, xa, wa);
  for (int st = s0; st < s1; st += 2) {
    if (st + 1 < s1) load(st + 1, xb2, wb2);
    mma(st, xa, wa, acc);
    if (st + 1 < s1) {
      if (st + 2 < s1) load(st + 2, xa, wa);
      mma(st + 1, xb2, wb2, acc);
    }
  }
  float4* red = (float4*)slab[w];  // [block jj][quad q][lane]; the wave's own slab (its LDS accesses complete in order)
#pragma unroll
  for (int jj = 0; jj < NB; ++jj)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(jj * 4 + q) * 64 + lane] = make_float4(acc[jj][4 * q], acc[jj][4 * q + 1], acc[jj][4 * q + 2], acc[jj][4 * q + 3]);
  __syncthreads();

  // one float4 (four channels of one row) per thread, summed over the waves in order
  if (tid >= NB * 256) return;
  const int jj = tid >> 8, q = (tid >> 6) & 3, l = tid & 63;
  float4 sum = ((const float4*)slab[0])[(jj * 4 + q) * 64 + l];
#pragma unroll
  for (int x = 1; x < CS_WAVES; ++x) {
    const float4 v = ((const float4*)slab[x])[(jj * 4 + q) * 64 + l];
    sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
  }
  // lane l of the MFMA holds output row r0 + l % 32 and channels co0 + jj * 32 + q * 8 + (l / 32) * 4 + 0..3
  const int ro = r0 + (l & 31), cn = jj * 32 + q * 8 + (l >> 5) * 4;
  const int ncols = min(NB * 32, c.Cout - co0);
  if (ro > r_hi || cn >= ncols) return;
  const size_t orow = (size_t)c.out_off[b] + (size_t)(ro * c.s_out + oo);
  if (cn + 3 < ncols) conv_epilogue4(c, orow, co0 + cn, sum);
  else conv_epilogue_part(c, orow, co0 + cn, ncols - cn, sum);
}

// The fp32 convolution for small grids (the f0 predictor of a streaming window: ~50 frames x 512 channels), on the
// same plan as conv_bf16_split_kernel: 32 output rows x NB * 32 output channels per workgroup, the (tap, 32-channel input
// chunk) steps split over the waves, operands straight into registers with the next step's loads in flight, fp32 MFMA
// (v_mfma_f32_32x32x2f32; lane half h supplies channels h * 16 + u of MFMA u on both sides), blocks summed in LDS in
// wave order.
template <int NB>
__global__ void __launch_bounds__(64 * CS_WAVES) conv_f32_split_kernel(ConvDesc c) {
  __shared__ float4 red[CS_WAVES][NB][4][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, cl = lane & 31;
  const int b = blockIdx.z / c.n_phase, ph = blockIdx.z % c.n_phase;
  const int Tin = c.in_len[b], Tout = c.out_len[b];
  const int oo = c.off_out[ph];
  const int r_lo = oo >= 0 ? 0 : (-oo + c.s_out - 1) / c.s_out;
  const int r_hi = Tout - 1 - oo < 0 ? -1 : (Tout - 1 - oo) / c.s_out;
  const int r0 = r_lo + blockIdx.x * 32;
  if (r0 > r_hi) return;
  const int co0 = blockIdx.y * (NB * 32);
  const float* xb = c.x + (size_t)c.in_off[b] * c.ldx;
  const float* wph = c.w + (size_t)ph * c.Cout * c.taps * c.Cin;
  const int nch = (c.Cin + 31) / 32, NS = c.taps * nch;
  const int s0 = w * NS / CS_WAVES, s1 = (w + 1) * NS / CS_WAVES;
  const int r = r0 + cl;
  const bool vec = c.Cin % 4 == 0 && c.ldx % 4 == 0;  // 16-byte loads of whole 4-channel groups

  // step s: tap j = s / nch, this lane's channels cc .. cc + 15 with cc = (s % nch) * 32 + h * 16, activation applied
  auto load = [&](int st, float4 (&xv)[4], float4 (&wv)[NB][4]) {
    const int j = st / nch, cc = (st - j * nch) * 32 + h * 16;
    const int in_row = r * c.s_in + j * c.d_in + c.off_in[ph];
    const bool rok = r <= r_hi && in_row >= 0 && in_row < Tin;
    const float* xp = xb + (size_t)(rok ? in_row : 0) * c.ldx + cc;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (vec && rok && cc + e * 4 + 3 < c.Cin) xv[e] = *(const float4*)(xp + e * 4);
      else {
        float t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u] = (rok && cc + e * 4 + u < c.Cin) ? xp[e * 4 + u] : 0.f;
        xv[e] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
#pragma unroll
    for (int jj = 0; jj < NB; ++jj) {
      const int co = co0 + jj * 32 + cl;
      const float* wp = wph + ((size_t)(co < c.Cout ? co : 0) * c.taps + j) * c.Cin + cc;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (vec && co < c.Cout && cc + e * 4 + 3 < c.Cin) wv[jj][e] = *(const float4*)(wp + e * 4);
        else {
          float t[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) t[u] = (co < c.Cout && cc + e * 4 + u < c.Cin) ? wp[e * 4 + u] : 0.f;
          wv[jj][e] = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
    }
  };
  auto mma = [&](int st, const float4 (&xv)[4], const float4 (&wv)[NB][4], f32x16 (&acc)[NB]) {
    const int j = st / nch, cc = (st - j * nch) * 32 + h * 16;
    const int in_row = r * c.s_in + j * c.d_in + c.off_in[ph];
    const bool rok = r <= r_hi && in_row >= 0 && in_row < Tin;
    const float xs[16] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w,
                          xv[2].x, xv[2].y, xv[2].z, xv[2].w, xv[3].x, xv[3].y, xv[3].z, xv[3].w};
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int ci = cc + u;
      const bool ok = rok && ci < c.Cin;
      float v = xs[u];
      if (c.pre && ok) v = pre_act(v, c.pre, c.slope, c.alpha ? c.alpha[ci] : 0.f, c.inv ? c.inv[ci] : 0.f);
      v = ok ? v : 0.f;
#pragma unroll
      for (int jj = 0; jj < NB; ++jj) {
        const float4 w4 = wv[jj][u >> 2];
        const float a = (u & 3) == 0 ? w4.x : (u & 3) == 1 ? w4.y : (u & 3) == 2 ? w4.z : w4.w;
        acc[jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, v, acc[jj], 0, 0, 0);
      }
    }
  };

  f32x16 acc[NB];
#pragma unroll
  for (int jj = 0; jj < NB; ++jj)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[jj][i] = 0.f;
  float4 xa[4], xb2[4], wa[NB][4], wb2[NB][4];
  if (s0 < s1) load(s0, xa, wa);
  for (int st = s0; st < s1; st += 2) {
    if (st + 1 < s1) load(st + 1, xb2, wb2);
    mma(st, xa, wa, acc);
    if (st + 1 < s1) {
      if (st + 2 < s1) load(st + 2, xa, wa);
      mma(st + 1, xb2, wb2, acc);
    }
  }
#pragma unroll
  for (int jj = 0; jj < NB; ++jj)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[w][jj][q][lane] = make_float4(acc[jj][4 * q], acc[jj][4 * q + 1], acc[jj][4 * q + 2], acc[jj][4 * q + 3]);
  __syncthreads();
  if (tid >= NB * 256) return;
  const int jj = tid >> 8, q = (tid >> 6) & 3, l = tid & 63;
  float4 sum = red[0][jj][q][l];
#pragma unroll
  for (int x = 1; x < CS_WAVES; ++x) {
    const float4 v = red[x][jj][q][l];
    sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
  }
  const int ro = r0 + (l & 31), cn = jj * 32 + q * 8 + (l >> 5) * 4;
  const int ncols = min(NB * 32, c.Cout - co0);
  if (ro > r_hi || cn >= ncols) return;
  const size_t orow = (size_t)c.out_off[b] + (size_t)(ro * c.s_out + oo);
  if (cn + 3 < ncols) conv_epilogue4<true>(c, orow, co0 + cn, sum);
  else conv_epilogue_part<true>(c, orow, co0 + cn, ncols - cn, sum);
}

// f0 = |w . x + b| per frame (one wave per frame row, Linear(C -> 1) then abs)
__global__ void __launch_bounds__(256) f0_head_kernel(const float* x, int C, const float* w, const float* b, float* f0, int rows) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  float s = 0.f;
  for (int c = lane; c < C; c += 64) s += x[(size_t)r * C + c] * w[c];
  s = wave_sum(s);
  if (lane == 0) f0[r] = fabsf(s + b[0]);
}

// Frame-rate phase of harmonic h of item i: rad_f = (f0_f (h + 1) / sr) mod 1; phase_f = (sum_{g <= f} rad_g) 2 pi;
// stored already multiplied by the upsampling scale (the reference's F.interpolate(phase * 480, scale 480) input).
// The running sum is an fp64 accumulation rounded to fp32 per frame, as torch's CPU cumsum does for fp32.  One wave per
// (item, harmonic) scans 64 frames at a time (shuffle scan, then the carry of the earlier frames): rad values of f0
// above ~1e-4 Hz are multiples of 2^-38 and the sums stay below the frame count, so fp64 holds every partial sum
// exactly and the scan equals the sequential sum.
__global__ void __launch_bounds__(256) phase_kernel(const float* f0, const int* fr_off, const int* fr_len, int n_items, int harm, float sr,
                                                    float scale, float* phase) {
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (w >= n_items * harm) return;
  const int it = w / harm, h = w % harm;
  const int o = fr_off[it], T = fr_len[it];
  const float mult = (float)(h + 1);
  double carry = 0.0;
  for (int b = 0; b < T; b += 64) {
    const int f = b + lane;
    double r = 0.0;
    if (f < T) {
      const float fn = __fmul_rn(f0[o + f], mult);
      r = (double)fmodf(__fdiv_rn(fn, sr), 1.0f);
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const double t = __shfl_up(r, d, 64);
      if (lane >= d) r += t;
    }
    const double cum = carry + r;
    if (f < T) {
      const float ph = __fmul_rn(__fmul_rn((float)cum, 2.0f), 3.14159265358979323846f);
      phase[(size_t)(o + f) * harm + h] = __fmul_rn(ph, scale);
    }
    carry = __shfl(cum, 63, 64);
  }
}

// Per sample n of item i: phase_n by linear interpolation of the frame phases (align_corners=False, source index
// (n + 0.5) / scale - 0.5 clamped at 0), sine = sin(phase) amp, voiced/unvoiced noise mix, tanh(Linear(9 -> 1)); the
// first S samples come from the item's source cache.
__global__ void source_kernel(const float* phase, const float* f0, const int* fr_off, const int* fr_len, const int* smp_off,
                              int n_items, int harm, float inv_scale, int up, float amp, float noise_std, float unv, float thr,
                              const float* noise, const float* lw, const float* lb, const float* cache, int S, float* out) {
  const int it = blockIdx.y;
  const int T = fr_len[it];
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int ns = T * up;
  if (n >= ns) return;
  const size_t so = (size_t)smp_off[it] + n;
  if (n < S) {
    out[so] = cache[(size_t)it * S + n];
    return;
  }
  const int fo = fr_off[it];
  float src = __fsub_rn(__fmul_rn(inv_scale, __fadd_rn((float)n, 0.5f)), 0.5f);
  if (src < 0.f) src = 0.f;
  int i0 = (int)src;
  if (i0 > T - 1) i0 = T - 1;
  const int i1 = i0 + (i0 < T - 1 ? 1 : 0);
  const float l1 = __fsub_rn(src, (float)i0), l0 = __fsub_rn(1.0f, l1);
  const float fv = f0[fo + n / up];
  const float uv = fv > thr ? 1.0f : 0.0f;
  const float namp = __fadd_rn(__fmul_rn(uv, noise_std), __fmul_rn(__fsub_rn(1.0f, uv), unv));
  float acc = 0.f;
  for (int h = 0; h < harm; ++h) {
    // torch's CPU kernel rounds l1 * p1 and fuses l0 * p0 into the sum
    const float p = fmaf(l0, phase[(size_t)(fo + i0) * harm + h], __fmul_rn(l1, phase[(size_t)(fo + i1) * harm + h]));
    float sine = __fmul_rn(sinf(p), amp);
    sine = __fadd_rn(__fmul_rn(sine, uv), __fmul_rn(namp, noise[so * harm + h]));
    acc = fmaf(sine, lw[h], acc);
  }
  out[so] = tanhf(__fadd_rn(acc, lb[0]));
}

// STFT of the source (n_fft 16, hop 4, centred, reflect padding, periodic Hann window): frame f of item i ->
// [re_0..re_8 | im_0..im_8 | 14 zeros] (STFT_LD floats, written as 16-byte stores)
__global__ void stft_kernel(const float* s, const int* smp_off, const int* smp_len, const int* fr_off, const int* fr_len,
                            const float* win, float* out) {
  const int it = blockIdx.y;
  const int f = blockIdx.x * blockDim.x + threadIdx.x;
  const int F = fr_len[it];
  if (f >= F) return;
  const int n = smp_len[it];
  const float* x = s + smp_off[it];
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    int p = f * 4 + k - 8;
    if (p < 0) p = -p;
    if (p >= n) p = 2 * (n - 1) - p;
    v[k] = __fmul_rn(x[p], win[k]);
  }
  float o[STFT_LD];
#pragma unroll
  for (int b = 0; b < 9; ++b) {
    float re = 0.f, im = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      re = fmaf(v[k], kCos16[(b * k) & 15], re);
      im = fmaf(-v[k], kSin16[(b * k) & 15], im);
    }
    o[b] = re;
    o[9 + b] = im;
  }
#pragma unroll
  for (int b = 18; b < STFT_LD; ++b) o[b] = 0.f;
  float4* dst = (float4*)(out + (size_t)(fr_off[it] + f) * STFT_LD);
#pragma unroll
  for (int q = 0; q < STFT_LD / 4; ++q) dst[q] = make_float4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
}

// ISTFT (``istft_overlap_add``): mag = min(exp(x_re), 100), phase = sin(x_im), spectrum mag (cos phase, sin phase);
// inverse real FFT of each frame, windowed, overlap-added, divided by the summed squared window; n_fft / 2 trimmed at
// both ends; clamped to +-limit.  A block takes IST_F consecutive frames: each thread computes one frame's 16 inverse-FFT
// values once (into LDS), then the block writes the 4 (IST_F - 3) samples those frames cover completely, each the sum
// over its <= 4 frames in frame order.
constexpr int IST_F = 256;
__global__ void __launch_bounds__(256) istft_kernel(const float* x, const int* fr_off, const int* fr_len, const int* smp_off, const float* win,
                                                    float limit, float* out) {
  __shared__ float ys[IST_F * 17];  // frame t of the block, value i at t * 17 + i (already times 1 / 16)
  const int it = blockIdx.y;
  const int F = fr_len[it];
  const int B0 = blockIdx.x * (IST_F - 3);
  if (B0 >= F) return;
  const int t = threadIdx.x;
  if (B0 + t < F) {
    const float* xf = x + (size_t)(fr_off[it] + B0 + t) * 18;
    float re[9], im[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      const float mag = fminf(expf(xf[k]), 100.0f);
      const float ph = sinf(xf[9 + k]);
      re[k] = __fmul_rn(mag, cosf(ph));
      im[k] = __fmul_rn(mag, sinf(ph));
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      // irfft at index i: (1/16) [X0 + (-1)^i X8 + 2 sum_{k=1..7} (Re X_k cos(2 pi k i / 16) - Im X_k sin(2 pi k i / 16))]
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const float c = kCos16[(k * i) & 15], s = kSin16[(k * i) & 15];
        // the imaginary parts of DC and Nyquist are ignored
        acc += (k == 0 || k == 8) ? re[k] * c : 2.0f * (re[k] * c - im[k] * s);
      }
      ys[t * 17 + i] = acc * (1.0f / 16.0f);
    }
  }
  __syncthreads();
  // padded sample p (output n = p - 8) sees frames ceil((p - 15) / 4) .. p / 4; this block's frames cover
  // p in [4 B0 + 12, 4 (B0 + IST_F - 3) + 12) (block 0 from p = 8), and outputs end at p = 4 F + 4
  const int p_lo = B0 == 0 ? 8 : 4 * B0 + 12;
  const int p_hi = min(4 * (B0 + IST_F - 3) + 12, 4 * F + 4);
  for (int p = p_lo + t; p < p_hi; p += blockDim.x) {
    int fa = (p - 15 + 3) / 4;
    if (p - 15 < 0) fa = 0;
    int fb = p / 4;
    if (fb > F - 1) fb = F - 1;
    float y = 0.f, env = 0.f;
    for (int f = fa; f <= fb; ++f) {
      const int i = p - 4 * f;
      const float w = win[i];
      y = fmaf(ys[(f - B0) * 17 + i], w, y);
      env = fmaf(w, w, env);
    }
    float v = y / env;
    v = fminf(fmaxf(v, -limit), limit);
    out[smp_off[it] + p - 8] = v;
  }
}

// y = Snake(x) for a packed [rows, C] buffer, four channels per thread (the same per-element function the convs
// apply on load, so a conv reading y with no pre-activation sees the values it would have computed)
__global__ void __launch_bounds__(256) snake_kernel(const float4* x, int C4, long n4, const float* alpha, const float* inv, float4* y) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256) {
    const int c = (int)(i % C4) * 4;
    const float4 v = x[i];
    y[i] = make_float4(pre_act(v.x, PRE_SNAKE, 0.f, alpha[c], inv[c]), pre_act(v.y, PRE_SNAKE, 0.f, alpha[c + 1], inv[c + 1]),
                       pre_act(v.z, PRE_SNAKE, 0.f, alpha[c + 2], inv[c + 2]), pre_act(v.w, PRE_SNAKE, 0.f, alpha[c + 3], inv[c + 3]));
  }
}

// rows 1.. of each item's ups output were written one row down; row 0 = input row 1 (ReflectionPad1d((1, 0)))
__global__ void reflect_kernel(float* x, int C, const int* off, int n_items) {
  const int it = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C || it >= n_items) return;
  float* b = x + (size_t)off[it] * C;
  b[c] = b[2 * C + c];
}

inline unsigned cdiv(long long a, long long b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

hipError_t snake_rows(const float* x, int C, long rows, const float* alpha, const float* inv, float* y, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (C % 4 || x == y || ((size_t)x & 15) || ((size_t)y & 15)) return hipErrorInvalidValue;
  const long n4 = rows * (C / 4);
  const int grid = (int)std::min<long>((n4 + 255) / 256, 8192);
  hipLaunchKernelGGL(snake_kernel, dim3(grid), dim3(256), 0, st, (const float4*)x, C / 4, n4, alpha, inv, (float4*)y);
  return hipGetLastError();
}

hipError_t conv_f32(const ConvDesc& c, int max_rows, hipStream_t st) {
  if (c.n_items <= 0 || max_rows <= 0) return hipSuccess;
  if (c.n_phase < 1 || c.n_phase > 8) return hipErrorInvalidValue;
  // grids that would keep fewer than half the CUs busy: 32-row tiles with the taps and channels split over the waves
  const long tiles = (long)cdiv(max_rows, 64) * cdiv(c.Cout, 64) * c.n_items * c.n_phase;
  if (tiles < 128) {
    // 32 output channels per workgroup while that grid fits the chip in one round (half the weight bytes each), else 64
    const long t32 = (long)cdiv(max_rows, 32) * cdiv(c.Cout, 32) * c.n_items * c.n_phase;
    if (t32 <= 256) {
      dim3 grid(cdiv(max_rows, 32), cdiv(c.Cout, 32), c.n_items * c.n_phase);
      hipLaunchKernelGGL(conv_f32_split_kernel<1>, grid, dim3(64 * CS_WAVES), 0, st, c);
    } else {
      dim3 grid(cdiv(max_rows, 32), cdiv(c.Cout, 64), c.n_items * c.n_phase);
      hipLaunchKernelGGL(conv_f32_split_kernel<2>, grid, dim3(64 * CS_WAVES), 0, st, c);
    }
    return hipGetLastError();
  }
  // 64 output channels per workgroup, 32 where the output has no more (conv_post's 18)
  // undilated convs whose Cin is not a multiple of 32 take their K flat
  const bool flat = c.d_in == 1 && c.Cin % F_BK != 0;
  // the DMA-staged kernel: 32-channel K stages and 16-byte rows (activations and weights)
  if (c.Cin % 32 == 0 && c.ldx % 4 == 0 && ((size_t)c.x & 15) == 0 && ((size_t)c.w & 15) == 0 &&
      (c.pre == PRE_NONE || c.pre == PRE_LEAKY)) {
    const int wn = c.Cout <= 32 ? 1 : 2;
    dim3 grid(cdiv(max_rows, F_BM), cdiv(c.Cout, 32 * wn), c.n_items * c.n_phase);
#define T2W_FD(W, P) hipLaunchKernelGGL((conv_f32_dma_kernel<W, P>), grid, dim3(256), 0, st, c)
    if (wn == 1) {
      if (c.pre == PRE_NONE) T2W_FD(1, PRE_NONE);
      else T2W_FD(1, PRE_LEAKY);
    } else {
      if (c.pre == PRE_NONE) T2W_FD(2, PRE_NONE);
      else T2W_FD(2, PRE_LEAKY);
    }
#undef T2W_FD
    return hipGetLastError();
  }
  if (c.Cout <= 32) {
    dim3 grid(cdiv(max_rows, F_BM), 1, c.n_items * c.n_phase);
    if (flat) hipLaunchKernelGGL((conv_f32_kernel<1, true>), grid, dim3(256), 0, st, c);
    else hipLaunchKernelGGL((conv_f32_kernel<1, false>), grid, dim3(256), 0, st, c);
  } else {
    dim3 grid(cdiv(max_rows, F_BM), cdiv(c.Cout, 64), c.n_items * c.n_phase);
    if (flat) hipLaunchKernelGGL((conv_f32_kernel<2, true>), grid, dim3(256), 0, st, c);
    else hipLaunchKernelGGL((conv_f32_kernel<2, false>), grid, dim3(256), 0, st, c);
  }
  return hipGetLastError();
}

// LDS of a BM-row tile: the slab, and at least the epilogue's 32-row x 64-channel fp32 block per wave
size_t conv_bf16_lds(int BM) {
  const size_t slab = (size_t)(BM + HB_MAXSPAN) * 8 * sizeof(uint4), epi = 4 * 32 * 16 * sizeof(float4);
  return slab > epi ? slab : epi;
}

hipError_t conv_bf16(const ConvDesc& c, const bf16_t* wbf, int max_rows, hipStream_t st) {
  if (c.n_items <= 0 || max_rows <= 0) return hipSuccess;
  if (c.epi == EPI_SNAKE) return hipErrorInvalidValue;  // fp32 convs only
  if (c.n_phase < 1 || c.n_phase > 8 || c.s_in != 1 || c.ldx % 4 || c.ldy % 4) return hipErrorInvalidValue;
  const int span = (c.taps - 1) * (c.d_in < 0 ? -c.d_in : c.d_in);
  if (span > HB_MAXSPAN) return hipErrorInvalidValue;
  // 512-row tiles when there are enough of them for the chip, 128 when those fill at least half of it, else 32-row
  // tiles with the taps split over the waves
  const long tiles512 = (long)cdiv(max_rows, 512) * cdiv(c.Cout, HB_BN) * c.n_items * c.n_phase;
  const long tiles128 = (long)cdiv(max_rows, 128) * cdiv(c.Cout, HB_BN) * c.n_items * c.n_phase;
  if (tiles128 < 128) {
    // 32 output channels per workgroup while that grid fits the chip in one round, else 64
    const long t32 = (long)cdiv(max_rows, 32) * cdiv(c.Cout, 32) * c.n_items * c.n_phase;
    if (t32 <= 256) {
      dim3 grid(cdiv(max_rows, 32), cdiv(c.Cout, 32), c.n_items * c.n_phase);
      hipLaunchKernelGGL(conv_bf16_split_kernel<1>, grid, dim3(64 * CS_WAVES), 0, st, c, wbf);
    } else {
      dim3 grid(cdiv(max_rows, 32), cdiv(c.Cout, 64), c.n_items * c.n_phase);
      hipLaunchKernelGGL(conv_bf16_split_kernel<2>, grid, dim3(64 * CS_WAVES), 0, st, c, wbf);
    }
  } else if (!c.wfr) {
    return hipErrorInvalidValue;  // the slab tiles read the fragment-ordered copy
  } else if (tiles512 >= 256) {
    constexpr int BM = 512;
    const size_t lds = conv_bf16_lds(BM);
    static const hipError_t attr =  // once per process (thread-safe initialisation)
        hipFuncSetAttribute((const void*)conv_bf16_kernel<BM>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    dim3 grid(cdiv(max_rows, BM), cdiv(c.Cout, HB_BN), c.n_items * c.n_phase);
    hipLaunchKernelGGL(conv_bf16_kernel<BM>, grid, dim3(256), lds, st, c, wbf);
  } else {
    constexpr int BM = 128;
    const size_t lds = conv_bf16_lds(BM);
    dim3 grid(cdiv(max_rows, BM), cdiv(c.Cout, HB_BN), c.n_items * c.n_phase);
    hipLaunchKernelGGL(conv_bf16_kernel<BM>, grid, dim3(256), lds, st, c, wbf);
  }
  return hipGetLastError();
}

namespace {
// one thread per 16-byte unit of the fragment-ordered copy (layout in hift_internal.h)
__global__ void weight_fragments_kernel(const uint4* __restrict__ w, uint4* __restrict__ f, int taps, int nib, long n16) {
  const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
  if (i >= n16) return;
  const int lane = (int)(i & 63);
  long blk = i >> 6;  // ((row block) * taps + j) * nib + ib
  const int ib = (int)(blk % nib);
  blk /= nib;
  const int j = (int)(blk % taps);
  const long row = (blk / taps) * 32 + (lane & 31);  // ph * (Cout padded) + output channel
  f[i] = w[((row * taps + j) * nib * 16 + ib * 16 + (lane >> 5) * 8) >> 3];
}
}  // namespace

hipError_t conv_weight_fragments(const uint16_t* wbf, uint16_t* out, int n_phase, int Cout, int taps, int Cin, hipStream_t st) {
  if (!wbf || !out || n_phase < 1 || Cout < 1 || taps < 1 || Cin < 1) return hipErrorInvalidValue;
  const long co_pad = (Cout + 63) & ~63, ci_pad = (Cin + 63) & ~63;
  const long n16 = (long)n_phase * co_pad * taps * ci_pad / 8;
  hipLaunchKernelGGL(weight_fragments_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st, (const uint4*)wbf, (uint4*)out, taps,
                     (int)(ci_pad / 16), n16);
  return hipGetLastError();
}

namespace {
size_t resblock_pair_lds(int C) {
  const int BM1 = 32768 / C;
  const size_t s1 = (size_t)(BM1 + RP_SPAN) * 8 * sizeof(uint4), s2 = (size_t)(BM1 + 16) * C * sizeof(bf16_t);
  const size_t epi = 4 * 32 * 16 * sizeof(float4);
  return std::max(std::max(s1, s2), epi);
}

template <int C>
hipError_t launch_pair(const ConvDesc& c1, const ConvDesc& c2, int max_rows, hipStream_t st) {
  const size_t lds = resblock_pair_lds(C);
  static const hipError_t attr =  // once per process (thread-safe initialisation)
      hipFuncSetAttribute((const void*)resblock_pair_kernel<C>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  dim3 grid(cdiv(max_rows, resblock_pair_rows(C, c1.taps)), c1.n_items);
  hipLaunchKernelGGL(resblock_pair_kernel<C>, grid, dim3(256), lds, st, c1, c2);
  return hipGetLastError();
}
}  // namespace

int resblock_pair_rows(int C, int k) { return 32768 / C - (k - 1); }

bool resblock_pair_fits(int C, int k, int dil) {
  return (C == 64 || C == 128 || C == 256) && k >= 1 && (k & 1) && dil >= 1 && (k - 1) * dil <= RP_SPAN;
}

hipError_t resblock_pair_bf16(const ConvDesc& c1, const ConvDesc& c2, int max_rows, hipStream_t st) {
  if (c1.n_items <= 0 || max_rows <= 0) return hipSuccess;
  if (c2.epi == EPI_SNAKE) return hipErrorInvalidValue;  // fp32 convs only
  const int C = c1.Cin, k = c1.taps;
  const bool same = c1.Cout == C && c2.Cin == C && c2.Cout == C && c2.taps == k && c1.ldx == C && c1.ldy == C && c2.ldx == C &&
                    c2.ldy == C && c1.n_items == c2.n_items && c1.in_off == c2.out_off && c1.in_len == c2.out_len;
  const bool geom = c1.s_in == 1 && c2.s_in == 1 && c1.s_out == 1 && c2.s_out == 1 && c1.n_phase == 1 && c2.n_phase == 1 &&
                    c2.d_in == 1 && c1.off_in[0] == -c1.d_in * ((k - 1) / 2) && c2.off_in[0] == -((k - 1) / 2) &&
                    c1.off_out[0] == 0 && c2.off_out[0] == 0;
  const bool acts = c1.pre == PRE_SNAKE && c2.pre == PRE_SNAKE && c1.epi == EPI_STORE && c2.res == c1.x &&
                    (c2.epi == EPI_RES || c2.epi == EPI_ADD_RES || c2.epi == EPI_RES_MEAN);
  if (!same || !geom || !acts || !resblock_pair_fits(C, k, c1.d_in) || !c1.wfr || !c2.wfr) return hipErrorInvalidValue;
  if (c2.y == c1.x || (c2.epi == EPI_RES_MEAN && c2.sum == c1.x)) return hipErrorInvalidValue;  // halo rows of x are read by other workgroups
  if (C == 64) return launch_pair<64>(c1, c2, max_rows, st);
  if (C == 128) return launch_pair<128>(c1, c2, max_rows, st);
  return launch_pair<256>(c1, c2, max_rows, st);
}

hipError_t f0_head(const float* x, int C, const float* w, const float* b, float* f0, int rows, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(f0_head_kernel, dim3(cdiv(rows, 4)), dim3(256), 0, st, x, C, w, b, f0, rows);
  return hipGetLastError();
}

hipError_t nsf_phase(const float* f0, const int* fr_off, const int* fr_len, int n_items, int harm, float sr, float scale, float* phase,
                     hipStream_t st) {
  hipLaunchKernelGGL(phase_kernel, dim3(cdiv(n_items * harm, 4)), dim3(256), 0, st, f0, fr_off, fr_len, n_items, harm, sr, scale, phase);
  return hipGetLastError();
}

hipError_t nsf_source(const float* phase, const float* f0, const int* fr_off, const int* fr_len, const int* smp_off, int n_items,
                      int max_frames, int harm, float inv_scale, int up, float amp, float noise_std, float unv, float thr,
                      const float* noise, const float* lw, const float* lb, const float* cache, int S, float* out, hipStream_t st) {
  dim3 grid(cdiv((long long)max_frames * up, 256), n_items);
  hipLaunchKernelGGL(source_kernel, grid, dim3(256), 0, st, phase, f0, fr_off, fr_len, smp_off, n_items, harm, inv_scale, up, amp, noise_std,
                     unv, thr, noise, lw, lb, cache, S, out);
  return hipGetLastError();
}

hipError_t stft16(const float* s, const int* smp_off, const int* smp_len, const int* fr_off, const int* fr_len, int n_items, int max_fr,
                  const float* win, float* out, hipStream_t st) {
  hipLaunchKernelGGL(stft_kernel, dim3(cdiv(max_fr, 128), n_items), dim3(128), 0, st, s, smp_off, smp_len, fr_off, fr_len, win, out);
  return hipGetLastError();
}

hipError_t istft16(const float* x, const int* fr_off, const int* fr_len, const int* smp_off, int n_items, int max_smp, const float* win,
                   float limit, float* out, hipStream_t st) {
  const int max_fr = max_smp / 4 + 1;  // an item of F frames has (F - 1) 4 samples
  hipLaunchKernelGGL(istft_kernel, dim3(cdiv(max_fr, IST_F - 3), n_items), dim3(256), 0, st, x, fr_off, fr_len, smp_off, win, limit, out);
  return hipGetLastError();
}

hipError_t reflect_rows(float* x, int C, const int* off, int n_items, hipStream_t st) {
  hipLaunchKernelGGL(reflect_kernel, dim3(cdiv(C, 256), n_items), dim3(256), 0, st, x, C, off, n_items);
  return hipGetLastError();
}

}  // namespace t2w
