// Internal launch interfaces of the HiFT kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace t2w {

enum PreAct { PRE_NONE = 0, PRE_LEAKY = 1, PRE_SNAKE = 2 };
// EPI_SNAKE: y = Snake(conv + bias) with the descriptor's alpha / inv (the next conv's pre-activation, applied once)
enum ConvEpi { EPI_STORE = 0, EPI_ELU = 1, EPI_RES = 2, EPI_ADD_RES = 3, EPI_RES_MEAN = 4, EPI_SNAKE = 5 };

// y[out_off[b] + r * s_out + off_out[ph], co] = epi(bias[co] + sum_{j, ci} w[ph, co, j, ci] act(x[in_off[b] + r * s_in +
// j * d_in + off_in[ph], ci])), inputs outside [0, in_len[b]) read as zero.
struct ConvDesc {
  const float* x; int ldx;
  const int* in_off; const int* in_len;
  float* y; int ldy;
  const int* out_off; const int* out_len;
  const float* w; const float* bias;  // w [n_phase, Cout, taps, Cin]
  const uint16_t* wbf;                // bf16 weights for conv_bf16 (or null)
  const uint16_t* wfr;                // the same weights in MFMA fragment order (conv_weight_fragments); the tile kernels read these
  int Cin, Cout, taps;
  int s_in, d_in, s_out;
  int n_phase;
  int off_in[8], off_out[8];
  int pre; float slope; const float* alpha; const float* inv;
  int epi; const float* res; float* sum; int sum_mode; int sum_div;
  int n_items;
};

hipError_t conv_f32(const ConvDesc& c, int max_rows, hipStream_t st);
// stride-1 / polyphase convs on bf16 MFMA; wbf: bf16 weights [n_phase, Cout padded to 64, taps, Cin padded to 64], and
// c.wfr the same weights in fragment order (the slab-tile kernels need it)
hipError_t conv_bf16(const ConvDesc& c, const uint16_t* wbf, int max_rows, hipStream_t st);
// wbf [n_phase, Cout padded to 64, taps, Cin padded to 64] -> out (same size) in MFMA fragment order: for phase ph, output
// block cb of 32 channels, tap j and input block ib of 16 channels, one 1 KB block whose lane l holds the 8 weights of
// output channel cb * 32 + l % 32, input channels ib * 16 + (l / 32) * 8 .. + 7 (the A operand of a 32x32x16 MFMA)
hipError_t conv_weight_fragments(const uint16_t* wbf, uint16_t* out, int n_phase, int Cout, int taps, int Cin, hipStream_t st);
// One ResBlock dilation (conv c1 with Snake, conv c2 with Snake and the residual c1.x) in one kernel on bf16 MFMA,
// conv1's output kept in LDS.  c2 writes y (EPI_RES / EPI_ADD_RES) or the running mean (EPI_RES_MEAN); y must not be x.
bool resblock_pair_fits(int C, int k, int dil);
int resblock_pair_rows(int C, int k);  // output rows per workgroup
hipError_t resblock_pair_bf16(const ConvDesc& c1, const ConvDesc& c2, int max_rows, hipStream_t st);
hipError_t f0_head(const float* x, int C, const float* w, const float* b, float* f0, int rows, hipStream_t st);
hipError_t nsf_phase(const float* f0, const int* fr_off, const int* fr_len, int n_items, int harm, float sr, float scale, float* phase,
                     hipStream_t st);
hipError_t nsf_source(const float* phase, const float* f0, const int* fr_off, const int* fr_len, const int* smp_off, int n_items,
                      int max_frames, int harm, float inv_scale, int up, float amp, float noise_std, float unvoiced_amp, float thr,
                      const float* noise, const float* lw, const float* lb, const float* cache, int S, float* out, hipStream_t st);
// STFT frames are rows of STFT_LD floats: the 9 real parts, the 9 imaginary parts, then zeros, so that the source
// downsampling convs read 16-byte-aligned rows of 32 channels (their weights padded alike) on the DMA-staged kernel
constexpr int STFT_LD = 32;
hipError_t stft16(const float* s, const int* smp_off, const int* smp_len, const int* fr_off, const int* fr_len, int n_items, int max_fr,
                  const float* win, float* out, hipStream_t st);
hipError_t istft16(const float* x, const int* fr_off, const int* fr_len, const int* smp_off, int n_items, int max_smp, const float* win,
                   float limit, float* out, hipStream_t st);
hipError_t reflect_rows(float* x, int C, const int* off, int n_items, hipStream_t st);
// y = Snake(x) element by element over `rows` packed rows of C channels (C % 4 == 0), y != x
hipError_t snake_rows(const float* x, int C, long rows, const float* alpha, const float* inv, float* y, hipStream_t st);

int set_error(const char* what, hipError_t e);  // records the message for t2w_last_error(); returns 1

}  // namespace t2w
