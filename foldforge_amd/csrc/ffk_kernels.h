// Host-side launch interfaces of the pair-stack kernels (one struct per op, filled by
// the C-ABI layer in api.hip after it has validated shapes and carved the workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ffk_device.h"

namespace ffk {

struct TrimulArgs {
  const bf16* z;
  const uint8_t* mask;
  const float *ln_w, *ln_b, *lno_w, *lno_b;
  const bf16* wp;  // [4h][c]: left, left_gate, right, right_gate
  const bf16* wg;  // [c][c]
  const bf16* wo;  // [c][h]
  bf16 *A, *B, *P;  // [batch][h][np][np]
  float* maskf;     // [batch][np] scratch: the key mask as 1 / 0, zero past n
  bf16* out;
  int batch, n, np, outgoing, residual;
  float eps;
};
void launch_trimul(const TrimulArgs& a, hipStream_t stream);

struct TriattnArgs {
  const bf16* z;
  const uint8_t* mask;
  const float *ln_w, *ln_b;
  const bf16* wqkv;  // [3 * 128][128], query rows carry d^-1/2 * log2(e)
  const bf16* wb;    // [32][128], rows < heads carry log2(e) * to_bias, others zero
  const bf16* wg;    // [128][128] to_gate
  const bf16* wo;    // [128][128] to_out
  bf16 *q, *k, *vt;  // [batch * heads][np][np][32], vt: [batch * heads][np][32][np]
  float* bias;       // [batch * heads][np / 32][np / 32][2][32][16] blocked, see triattn.hip
  bf16* o;           // [batch][n][n][128] z-frame attention output
  bf16* out;
  int batch, n, np, heads, starting, transposed_bias, residual;
  float eps;
};
void launch_triattn(const TriattnArgs& a, hipStream_t stream);

struct FlashArgs {
  const bf16 *q, *k, *vt;
  const float* bias;  // blocked pair bias (log2 units, -inf at masked keys)
  bf16* o;
  int64_t batch, rows, np, rows_valid, n_valid, o_sb, o_sr, o_sj;
  int heads;
};
void launch_flash(const FlashArgs& a, hipStream_t stream);

struct TransitionArgs {
  const bf16* x;
  const float *ln_w, *ln_b;
  const bf16* w;  // expand_a, expand_b, squeeze as written by launch_transition_pack
  bf16* out;
  int64_t rows;
  int residual;
  float eps;
};
// expand_a [4c][c], expand_b [4c][c], squeeze [c][4c] (fp32) -> the transition kernel's packed
// bf16 weight stream (3 * 4c * c elements).
void launch_transition_pack(const float* wa, const float* wb, const float* ws, bf16* dst,
                            hipStream_t stream);
void launch_transition(const TransitionArgs& a, hipStream_t stream);

struct PackSeg {
  const float* src;  // NULL: write zeros
  bf16* dst;
  int64_t n;
  float scale;
  int swap23;        // 1: dst[i] = src[i with index bits 2 and 3 exchanged]
};
struct PackJob {
  PackSeg seg[8];
  int nseg;
};
void launch_pack(const PackJob& job, hipStream_t stream);

// Compute units of the current device (cached per device).
int cu_count();

void launch_layer_norm(const void* x, const float* w, const float* b, void* y, int64_t rows,
                       int cols, float eps, int dtype, hipStream_t stream);

}  // namespace ffk
