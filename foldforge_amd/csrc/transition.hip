// Fused pair transition on gfx950: x + squeeze(silu(expand_a(LN(x))) * expand_b(LN(x))).
//
// Equations: src/foldforge/models/checkpoints/legacy/reference/transition.py:40-41 and
// src/foldforge/modules/dense/diffusion_transformer.py:36-44 (SwiGLU). One workgroup owns
// 64 rows: the LayerNorm'd rows stay in LDS, the 4c-wide hidden layer is produced 64
// channels at a time (MFMA), gated, parked in LDS as bf16 and immediately contracted
// into the 64 x 128 output accumulator, so the hidden activations never reach HBM:
// the kernel reads x once and writes the output once.
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kTrTM = 64;           // rows per workgroup
constexpr int kTrHC = 64;           // hidden channels per step
constexpr int kTrHS = kTrHC + 8;    // LDS row stride of the hidden chunk

// grid ceil(rows / 64); block 256 = 2 (row tiles) x 2 waves.
__global__ __launch_bounds__(256) void transition_128x4(
    const bf16* __restrict__ x, const float* __restrict__ ln_w, const float* __restrict__ ln_b,
    const bf16* __restrict__ wa, const bf16* __restrict__ wb, const bf16* __restrict__ ws,
    bf16* __restrict__ out, int64_t rows, int residual, float eps) {
  constexpr int C = 128, HID = 512;
  __shared__ __attribute__((aligned(16))) bf16 zr[kTrTM * kRow];
  __shared__ __attribute__((aligned(16))) bf16 xh[kTrTM * kRow];
  __shared__ __attribute__((aligned(16))) bf16 hb[kTrTM * kTrHS];
  const int64_t row0 = (int64_t)blockIdx.x * kTrTM;
  const int valid = (int)min<int64_t>(kTrTM, rows - row0);
  const int tid = threadIdx.x;
  ln_tile_128<kTrTM>(x + row0 * C, C, valid, ln_w, ln_b, eps, xh, zr);
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int rt = wave >> 1;  // row tile (32 rows) of this wave
  const int hw = wave & 1;   // hidden tile (32 of the 64 chunk channels) / output half
  const bf16* xrow = xh + (rt * 32 + li) * kRow;
  f32x16 acc[2] = {zero16(), zero16()};  // output channels 64*hw + 32*t + li
#pragma unroll 1
  for (int h0 = 0; h0 < HID; h0 += kTrHC) {
    const int hc = h0 + 32 * hw + li;  // hidden channel of this lane (B column)
    f32x16 aa = zero16(), ab = zero16();
    mma_rows<128>(xrow, wa + (int64_t)hc * C, g, aa);
    mma_rows<128>(xrow, wb + (int64_t)hc * C, g, ab);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int p = rt * 32 + acc_row(q, g);
      hb[p * kTrHS + 32 * hw + li] = (bf16)(siluf_(aa[q]) * ab[q]);
    }
    __syncthreads();
    const bf16* hrow = hb + (rt * 32 + li) * kTrHS;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c = 64 * hw + 32 * t + li;
      mma_rows<kTrHC>(hrow, ws + (int64_t)c * HID + h0, g, acc[t]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int c = 64 * hw + 32 * t + li;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int p = rt * 32 + acc_row(q, g);
      if (p < valid) {
        float v = acc[t][q];
        if (residual) v += (float)zr[p * kRow + c];
        out[(row0 + p) * C + c] = (bf16)v;
      }
    }
  }
}

void launch_transition(const TransitionArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.rows + kTrTM - 1) / kTrTM;
  transition_128x4<<<dim3((unsigned)blocks), 256, 0, stream>>>(a.x, a.ln_w, a.ln_b, a.wa, a.wb,
                                                               a.ws, a.out, a.rows, a.residual,
                                                               a.eps);
}

}  // namespace ffk
