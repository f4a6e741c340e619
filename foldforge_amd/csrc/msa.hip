// MSA pair-weighted averaging on gfx950 (the MSA stack's pair-to-MSA update).
//
// Equations: src/foldforge/models/checkpoints/legacy/attention.py:203-223 (MSAAttention):
//   x = LN_msa(m); w[h, i, :] = softmax_j(LN_pair(z)[i, j] . W_b[h]) over valid keys j;
//   o[s, i, h] = sum_j w[h, i, j] v[s, j, h], v = x W_v^T; out = m + (sigmoid(x W_g^T) o) W_out^T.
// The weights do not depend on the MSA row s, so per head the average is one GEMM
//   O_h[(s, c)][i] = sum_j v^T_h[(s, c)][j] w_h[i][j]
// with all S MSA rows stacked along M. The C-ABI (api.hip) runs:
//   row_gemm<kEpiPwa, kXLn> (single.hip): LN_msa + value / gate projections -> v^T, gate
//   apb_pair_bias (single.hip): pair logits in log2 units, masked keys very negative
//   pwa_softmax: the softmax of every (batch, head, query) row -> bf16 weights
//   pwa_average: the per-head GEMM, gated -> fp32 (gate * o)
//   row_gemm<kEpiResid, kXF32>: the output projection and the residual.
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

namespace {

// A row whose largest logit is below this has no valid key: its weights are all zero.
constexpr float kNoKey = -1e29f;

// One wave per row of np logits: maximum, exp2 sum, then the normalised bf16 weights.
__global__ __launch_bounds__(256) void pwa_softmax(PwaSoftmaxArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= a.rows) return;
  const float* x = a.logits + row * a.np;
  bf16* w = a.w + row * a.np;
  float mx = -INFINITY;
  for (int j = 4 * lane; j < a.np; j += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(x + j);
    mx = fmaxf(fmaxf(mx, fmaxf(v[0], v[1])), fmaxf(v[2], v[3]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = 0.f;
  for (int j = 4 * lane; j < a.np; j += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(x + j);
#pragma unroll
    for (int e = 0; e < 4; ++e) sum += fast_exp2(v[e] - mx);
  }
  sum = wave_sum(sum);
  const float inv = mx > kNoKey ? 1.f / sum : 0.f;
  for (int j = 4 * lane; j < a.np; j += 256) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(x + j);
    bf16x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (bf16)(fast_exp2(v[e] - mx) * inv);
    *reinterpret_cast<bf16x4*>(w + j) = o;
  }
}

// grid (ceil(S dh / 128), ceil(n / 64), batch * heads); block 256: wave w computes rows
// 32 w .. 32 w + 31 of the workgroup's 128 (s, c) rows for its 64 queries (two 32 x 32 MFMA
// tiles sharing the A operand). A = v^T rows, B = weight rows, both key-contiguous; keys are
// consumed in groups of 64, lane half g taking keys 64 kg + 32 g + 8 t .. + 7 for step t.
// Epilogue: lane (li, g) holds query q0 + li (or + 32) and rows r = r0 + 8 v + 4 g + e, i.e.
// (s, c) = (r / dh, r % dh): four consecutive channels of one MSA row.
__global__ __launch_bounds__(256) void pwa_average(PwaAverageArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 31, g = lane >> 5;
  const int64_t bh = blockIdx.z;
  const int64_t b = bh / a.heads;
  const int h = (int)(bh - b * a.heads);
  const int rows = a.depth * a.dh, n = a.n, np = a.np;
  const int r0 = blockIdx.x * 128 + 32 * wave;
  if (r0 >= rows) return;  // no barrier in this kernel
  const int q0 = blockIdx.y * 64;
  const bf16* arow = a.vt + (bh * rows + min(r0 + li, rows - 1)) * np + 32 * g;
  const bf16* b0row = a.w + (bh * n + min(q0 + li, n - 1)) * np + 32 * g;
  const bf16* b1row = a.w + (bh * n + min(q0 + 32 + li, n - 1)) * np + 32 * g;
  f32x16 acc0 = zero16(), acc1 = zero16();
  for (int k0 = 0; k0 < np; k0 += 64) {
    bf16x8 af[4], bf0[4], bf1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      af[t] = ld8(arow + k0 + 8 * t);
      bf0[t] = ld8(b0row + k0 + 8 * t);
      bf1[t] = ld8(b1row + k0 + 8 * t);
    }
    if (k0 + 64 > n) {  // keys past n: their v^T entries were never written
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (k0 + 32 * g + 8 * t + e >= n) af[t][e] = (bf16)0.f;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc0 = mfma32(af[t], bf0[t], acc0);
      acc1 = mfma32(af[t], bf1[t], acc1);
    }
  }
  const int hd = a.heads * a.dh;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const f32x16& acc = half == 0 ? acc0 : acc1;
    const int q = q0 + 32 * half + li;
    if (q >= n) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = r0 + 8 * v + 4 * g;
      if (r >= rows) continue;
      const int s = r / a.dh, c = r - s * a.dh;
      const int64_t off = ((b * a.depth + s) * n + q) * hd + h * a.dh + c;
      const bf16x4 gv = *reinterpret_cast<const bf16x4*>(a.gate + off);
      f32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = acc[4 * v + e] * (float)gv[e];
      *reinterpret_cast<f32x4*>(a.og + off) = y;
    }
  }
}

}  // namespace

void launch_pwa_softmax(const PwaSoftmaxArgs& a, hipStream_t stream) {
  pwa_softmax<<<dim3((unsigned)((a.rows + 3) / 4)), 256, 0, stream>>>(a);
}

void launch_pwa_average(const PwaAverageArgs& a, hipStream_t stream) {
  const int rows = a.depth * a.dh;
  pwa_average<<<dim3((unsigned)((rows + 127) / 128), (unsigned)((a.n + 63) / 64),
                     (unsigned)(a.batch * a.heads)),
                256, 0, stream>>>(a);
}

}  // namespace ffk
