// Triangle attention around the starting / ending node on gfx950.
//
// Equations: src/foldforge/models/checkpoints/legacy/attention.py:108-163 with the masked
// softmax of legacy/reference/attention.py:77-100. Three kernels per call:
//   1. triattn_project  z -> LN_pair -> q (scaled by d^-1/2 log2 e), k, v^T and the pair
//                       bias (log2 e scaled, fp16, -inf at masked keys). A tile is 128
//                       positions along one attention row: a row of z (starting) or a
//                       column of z (ending), so every store is contiguous.
//   2. flash_attn_bias  per (row, head, 128 queries): S^T = bias^T + K Q^T on MFMA (the
//                       bias tile is the accumulator's initial value), online softmax in
//                       fp32 with exp2, O^T += V^T P^T on MFMA. The N^3 H logits never
//                       leave registers.
//   3. triattn_output   out = z + (sigmoid(LN_pair(z) W_g^T) * o) W_out^T.
// The gate is recomputed from z in kernel 3 rather than stored (z is read there for the
// residual anyway).
//
// Flash layout (one wave = 32 queries): S^T is a 32 keys x 32 queries MFMA tile, so each
// lane owns ONE query and 16 of the 32 keys: the softmax row max / sum are in-lane plus a
// single exchange with lane l ^ 32. P^T comes out of the S^T accumulator already in the
// B-operand order of the P V product; V^T rows are read with the matching key order.
#include <math.h>

#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kTaTP = 128;  // projection tile (positions)
constexpr int kTaTO = 64;   // output tile (positions)
constexpr int kTaQ = 128;   // queries per flash workgroup
constexpr int kTaK = 32;    // keys per flash step

// grid (np / 128, np, batch); block 256.
__global__ __launch_bounds__(256) void triattn_project(
    const bf16* __restrict__ z, const uint8_t* __restrict__ mask, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ wqkv, const bf16* __restrict__ wb,
    bf16* __restrict__ qo, bf16* __restrict__ ko, bf16* __restrict__ vto, f16* __restrict__ bo,
    int n, int np, int heads, int starting, int transposed_bias, float eps) {
  __shared__ __attribute__((aligned(16))) bf16 xh[kTaTP * kRow];
  __shared__ float keep[kTaTP];
  const int s0 = blockIdx.x * kTaTP;
  const int r = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int valid = (r < n) ? max(0, min(kTaTP, n - s0)) : 0;
  const bf16* base = z;
  int64_t stride = 128;
  if (valid > 0) {
    if (starting) {
      base = z + (((int64_t)b * n + r) * n + s0) * 128;
    } else {
      base = z + (((int64_t)b * n + s0) * n + r) * 128;
      stride = (int64_t)n * 128;
    }
  }
  ln_tile_128<kTaTP>(base, stride, valid, ln_w, ln_b, eps, xh, nullptr);
  // The bias entry at tile position t is for key s0 + t (query-major layout) or for key r
  // (key-major layout: the AF3 ending node, whose bias is not transposed).
  const bool key_major = !starting && !transposed_bias;
  if (tid < kTaTP) {
    const int key = key_major ? r : s0 + tid;
    keep[tid] = (key < n && mask[(int64_t)b * n + key] != 0) ? 1.f : 0.f;
  }
  __syncthreads();

  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int p0 = 32 * wave;  // this wave's 32 positions
  const bf16* xrow_li = xh + (p0 + li) * kRow;
  const int64_t rowplane = (int64_t)np * np;
  // q, k: D[position][d] (A = x rows, B = weight rows); lane li holds channel d = li.
#pragma unroll 1
  for (int t = 0; t < 2 * heads; ++t) {
    const int hh = t % heads;
    f32x16 acc = zero16();
    mma_rows<128>(xrow_li, wqkv + (int64_t)(t * 32 + li) * 128, g, acc);
    bf16* dst = (t < heads ? qo : ko) +
                ((((int64_t)b * heads + hh) * np + r) * np + s0 + p0) * 32 + li;
#pragma unroll
    for (int q = 0; q < 16; ++q) dst[(int64_t)acc_row(q, g) * 32] = (bf16)acc[q];
  }
  // v^T: D[d][position] (A = weight rows, B = x rows); lane li holds position p0 + li.
#pragma unroll 1
  for (int hh = 0; hh < heads; ++hh) {
    f32x16 acc = zero16();
    mma_rows<128>(wqkv + (int64_t)(2 * 128 + hh * 32 + li) * 128, xrow_li, g, acc);
    bf16* dst = vto + ((((int64_t)b * heads + hh) * np + r) * 32) * np + s0 + p0 + li;
#pragma unroll
    for (int q = 0; q < 16; ++q) dst[(int64_t)acc_row(q, g) * np] = (bf16)acc[q];
  }
  // bias: D[head][position] with the head rows zero-padded to 32.
  {
    f32x16 acc = zero16();
    mma_rows<128>(wb + (int64_t)li * 128, xrow_li, g, acc);
    const float kp = keep[p0 + li];
    if (g == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q < heads) {
          const float v = kp != 0.f ? acc[q] : -INFINITY;
          bo[(((int64_t)b * heads + q) * np + r) * np + s0 + p0 + li] = (f16)v;
        }
      }
    }
  }
}

// grid (np / 128, rows, batch * heads); block 256 (4 waves x 32 queries).
template <bool KEY_MAJOR>
__global__ __launch_bounds__(256) void flash_attn_bias(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ vt,
    const f16* __restrict__ bias, bf16* __restrict__ o, int heads, int64_t rows, int64_t np,
    int64_t rows_valid, int64_t n_valid, int64_t o_sb, int64_t o_sr, int64_t o_sj) {
  const int64_t j0 = (int64_t)blockIdx.x * kTaQ;
  const int64_t r = blockIdx.y;
  if (r >= rows_valid || j0 >= n_valid) return;  // whole workgroup outside the output
  const int64_t bh = blockIdx.z;
  const int64_t bidx = bh / heads;
  const int h = (int)(bh % heads);
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int64_t j = j0 + 32 * wave + li;  // this lane's query

  const bf16* qrow = q + ((bh * rows + r) * np + j) * 32;
  const bf16x8 q0 = ld8(qrow + 8 * g), q1 = ld8(qrow + 16 + 8 * g);
  const bf16* kbase = k + (bh * rows + r) * np * 32;
  const bf16* vrow = vt + ((bh * rows + r) * 32 + li) * np;  // row d = li of V^T
  const f16* bb = bias + bh * np * np;

  float m = -INFINITY, l = 0.f;
  f32x16 O = zero16();
#pragma unroll 1
  for (int64_t kb = 0; kb < np; kb += kTaK) {
    f32x16 S;
    if (!KEY_MAJOR) {
      const f16* brow = bb + j * np + kb + 4 * g;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f16x4 v4 = *reinterpret_cast<const f16x4*>(brow + 8 * qd);
#pragma unroll
        for (int t = 0; t < 4; ++t) S[4 * qd + t] = (float)v4[t];
      }
    } else {
#pragma unroll
      for (int qq = 0; qq < 16; ++qq) S[qq] = (float)bb[(kb + acc_row(qq, g)) * np + j];
    }
    const bf16* krow = kbase + (kb + li) * 32;
    S = mfma32(ld8(krow + 8 * g), q0, S);
    S = mfma32(ld8(krow + 16 + 8 * g), q1, S);

    float tmax = S[0];
#pragma unroll
    for (int qq = 1; qq < 16; ++qq) tmax = fmaxf(tmax, S[qq]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnew = fmaxf(m, tmax);
    const float muse = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = fast_exp2(m - muse);
    float ps = 0.f;
    bf16x8 p0, p1;
#pragma unroll
    for (int qq = 0; qq < 8; ++qq) {
      const float e0 = fast_exp2(S[qq] - muse);
      const float e1 = fast_exp2(S[qq + 8] - muse);
      ps += e0 + e1;
      p0[qq] = (bf16)e0;
      p1[qq] = (bf16)e1;
    }
    l = l * alpha + ps;
#pragma unroll
    for (int qq = 0; qq < 16; ++qq) O[qq] *= alpha;
    m = mnew;
    // V^T operand in the key order of p0 / p1: keys {4g..4g+3, 8+4g..8+4g+3} (+16).
    const bf16* vk = vrow + kb + 4 * g;
    const bf16x4 va = *reinterpret_cast<const bf16x4*>(vk);
    const bf16x4 vb = *reinterpret_cast<const bf16x4*>(vk + 8);
    const bf16x4 vc = *reinterpret_cast<const bf16x4*>(vk + 16);
    const bf16x4 vd = *reinterpret_cast<const bf16x4*>(vk + 24);
    const bf16x8 a0 = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
    const bf16x8 a1 = {vc[0], vc[1], vc[2], vc[3], vd[0], vd[1], vd[2], vd[3]};
    O = mfma32(a0, p0, O);
    O = mfma32(a1, p1, O);
  }
  l += __shfl_xor(l, 32, 64);
  if (j >= n_valid) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  bf16* dst = o + bidx * o_sb + r * o_sr + j * o_sj + h * 32;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    bf16x4 w;
#pragma unroll
    for (int t = 0; t < 4; ++t) w[t] = (bf16)(O[4 * qd + t] * inv);
    *reinterpret_cast<bf16x4*>(dst + 8 * qd + 4 * g) = w;
  }
}

// out = z + (sigmoid(LN_pair(z) W_g^T) * o) W_out^T; grid (ceil(n / 64), n, batch).
__global__ __launch_bounds__(256) void triattn_output(
    const bf16* __restrict__ z, const bf16* __restrict__ o, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ wg, const bf16* __restrict__ wo,
    bf16* __restrict__ out, int n, int residual, float eps) {
  __shared__ __attribute__((aligned(16))) bf16 zr[kTaTO * kRow];
  __shared__ __attribute__((aligned(16))) bf16 xh[kTaTO * kRow];
  __shared__ __attribute__((aligned(16))) bf16 y[kTaTO * kRow];
  const int j0 = blockIdx.x * kTaTO, i = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int valid = min(kTaTO, n - j0);
  const int64_t zoff = (((int64_t)b * n + i) * n + j0) * 128;
  ln_tile_128<kTaTO>(z + zoff, 128, valid, ln_w, ln_b, eps, xh, zr);
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int f = 32 * wave + li;
#pragma unroll 1
  for (int pt = 0; pt < kTaTO / 32; ++pt) {
    f32x16 ag = zero16();
    mma_rows<128>(xh + (pt * 32 + li) * kRow, wg + f * 128, g, ag);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int p = pt * 32 + acc_row(q, g);
      const float ov = p < valid ? (float)o[zoff + (int64_t)p * 128 + f] : 0.f;
      y[p * kRow + f] = (bf16)(sigmoidf_(ag[q]) * ov);
    }
  }
  __syncthreads();
#pragma unroll 1
  for (int pt = 0; pt < kTaTO / 32; ++pt) {
    f32x16 ao = zero16();
    mma_rows<128>(y + (pt * 32 + li) * kRow, wo + f * 128, g, ao);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int p = pt * 32 + acc_row(q, g);
      if (p < valid) {
        float val = ao[q];
        if (residual) val += (float)zr[p * kRow + f];
        out[zoff + (int64_t)p * 128 + f] = (bf16)val;
      }
    }
  }
}

void launch_flash(const FlashArgs& a, hipStream_t stream) {
  dim3 grid(a.np / kTaQ, a.rows, a.batch * a.heads);
  if (a.key_major) {
    flash_attn_bias<true><<<grid, 256, 0, stream>>>(a.q, a.k, a.vt, a.bias, a.o, a.heads, a.rows,
                                                    a.np, a.rows_valid, a.n_valid, a.o_sb, a.o_sr,
                                                    a.o_sj);
  } else {
    flash_attn_bias<false><<<grid, 256, 0, stream>>>(a.q, a.k, a.vt, a.bias, a.o, a.heads,
                                                     a.rows, a.np, a.rows_valid, a.n_valid,
                                                     a.o_sb, a.o_sr, a.o_sj);
  }
}

void launch_triattn(const TriattnArgs& a, hipStream_t stream) {
  const int np = a.np;
  dim3 gp(np / kTaTP, np, a.batch);
  triattn_project<<<gp, 256, 0, stream>>>(a.z, a.mask, a.ln_w, a.ln_b, a.wqkv, a.wb, a.q, a.k,
                                          a.vt, a.bias, a.n, np, a.heads, a.starting,
                                          a.transposed_bias, a.eps);
  FlashArgs f;
  f.q = a.q;
  f.k = a.k;
  f.vt = a.vt;
  f.bias = a.bias;
  f.o = a.o;
  f.batch = a.batch;
  f.rows = np;
  f.np = np;
  f.rows_valid = a.n;
  f.n_valid = a.n;
  f.heads = a.heads;
  f.key_major = (!a.starting && !a.transposed_bias) ? 1 : 0;
  // o is written in the frame of z: row r of the attention is a row (starting) or a
  // column (ending) of z.
  const int64_t c = 128;
  f.o_sb = (int64_t)a.n * a.n * c;
  if (a.starting) {
    f.o_sr = (int64_t)a.n * c;
    f.o_sj = c;
  } else {
    f.o_sr = c;
    f.o_sj = (int64_t)a.n * c;
  }
  launch_flash(f, stream);
  dim3 go((a.n + kTaTO - 1) / kTaTO, a.n, a.batch);
  triattn_output<<<go, 256, 0, stream>>>(a.z, a.o, a.ln_w, a.ln_b, a.wg, a.wo, a.out, a.n,
                                         a.residual, a.eps);
}

}  // namespace ffk
