// Triangle multiplicative update (outgoing / incoming) on gfx950.
//
// Three kernels per call (equations: src/foldforge/models/checkpoints/legacy/reference/triangle.py:39-49):
//   1. trimul_project  z -> LN_pair -> A = (x W_l^T) * M * sigmoid(x W_lg^T), B likewise,
//                      written channel-major [B][h][np][np] so that the contraction is a
//                      K-contiguous batched GEMM in both directions (incoming tiles walk
//                      columns of z, which stores A^T).
//   2. trimul_contract P[bh] = X[bh] Y[bh]^T on MFMA, 128x128 tiles, LDS double buffer.
//   3. trimul_output   LN_out(P) W_out^T * sigmoid(LN_pair(z) W_g^T) + z, channel-last.
// The output gate is recomputed from z in kernel 3 (z is read there for the residual
// anyway) instead of being stored: 128 channels of gate would cost 2 x 67 MB of HBM
// traffic at N = 512 against 8.6 GFLOP of MFMA work.
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kTrimulTP = 128;  // positions per projection tile
constexpr int kTrimulTO = 64;   // positions per output tile
constexpr int kCT = 128;        // contraction output tile
constexpr int kCK = 32;         // contraction k step
constexpr int kCKP = kCK + 8;   // LDS row stride of a contraction operand tile

// grid (np / 128, np, batch); block 256.
// wp rows: [0,h) to_left, [h,2h) to_left_gate, [2h,3h) to_right, [3h,4h) to_right_gate.
__global__ __launch_bounds__(256) void trimul_project(
    const bf16* __restrict__ z, const uint8_t* __restrict__ mask, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ wp, bf16* __restrict__ a_out,
    bf16* __restrict__ b_out, int n, int np, int outgoing, float eps) {
  __shared__ __attribute__((aligned(16))) bf16 xh[kTrimulTP * kRow];
  __shared__ float pm[kTrimulTP];
  constexpr int H = 128;
  const int s0 = blockIdx.x * kTrimulTP;
  const int r = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int valid = (r < n) ? max(0, min(kTrimulTP, n - s0)) : 0;
  const bf16* base = z;
  int64_t stride = 128;
  if (valid > 0) {
    if (outgoing) {
      base = z + (((int64_t)b * n + r) * n + s0) * 128;
    } else {
      base = z + (((int64_t)b * n + s0) * n + r) * 128;
      stride = (int64_t)n * 128;
    }
  }
  ln_tile_128<kTrimulTP>(base, stride, valid, ln_w, ln_b, eps, xh, nullptr);
  if (tid < kTrimulTP) {
    float m = 0.f;
    if (tid < valid) {
      const uint8_t* mb = mask + (int64_t)b * n;
      m = (mb[r] != 0 && mb[s0 + tid] != 0) ? 1.f : 0.f;
    }
    pm[tid] = m;
  }
  __syncthreads();

  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int p = 32 * wave + li;  // position of this lane (D column)
  const bf16* xrow = xh + p * kRow;
  const float m = pm[p];
  const int64_t plane = (int64_t)np * np;
  const int64_t off = (int64_t)r * np + s0 + p;
#pragma unroll 1
  for (int branch = 0; branch < 2; ++branch) {
    bf16* dst = (branch == 0 ? a_out : b_out) + (int64_t)b * H * plane + off;
#pragma unroll 1
    for (int fc = 0; fc < H / 32; ++fc) {
      const bf16* wv = wp + (int64_t)(branch * 2 * H + fc * 32 + li) * 128;
      const bf16* wgt = wv + (int64_t)H * 128;
      f32x16 av = zero16(), ag = zero16();
      mma_rows<128>(wv, xrow, g, av);
      mma_rows<128>(wgt, xrow, g, ag);
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int f = fc * 32 + acc_row(q, g);
        dst[(int64_t)f * plane] = (bf16)(av[q] * m * sigmoidf_(ag[q]));
      }
    }
  }
}

// P[bh][i][j] = sum_k X[bh][i][k] * Y[bh][j][k]; all planes [np][np] bf16, np % 128 == 0.
// grid (np / 128, np / 128, batch * h); block 256 = 2 x 2 waves of 64 x 64.
__global__ __launch_bounds__(256) void trimul_contract(const bf16* __restrict__ X,
                                                       const bf16* __restrict__ Y,
                                                       bf16* __restrict__ P, int np) {
  __shared__ __attribute__((aligned(16))) bf16 xs[2][kCT * kCKP];
  __shared__ __attribute__((aligned(16))) bf16 ys[2][kCT * kCKP];
  const int j0 = blockIdx.x * kCT, i0 = blockIdx.y * kCT;
  const int64_t plane = (int64_t)np * np;
  const bf16* Xb = X + blockIdx.z * plane + (int64_t)i0 * np;
  const bf16* Yb = Y + blockIdx.z * plane + (int64_t)j0 * np;
  const int tid = threadIdx.x;
  // global -> LDS: a 128 x 32 tile is 512 chunks of 8 bf16; 2 per thread per operand.
  bf16x8 rx[2], ry[2];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 2, kc = (c & 3) * 8;
      rx[u] = ld8(Xb + (int64_t)row * np + k0 + kc);
      ry[u] = ld8(Yb + (int64_t)row * np + k0 + kc);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 2, kc = (c & 3) * 8;
      *reinterpret_cast<bf16x8*>(&xs[buf][row * kCKP + kc]) = rx[u];
      *reinterpret_cast<bf16x8*>(&ys[buf][row * kCKP + kc]) = ry[u];
    }
  };
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[a][c] = zero16();

  gload(0);
  sstore(0);
  __syncthreads();
  int buf = 0;
#pragma unroll 1
  for (int k0 = 0; k0 < np; k0 += kCK) {
    const bool more = k0 + kCK < np;
    if (more) gload(k0 + kCK);
#pragma unroll
    for (int kk = 0; kk < kCK; kk += 16) {
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        av[mi] = ld8(&xs[buf][(wm * 64 + mi * 32 + li) * kCKP + kk + 8 * g]);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
        bv[ni] = ld8(&ys[buf][(wn * 64 + ni * 32 + li) * kCKP + kk + 8 * g]);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(av[mi], bv[ni], acc[mi][ni]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  bf16* Pb = P + blockIdx.z * plane;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int j = j0 + wn * 64 + ni * 32 + li;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int i = i0 + wm * 64 + mi * 32 + acc_row(q, g);
        Pb[(int64_t)i * np + j] = (bf16)acc[mi][ni][q];
      }
    }
}

// out[b,i,j,:] = z + (LN_out(P[b,:,i,j]) W_out^T) * sigmoid(LN_pair(z[b,i,j]) W_g^T).
// grid (ceil(n / 64), n, batch); block 256.
__global__ __launch_bounds__(256) void trimul_output(
    const bf16* __restrict__ z, const bf16* __restrict__ P, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const float* __restrict__ lno_w,
    const float* __restrict__ lno_b, const bf16* __restrict__ wg, const bf16* __restrict__ wo,
    bf16* __restrict__ out, int n, int np, int residual, float eps) {
  __shared__ __attribute__((aligned(16))) bf16 zr[kTrimulTO * kRow];
  __shared__ __attribute__((aligned(16))) bf16 xh[kTrimulTO * kRow];
  __shared__ __attribute__((aligned(16))) bf16 y[kTrimulTO * kRow];
  __shared__ float red[4][kTrimulTO];
  constexpr int H = 128;
  const int j0 = blockIdx.x * kTrimulTO, i = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int valid = min(kTrimulTO, n - j0);
  const int64_t zoff = (((int64_t)b * n + i) * n + j0) * 128;
  ln_tile_128<kTrimulTO>(z + zoff, 128, valid, ln_w, ln_b, eps, xh, zr);

  // centre norm over the 128 hidden channels of P: wave q reads channels 32q..32q+31 of
  // the 64 positions (each read is 64 consecutive positions of one channel plane).
  {
    const int pos = tid & 63, q = tid >> 6;
    const int64_t plane = (int64_t)np * np;
    const bf16* pp = P + ((int64_t)b * H + 32 * q) * plane + (int64_t)i * np + j0 + pos;
    float v[32];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      v[e] = pos < valid ? (float)pp[(int64_t)e * plane] : 0.f;
      s += v[e];
    }
    red[q][pos] = s;
    __syncthreads();
    const float mean = (red[0][pos] + red[1][pos] + red[2][pos] + red[3][pos]) * (1.f / H);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      v[e] -= mean;
      ss += v[e] * v[e];
    }
    __syncthreads();
    red[q][pos] = ss;
    __syncthreads();
    const float var = (red[0][pos] + red[1][pos] + red[2][pos] + red[3][pos]) * (1.f / H);
    const float rstd = __builtin_amdgcn_rsqf(var + eps);
#pragma unroll
    for (int e8 = 0; e8 < 4; ++e8) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 32 * q + 8 * e8 + e;
        o[e] = (bf16)(v[8 * e8 + e] * rstd * lno_w[c] + lno_b[c]);
      }
      *reinterpret_cast<bf16x8*>(&y[pos * kRow + 32 * q + 8 * e8]) = o;
    }
  }
  __syncthreads();

  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int f = 32 * wave + li;  // output channel of this lane
#pragma unroll 1
  for (int pt = 0; pt < kTrimulTO / 32; ++pt) {
    f32x16 ag = zero16(), ao = zero16();
    mma_rows<128>(xh + (pt * 32 + li) * kRow, wg + f * 128, g, ag);
    mma_rows<128>(y + (pt * 32 + li) * kRow, wo + f * H, g, ao);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int p = pt * 32 + acc_row(q, g);
      if (p < valid) {
        float val = ao[q] * sigmoidf_(ag[q]);
        if (residual) val += (float)zr[p * kRow + f];
        out[zoff + (int64_t)p * 128 + f] = (bf16)val;
      }
    }
  }
}

void launch_trimul(const TrimulArgs& a, hipStream_t stream) {
  const int np = a.np;
  dim3 gp(np / kTrimulTP, np, a.batch);
  trimul_project<<<gp, 256, 0, stream>>>(a.z, a.mask, a.ln_w, a.ln_b, a.wp, a.A, a.B, a.n, np,
                                         a.outgoing, a.eps);
  dim3 gc(np / kCT, np / kCT, a.batch * 128);
  trimul_contract<<<gc, 256, 0, stream>>>(a.A, a.B, a.P, np);
  dim3 go((a.n + kTrimulTO - 1) / kTrimulTO, a.n, a.batch);
  trimul_output<<<go, 256, 0, stream>>>(a.z, a.P, a.ln_w, a.ln_b, a.lno_w, a.lno_b, a.wg, a.wo,
                                        a.out, a.n, np, a.residual, a.eps);
}

}  // namespace ffk
