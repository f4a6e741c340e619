// MSA pair-weighted averaging on gfx950 (the MSA stack's pair-to-MSA update).
//
// Equations: src/foldforge/models/checkpoints/legacy/attention.py:203-223 (MSAAttention):
//   x = LN_msa(m); w[h, i, :] = softmax_j(LN_pair(z)[i, j] . W_b[h]) over valid keys j;
//   o[s, i, h] = sum_j w[h, i, j] v[s, j, h], v = x W_v^T; out = m + (sigmoid(x W_g^T) o) W_out^T.
// The weights do not depend on the MSA row s, so per head the average is one GEMM
//   O_h[(s, c)][i] = sum_j v^T_h[(s, c)][j] w_h[i][j]
// with all S MSA rows stacked along M. The C-ABI (api.hip) runs (the token-row GEMMs through
// launch_row_gemm, which takes the streaming row_stream where the width allows):
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

constexpr int kPT = 128;         // output tile: 128 (s, c) rows x 128 queries
constexpr int kPK = 32;          // keys per LDS stage
constexpr int kPKP = kPK + 8;    // LDS row stride (80 B: conflict-free 16-byte reads)
constexpr int kPOS = kPT + 4;    // epilogue fp32 row stride: 64 x kPOS floats fit in the operand stages
static_assert(64 * kPOS * 4 <= 4 * kPT * kPKP * 2, "epilogue staging exceeds the operand LDS");

// Per (batch, head): O[(s, c)][i] = sum_j v^T[(s, c)][j] w[i][j], an NT GEMM with both operands
// key-contiguous. grid: ceil(S dh / 128) * ceil(n / 128) * batch * heads workgroups (renumbered
// so that neighbours share an XCD's L2), block 256 = 2 x 2 waves of 64 x 64; operands staged
// through LDS 32 keys at a time (register prefetch two stages ahead, double buffer, one barrier per stage).
// v^T is not written at keys >= n: those operand entries are zeroed as they are staged.
// Epilogue: lane (li, g) holds query q0' + li and rows r = r0' + 8 v + 4 g + e, i.e.
// (s, c) = (r / dh, r % dh): four consecutive channels of one MSA row (dh % 4 == 0).
__global__ __launch_bounds__(256) void pwa_average(PwaAverageArgs a) {
  // operand stages xs[2] then ys[2]; after the key loop the epilogue reuses it as fp32 [64][kPOS]
  __shared__ __attribute__((aligned(16))) bf16 lds[4 * kPT * kPKP];
  bf16 (*xs)[kPT * kPKP] = reinterpret_cast<bf16 (*)[kPT * kPKP]>(lds);
  bf16 (*ys)[kPT * kPKP] = reinterpret_cast<bf16 (*)[kPT * kPKP]>(lds + 2 * kPT * kPKP);
  const int rows = a.depth * a.dh, n = a.n, np = a.np;
  const int rt = (rows + kPT - 1) / kPT, qt = (n + kPT - 1) / kPT;
  const uint32_t wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / ((uint32_t)rt * qt);
  const int rem = (int)(wg - bh * rt * qt);
  const int r0 = (rem / qt) * kPT, q0 = (rem % qt) * kPT;
  const int64_t b = bh / a.heads;
  const int h = (int)(bh - b * a.heads);
  const bf16* X = a.vt + bh * rows * (int64_t)np;
  const bf16* Y = a.w + bh * n * (int64_t)np;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, g = lane >> 5;

  const bf16* xsrc[2];
  const bf16* ysrc[2];
  int soff[2], kcol[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int c = tid + 256 * u;
    const int row = c >> 2, kc = (c & 3) * 8;
    xsrc[u] = X + (int64_t)min(r0 + row, rows - 1) * np + kc;
    ysrc[u] = Y + (int64_t)min(q0 + row, n - 1) * np + kc;
    soff[u] = row * kPKP + kc;
    kcol[u] = kc;
  }
  // Two register sets carry the next two stages (stage s + 1 lands in LDS while stage s + 3 is
  // fetched), so a stage's global loads have two stages of MFMAs to land behind.
  bf16x8 rx0[2], ry0[2], rx1[2], ry1[2];
  auto gload = [&](bf16x8 (&rx)[2], bf16x8 (&ry)[2], int k0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      rx[u] = ld8(xsrc[u] + k0);
      ry[u] = ld8(ysrc[u] + k0);
    }
  };
  auto sstore = [&](bf16x8 (&rx)[2], const bf16x8 (&ry)[2], int k0, int buf) {
    if (k0 + kPK > n) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (k0 + kcol[u] + e >= n) rx[u][e] = (bf16)0.f;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      *reinterpret_cast<bf16x8*>(&xs[buf][soff[u]]) = rx[u];
      *reinterpret_cast<bf16x8*>(&ys[buf][soff[u]]) = ry[u];
    }
  };
  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = zero16();
  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < kPK; kk += 16) {
      bf16x8 av[2], bv[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) av[mi] = ld8(&xs[buf][(wm * 64 + mi * 32 + li) * kPKP + kk + 8 * g]);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) bv[ni] = ld8(&ys[buf][(wn * 64 + ni * 32 + li) * kPKP + kk + 8 * g]);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(av[mi], bv[ni], acc[mi][ni]);
    }
  };

  // np is a multiple of 64: an even number (>= 2) of stages, taken two per iteration (buffers 0, 1)
  const int ns = np / kPK;
  gload(rx0, ry0, 0);
  sstore(rx0, ry0, 0, 0);
  gload(rx1, ry1, kPK);
  if (ns > 2) gload(rx0, ry0, 2 * kPK);
  __syncthreads();
#pragma unroll 1
  for (int st = 0; st < ns; st += 2) {
    compute(0);                   // stage st; rx1 holds stage st + 1, rx0 stage st + 2 (if any)
    sstore(rx1, ry1, (st + 1) * kPK, 1);
    if (st + 3 < ns) gload(rx1, ry1, (st + 3) * kPK);
    __syncthreads();
    compute(1);                   // stage st + 1
    if (st + 2 < ns) {
      sstore(rx0, ry0, (st + 2) * kPK, 0);
      if (st + 4 < ns) gload(rx0, ry0, (st + 4) * kPK);
    }
    __syncthreads();
  }

  const int hd = a.heads * a.dh;
  if (a.dh % 8 == 0) {
    // Staged: one half of the queries (ni) at a time goes through LDS as fp32 [query][row]; each
    // lane then gates and stores 8 consecutive rows of one query, i.e. 16 bytes of one MSA
    // row's head channels (dh % 8 == 0 keeps such a piece inside one MSA row).
    float* T = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      if (ni) __syncthreads();
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          f32x4 y;
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = acc[mi][ni][4 * v + e];
          *reinterpret_cast<f32x4*>(&T[(wn * 32 + li) * kPOS + wm * 64 + mi * 32 + 8 * v + 4 * g]) = y;
        }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int id = tid + 256 * u, ql = id >> 4, rl = (id & 15) * 8;
        const int q = q0 + (ql >> 5) * 64 + ni * 32 + (ql & 31), r = r0 + rl;
        if (q >= n || r >= rows) continue;
        const int s = r / a.dh, c = r - s * a.dh;
        const int64_t off = ((b * a.depth + s) * n + q) * hd + h * a.dh + c;
        const bf16x8 gv = ld8(a.gate + off);
        const f32x4 y0 = *reinterpret_cast<const f32x4*>(&T[ql * kPOS + rl]);
        const f32x4 y1 = *reinterpret_cast<const f32x4*>(&T[ql * kPOS + rl + 4]);
        bf16x8 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = (bf16)(y0[e] * (float)gv[e]);
          o[4 + e] = (bf16)(y1[e] * (float)gv[4 + e]);
        }
        *reinterpret_cast<bf16x8*>(a.og + off) = o;
      }
    }
    return;
  }
#pragma unroll
  for (int ni = 0; ni < 2; ++ni) {
    const int q = q0 + wn * 64 + ni * 32 + li;
    if (q >= n) continue;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = r0 + wm * 64 + mi * 32 + 8 * v + 4 * g;
        if (r >= rows) continue;
        const int s = r / a.dh, c = r - s * a.dh;
        const int64_t off = ((b * a.depth + s) * n + q) * hd + h * a.dh + c;
        const bf16x4 gv = *reinterpret_cast<const bf16x4*>(a.gate + off);
        store4(a.og + off, acc[mi][ni][4 * v] * (float)gv[0], acc[mi][ni][4 * v + 1] * (float)gv[1],
               acc[mi][ni][4 * v + 2] * (float)gv[2], acc[mi][ni][4 * v + 3] * (float)gv[3]);
      }
  }
}

}  // namespace

void launch_pwa_softmax(const PwaSoftmaxArgs& a, hipStream_t stream) {
  pwa_softmax<<<dim3((unsigned)((a.rows + 3) / 4)), 256, 0, stream>>>(a);
}

void launch_pwa_average(const PwaAverageArgs& a, hipStream_t stream) {
  const int64_t rt = ((int64_t)a.depth * a.dh + kPT - 1) / kPT, qt = (a.n + kPT - 1) / kPT;
  pwa_average<<<dim3((unsigned)(rt * qt * a.batch * a.heads)), 256, 0, stream>>>(a);
}

}  // namespace ffk
