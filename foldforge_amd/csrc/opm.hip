// Outer product mean on gfx950 (the MSA stack's MSA-to-pair update).
//
// Equations: src/foldforge/models/checkpoints/legacy/primitives.py:40-136 (OuterProductMean)
// and legacy/reference/attention.py:57-74 (af3_outer_product_mean), in the engine's forms
// (src/foldforge/modules/engine/modules.py:184-210):
//   l[s, i] = m[s, i] (LN(msa[s, i]) W_l^T + b_l),  r[s, j] = m[s, j] (LN(msa[s, j]) W_r^T + b_r)
//   o[i, j, (c, e)] = sum_s l[s, i, c] r[s, j, e],   n[i, j] = sum_s m[s, i] m[s, j]
//   AF3: out = (o W_out^T + b) / (n + 1e-3); the clamp form divides by max(n, 1); the
//   normalize-before-projection form is (o / d) W_out^T + b.
// The C-ABI (api.hip) runs:
//   row_gemm<kEpiOpm, kXLn> (single.hip): LayerNorm + both projections, masked, stored with
//     the MSA rows contiguous (l^T, r^T [batch][n][32][sp], sp = depth padded to 64) and the
//     mask transposed
//   opm_count: n[i, j] as a 0/1 GEMM over the MSA rows (exact in fp32)
//   opm_pack: W_out rounded to bf16 in the contraction's k order
//   opm_contract: per workgroup a tile of 8 x 8 tokens: the 256 x 256 outer-product block
//     summed over all MSA rows on MFMA, rounded to bf16 into LDS, projected to c_z on MFMA,
//     divided by the count, bias and residual added.
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

namespace {

constexpr int kOpmC = 32;                   // channels per side (d_hidden)
constexpr int kOpmT = 8;                    // tokens per tile side
constexpr int kOpmRows = kOpmT * kOpmC;     // (token, channel) rows of one operand tile
constexpr int kOpmKC = 32;                  // MSA rows per LDS stage (the MSA padding is 64)
constexpr int kOpmKS = kOpmKC + 8;          // LDS row stride of a stage (conflict-free reads)
constexpr int kOpmCPR = kOpmKC / 8;         // 16-byte chunks per operand row and stage
constexpr int kOpmPT = kOpmRows * kOpmCPR / 512;  // chunks per thread and operand
constexpr int kOpmPairs = kOpmT * kOpmT;    // pairs per tile
constexpr int kOpmK2 = kOpmC * kOpmC;       // 1024: the projection's k
constexpr int kOpmOS = kOpmK2 + 8;          // LDS row stride of a pair's outer product

// Tile order within a batch element: runs of 8 tile rows, walked column by column, so the 32
// neighbouring workgroups an XCD holds at once (consecutive ids after xcd_remap) cover 8 tile
// rows x 4 tile columns and share each operand block through that XCD's L2 (a row-major order
// gives them one tile row and 32 distinct column operands). A bijection of [0, nti * ntj).
__device__ __forceinline__ void grouped_tile(int t, int nti, int ntj, int& ti, int& tj) {
  constexpr int kRows = 8;
  const int per = kRows * ntj, first = (t / per) * kRows;
  const int rows = min(nti - first, kRows), u = t - (t / per) * per;
  ti = first + u % rows;
  tj = u / rows;
}
constexpr size_t kOpmStageBytes = (size_t)2 * 2 * kOpmRows * kOpmKS * sizeof(bf16);
constexpr size_t kOpmOBytes = (size_t)kOpmPairs * kOpmOS * sizeof(bf16);
constexpr size_t kOpmLds = kOpmStageBytes > kOpmOBytes ? kOpmStageBytes : kOpmOBytes;

// One wave per 32 x 32 block of pairs: count[i][j] = sum_s mt[i][s] mt[j][s].
__global__ __launch_bounds__(64) void opm_count(OpmCountArgs a) {
  const int lane = threadIdx.x, li = lane & 31, g = lane >> 5;
  const int i0 = blockIdx.x * 32, j0 = blockIdx.y * 32;
  const int64_t b = blockIdx.z;
  const bf16* ar = a.mt + (b * a.n + min(i0 + li, a.n - 1)) * a.sp + 8 * g;
  const bf16* br = a.mt + (b * a.n + min(j0 + li, a.n - 1)) * a.sp + 8 * g;
  f32x16 acc = zero16();
  for (int k = 0; k < a.sp; k += 16) acc = mfma32(ld8(ar + k), ld8(br + k), acc);
  const int j = j0 + li;
  if (j >= a.n) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = i0 + acc_row(r, g);
    if (i < a.n) a.count[(b * a.n + i) * a.n + j] = acc[r];
  }
}

// wp[f][k'] = W[f][c * 32 + e] with k' = 32 e + 16 g + r and c = acc_row(r, g): the order in
// which a lane of the contraction holds its accumulators (see opm_contract).
__global__ __launch_bounds__(256) void opm_pack(const float* __restrict__ w, bf16* __restrict__ wp,
                                                int cz) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= cz * kOpmK2) return;
  const int f = idx / kOpmK2, kp = idx % kOpmK2;
  const int e = kp >> 5, q = kp & 31;
  const int c = acc_row(q & 15, q >> 4);
  wp[idx] = (bf16)w[(int64_t)f * kOpmK2 + c * kOpmC + e];
}

// grid: ceil(n / 8)^2 * batch workgroups of 512 threads.
// Phase 1 (outer products): wave w accumulates the 2 x 4 pairs (i0 + 2 (w / 2) + mi,
// j0 + 4 (w % 2) + nj); pair (i, j) is one 32 x 32 MFMA tile, A = l^T rows of token i, B = r^T
// rows of token j, k = MSA rows, staged through LDS 32 rows at a time (double buffer, one
// barrier per stage). Lane (li, g) ends with o[c = acc_row(r, g)][e = li] in acc[r].
// Phase 2 (projection): the 64 outer products go to LDS as bf16 rows of 1024 in the order
// k' = 32 e + 16 g + r (each lane writes 32 contiguous bytes); wave w then computes 32 output
// channels (w % 4) x 32 pairs (w / 4): A = packed W_out rows, B = outer-product rows.
__global__ __launch_bounds__(512) void opm_contract(OpmContractArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* xs = reinterpret_cast<bf16*>(smem);  // [2][kOpmRows][kOpmKS]
  bf16* ys = xs + 2 * kOpmRows * kOpmKS;     // [2][kOpmRows][kOpmKS]
  bf16* os = reinterpret_cast<bf16*>(smem);  // [kOpmPairs][kOpmOS], after phase 1
  const int n = a.n, sp = a.sp;
  const int nt = (n + kOpmT - 1) / kOpmT;
  const uint32_t t = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t b = t / ((uint32_t)nt * nt);
  int ti, tj;
  grouped_tile((int)(t - b * nt * nt), nt, nt, ti, tj);
  const int i0 = ti * kOpmT, j0 = tj * kOpmT;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, g = lane >> 5;

  // global -> LDS: an operand stage is 256 rows x kOpmKC MSA rows in chunks of 8 bf16
  const bf16* xsrc[kOpmPT];
  const bf16* ysrc[kOpmPT];
  int soff[kOpmPT];
#pragma unroll
  for (int u = 0; u < kOpmPT; ++u) {
    const int c = tid + 512 * u;
    const int row = c / kOpmCPR, kc = (c % kOpmCPR) * 8;
    const int ti_tok = min(i0 + (row >> 5), n - 1), tj_tok = min(j0 + (row >> 5), n - 1);
    xsrc[u] = a.lt + ((b * n + ti_tok) * kOpmC + (row & 31)) * sp + kc;
    ysrc[u] = a.rt + ((b * n + tj_tok) * kOpmC + (row & 31)) * sp + kc;
    soff[u] = row * kOpmKS + kc;
  }
  bf16x8 rx[kOpmPT], ry[kOpmPT];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < kOpmPT; ++u) {
      rx[u] = ld8(xsrc[u] + k0);
      ry[u] = ld8(ysrc[u] + k0);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kOpmPT; ++u) {
      *reinterpret_cast<bf16x8*>(xs + buf * kOpmRows * kOpmKS + soff[u]) = rx[u];
      *reinterpret_cast<bf16x8*>(ys + buf * kOpmRows * kOpmKS + soff[u]) = ry[u];
    }
  };

  const int wi = wave >> 1, wj = wave & 1;
  f32x16 acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) acc[mi][nj] = zero16();

  gload(0);
  sstore(0);
  __syncthreads();
  int buf = 0;
#pragma unroll 1
  for (int k0 = 0; k0 < sp; k0 += kOpmKC) {
    const bool more = k0 + kOpmKC < sp;
    if (more) gload(k0 + kOpmKC);
    const bf16* xb = xs + buf * kOpmRows * kOpmKS;
    const bf16* yb = ys + buf * kOpmRows * kOpmKS;
#pragma unroll
    for (int kk = 0; kk < kOpmKC; kk += 16) {
      bf16x8 av[2], bv[4];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
        av[mi] = ld8(xb + ((2 * wi + mi) * kOpmC + li) * kOpmKS + kk + 8 * g);
#pragma unroll
      for (int nj = 0; nj < 4; ++nj)
        bv[nj] = ld8(yb + ((4 * wj + nj) * kOpmC + li) * kOpmKS + kk + 8 * g);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int nj = 0; nj < 4; ++nj) acc[mi][nj] = mfma32(av[mi], bv[nj], acc[mi][nj]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();  // also ends every read of the stages before the outer products land
    buf ^= 1;
  }

#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      const int p = (2 * wi + mi) * kOpmT + 4 * wj + nj;
      bf16x8 lo, hi;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        lo[r] = (bf16)acc[mi][nj][r];
        hi[r] = (bf16)acc[mi][nj][8 + r];
      }
      bf16* dst = os + p * kOpmOS + li * 32 + 16 * g;
      *reinterpret_cast<bf16x8*>(dst) = lo;
      *reinterpret_cast<bf16x8*>(dst + 8) = hi;
    }
  __syncthreads();

  const int pw = wave >> 2, fw = wave & 3;
  const bf16* wrow = a.wp + (int64_t)(32 * fw + li) * kOpmK2 + 8 * g;
  const bf16* orow = os + (32 * pw + li) * kOpmOS + 8 * g;
  f32x16 acc2 = zero16();
#pragma unroll 2
  for (int k = 0; k < kOpmK2; k += 64) {
    bf16x8 wv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) wv[s] = ld8(wrow + k + 16 * s);
#pragma unroll
    for (int s = 0; s < 4; ++s) acc2 = mfma32(wv[s], ld8(orow + k + 16 * s), acc2);
  }

  const int p = 32 * pw + li;
  const int i = i0 + p / kOpmT, j = j0 + p % kOpmT;
  if (i >= n || j >= n) return;
  const int64_t pij = (b * n + i) * n + j;
  const float cnt = a.count[pij];
  const float d = a.count_offset >= 0.f ? cnt + a.count_offset : fmaxf(cnt, 1.f);
  const int64_t off = pij * a.cz;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int f = 32 * fw + 8 * v + 4 * g;
    const f32x4 bias = *reinterpret_cast<const f32x4*>(a.bias + f);
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      y[e] = a.normalize_before_proj ? acc2[4 * v + e] / d + bias[e] : (acc2[4 * v + e] + bias[e]) / d;
    if (a.res) {
      const bf16x4 r = *reinterpret_cast<const bf16x4*>(a.res + off + f);
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] += (float)r[e];
    }
    store4(a.out + off + f, y[0], y[1], y[2], y[3]);
  }
}


// ---------------------------------------------------------------------------- grouped (Chai-1)
// Chai-1's grouped outer product mean (legacy/primitives.py:122-136, 8 groups of 8 channels a
// side; src/foldforge/modules/dense/spec.py:687-688): products only within each group, summed
// over the MSA rows and divided by nothing,
//   p[i, j, (g, k, l)] = sum_s l[s, i, 8 g + k] r[s, j, 8 g + l]            (512 per pair)
//   out[i, j] = LN_0.1(p[i, j]) W_out^T + b_out                 (product norm over the 512)
// grid: ceil(n / 4) * ceil(n / 8) * batch workgroups of 512 threads, one tile of 4 x 8 tokens.
// Phase 1: per group the products are one dense product, rows (token i, k) x columns (token j,
// l) over the MSA rows, so wave w takes group w: two 32 x 32 MFMA tiles, rows (i = row / 8,
// k = row % 8) for the tile's 4 tokens i, columns (j = 4 h + li / 8, l = li % 8) for h = 0, 1.
// Lane (li, g) holds row acc_row(r, g) of column li in acc[h][r]; the products go to LDS in
// fp32 in the (g, k, l) order. In the operand stages token t's 64 rows (8 groups x 8) start
// 128 t bytes later than unpadded, so the 16 lanes of a read (two neighbouring tokens' 8 rows of
// one group, 80-byte rows) cover all 64 banks.
// Phase 2: one wave per pair normalises the 512 products (two passes over 8 per lane), rounds
// them to bf16 rows; phase 3: the c_z / 32 output tiles (each over 32 pairs, k = 512; at c_z
// 128 the k range is split over two waves and summed through LDS), bias and residual added.
constexpr int kOgC = 64;                      // channels per side (8 groups x 8)
constexpr int kOgTI = 4, kOgTJ = 8;           // tokens per tile side
constexpr int kOgPairs = kOgTI * kOgTJ;       // 32
constexpr int kOgN = 512;                     // products per pair
constexpr int kOgNS = kOgN + 8;               // LDS row stride of a normalised pair (bf16)
constexpr int kOgXRows = kOgTI * kOgC, kOgYRows = kOgTJ * kOgC;
constexpr int kOgXPT = kOgXRows * kOpmCPR / 512, kOgYPT = kOgYRows * kOpmCPR / 512;
constexpr int kOgTokPad = 64;                 // stage rows of token t shifted by t x 128 bytes (bf16 units)
constexpr int kOgXB = kOgXRows * kOpmKS + kOgTI * kOgTokPad;  // one stage of each operand
constexpr int kOgYB = kOgYRows * kOpmKS + kOgTJ * kOgTokPad;
constexpr size_t kOgStageBytes = (size_t)2 * (kOgXB + kOgYB) * sizeof(bf16);
constexpr size_t kOgProdBytes = (size_t)kOgPairs * kOgN * sizeof(float);
constexpr size_t kOgNormBytes = (size_t)kOgPairs * kOgNS * sizeof(bf16);
constexpr size_t kOgLds = kOgStageBytes > kOgProdBytes + kOgNormBytes ? kOgStageBytes : kOgProdBytes + kOgNormBytes;

template <int CZ>
__global__ __launch_bounds__(512) void opm_contract_grouped(OpmGroupedArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* xs = reinterpret_cast<bf16*>(smem);  // [2][kOgXB]: rows (token, channel) x kOpmKS
  bf16* ys = xs + 2 * kOgXB;                 // [2][kOgYB]
  float* prod = reinterpret_cast<float*>(smem);                     // [32][512], after phase 1
  bf16* nrm = reinterpret_cast<bf16*>(smem + kOgProdBytes);         // [32][kOgNS]
  float* red = reinterpret_cast<float*>(smem);                      // phase 3 (c_z 128) partials
  const int n = a.n, sp = a.sp;
  const int nti = (n + kOgTI - 1) / kOgTI, ntj = (n + kOgTJ - 1) / kOgTJ;
  const uint32_t t = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t b = t / ((uint32_t)nti * ntj);
  int ti, tj;
  grouped_tile((int)(t - b * nti * ntj), nti, ntj, ti, tj);
  const int i0 = ti * kOgTI, j0 = tj * kOgTJ;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, g = lane >> 5;

  // global -> LDS: a stage is the operand rows (token, channel) x kOpmKC MSA rows, 8 bf16 a chunk
  const bf16* xsrc[kOgXPT];
  const bf16* ysrc[kOgYPT];
  int xoff[kOgXPT], yoff[kOgYPT];
#pragma unroll
  for (int u = 0; u < kOgXPT; ++u) {
    const int c = tid + 512 * u, row = c / kOpmCPR, kc = (c % kOpmCPR) * 8;
    const int tok = min(i0 + row / kOgC, n - 1);
    xsrc[u] = a.lt + ((b * n + tok) * kOgC + row % kOgC) * sp + kc;
    xoff[u] = row * kOpmKS + kc + (row / kOgC) * kOgTokPad;
  }
#pragma unroll
  for (int u = 0; u < kOgYPT; ++u) {
    const int c = tid + 512 * u, row = c / kOpmCPR, kc = (c % kOpmCPR) * 8;
    const int tok = min(j0 + row / kOgC, n - 1);
    ysrc[u] = a.rt + ((b * n + tok) * kOgC + row % kOgC) * sp + kc;
    yoff[u] = row * kOpmKS + kc + (row / kOgC) * kOgTokPad;
  }
  bf16x8 rx[kOgXPT], ry[kOgYPT];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < kOgXPT; ++u) rx[u] = ld8(xsrc[u] + k0);
#pragma unroll
    for (int u = 0; u < kOgYPT; ++u) ry[u] = ld8(ysrc[u] + k0);
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kOgXPT; ++u)
      *reinterpret_cast<bf16x8*>(xs + buf * kOgXB + xoff[u]) = rx[u];
#pragma unroll
    for (int u = 0; u < kOgYPT; ++u)
      *reinterpret_cast<bf16x8*>(ys + buf * kOgYB + yoff[u]) = ry[u];
  };

  // this lane's operand rows: token li / 8 (i; j within each half), channel 8 w + li % 8
  const int ti8 = li >> 3, ch = 8 * wave + (li & 7);
  const int arow = (ti8 * kOgC + ch) * kOpmKS + ti8 * kOgTokPad + 8 * g;
  int brow[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) brow[h] = ((4 * h + ti8) * kOgC + ch) * kOpmKS + (4 * h + ti8) * kOgTokPad + 8 * g;
  f32x16 acc[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) acc[h] = zero16();

  gload(0);
  sstore(0);
  __syncthreads();
  int buf = 0;
#pragma unroll 1
  for (int k0 = 0; k0 < sp; k0 += kOpmKC) {
    const bool more = k0 + kOpmKC < sp;
    if (more) gload(k0 + kOpmKC);
    const bf16* xb = xs + buf * kOgXB;
    const bf16* yb = ys + buf * kOgYB;
#pragma unroll
    for (int kk = 0; kk < kOpmKC; kk += 16) {
      const bf16x8 av = ld8(xb + arow + kk);
#pragma unroll
      for (int h = 0; h < 2; ++h) acc[h] = mfma32(av, ld8(yb + brow[h] + kk), acc[h]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();  // also ends every read of the stages before the products land
    buf ^= 1;
  }

  // the in-group products, fp32, at p (g, k, l) order: acc[h][r] is row acc_row(r, g) =
  // (i = r / 4, k = 4 g + r % 4) of column li = (j = 4 h + li / 8, l = li % 8), group w
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int pair = (r >> 2) * kOgTJ + 4 * h + ti8;
      prod[pair * kOgN + wave * 64 + (4 * g + (r & 3)) * 8 + (li & 7)] = acc[h][r];
    }
  __syncthreads();

  // product norm: wave w normalises pairs 4 w .. 4 w + 3, lane L the products 8 L .. 8 L + 7
  {
    float nw[8], nb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      nw[e] = a.norm_w[8 * lane + e];
      nb[e] = a.norm_b[8 * lane + e];
    }
#pragma unroll 1
    for (int u = 0; u < 4; ++u) {
      const int pair = 4 * wave + u;
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(prod + pair * kOgN + 8 * lane);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(prod + pair * kOgN + 8 * lane + 4);
      float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      float s1 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s1 += x[e];
      const float mean = wave_sum(s1) * (1.f / kOgN);
      float s2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x[e] -= mean;
        s2 += x[e] * x[e];
      }
      const float rstd = __builtin_amdgcn_rsqf(wave_sum(s2) * (1.f / kOgN) + a.norm_eps);
      bf16x8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (bf16)(x[e] * rstd * nw[e] + nb[e]);
      *reinterpret_cast<bf16x8*>(nrm + pair * kOgNS + 8 * lane) = y;
    }
  }
  __syncthreads();

  // output projection: D[f][pair] = W_out[f] . nrm[pair] (A = bf16 weight rows, B = pair rows)
  constexpr int NT = CZ / 32;             // output tiles
  constexpr int KSPLIT = 8 / NT;          // waves per tile (k split)
  constexpr int KW = kOgN / KSPLIT;       // k per wave
  const int ft = wave % NT, kpart = wave / NT;
  const bf16* wrow = a.wp + (int64_t)(32 * ft + li) * kOgN + kpart * KW + 8 * g;
  const bf16* orow = nrm + li * kOgNS + kpart * KW + 8 * g;
  f32x16 acc2 = zero16();
#pragma unroll 4
  for (int k = 0; k < KW; k += 16) acc2 = mfma32(ld8(wrow + k), ld8(orow + k), acc2);
  if (KSPLIT > 1) {
    // (the product rows are no longer read: the partials of waves NT .. 7 go where they were)
    if (kpart > 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((kpart - 1) * NT * 64 + ft * 64 + lane) * 16 + r] = acc2[r];
    }
    __syncthreads();
    if (kpart != 0) return;
#pragma unroll
    for (int w = 1; w < KSPLIT; ++w)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc2[r] += red[((w - 1) * NT * 64 + ft * 64 + lane) * 16 + r];
  }
  const int pair = li;
  const int i = i0 + pair / kOgTJ, j = j0 + pair % kOgTJ;
  if (i >= n || j >= n) return;
  const int64_t off = ((b * n + i) * n + j) * CZ;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int f = 32 * ft + 8 * v + 4 * g;
    const f32x4 bias = *reinterpret_cast<const f32x4*>(a.bias + f);
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = acc2[4 * v + e] + bias[e];
    if (a.res) {
      const bf16x4 r = *reinterpret_cast<const bf16x4*>(a.res + off + f);
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] += (float)r[e];
    }
    store4(a.out + off + f, y[0], y[1], y[2], y[3]);
  }
}
}  // namespace

void launch_opm_count(const OpmCountArgs& a, hipStream_t stream) {
  const unsigned t = (unsigned)((a.n + 31) / 32);
  opm_count<<<dim3(t, t, (unsigned)a.batch), 64, 0, stream>>>(a);
}

void launch_opm_pack(const float* w, bf16* wp, int cz, hipStream_t stream) {
  opm_pack<<<dim3((unsigned)((cz * kOpmK2 + 255) / 256)), 256, 0, stream>>>(w, wp, cz);
}

void launch_opm_contract(const OpmContractArgs& a, hipStream_t stream) {
  const int64_t nt = (a.n + kOpmT - 1) / kOpmT;
  // beyond the default dynamic LDS size: the attribute is set on every launch (cheap, and valid
  // for whichever device is current)
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(opm_contract),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kOpmLds);
  opm_contract<<<dim3((unsigned)(nt * nt * a.batch)), 512, kOpmLds, stream>>>(a);
}

void launch_opm_contract_grouped(const OpmGroupedArgs& a, hipStream_t stream) {
  const int64_t tiles = (int64_t)((a.n + kOgTI - 1) / kOgTI) * ((a.n + kOgTJ - 1) / kOgTJ) * a.batch;
  auto kernel = a.cz == 256 ? opm_contract_grouped<256> : opm_contract_grouped<128>;
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kOgLds);
  kernel<<<dim3((unsigned)tiles), 512, kOgLds, stream>>>(a);
}

}  // namespace ffk
