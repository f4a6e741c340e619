// Pair ops at widths other than the fused kernels' (the template stack's 64-channel pair, hidden
// widths of 64 or 256, triangle-attention heads of 16): the shared pieces below, the rest is
// the token-row GEMMs of single.hip, the contraction of trimul.hip and the attention of
// single.hip, composed by api.hip.
#include <algorithm>

#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

namespace {

constexpr int kRowTile = 64;  // tokens per workgroup (consecutive j of one row i)

// Channel planes -> token rows through LDS: workgroup (j tile, i, b) reads the 64-token row
// segment of every channel plane (128 contiguous bytes per channel), then writes the 64 token
// rows of hid channels (contiguous in the output, since the tokens are consecutive).
__global__ __launch_bounds__(256) void planes_to_rows(const bf16* __restrict__ planes,
                                                      bf16* __restrict__ rows, int hid, int n,
                                                      int np) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* t = reinterpret_cast<bf16*>(smem);  // [hid][kRowTile + 2]
  constexpr int kS = kRowTile + 2;          // odd word stride: conflict-free column reads
  const int j0 = blockIdx.x * kRowTile, i = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int64_t gg = (int64_t)np * np;
  const bf16* src = planes + b * hid * gg + (int64_t)i * np + j0;
  // read: thread -> (channel, 8 tokens); kRowTile / 8 = 8 chunks per channel
  for (int idx = threadIdx.x; idx < hid * (kRowTile / 8); idx += 256) {
    const int c = idx >> 3, q = idx & 7;
    const bf16x8 v = ld8(src + (int64_t)c * gg + 8 * q);  // np % 128 == 0: inside the plane
#pragma unroll
    for (int e = 0; e < 8; ++e) t[c * kS + 8 * q + e] = v[e];
  }
  __syncthreads();
  const int valid = min(kRowTile, n - j0);
  bf16* dst = rows + ((b * n + i) * n + j0) * hid;
  // write: consecutive threads take consecutive 8-channel chunks of consecutive tokens
  for (int idx = threadIdx.x; idx < valid * (hid / 8); idx += 256) {
    const int j = idx / (hid / 8), c8 = (idx - j * (hid / 8)) * 8;
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = t[(c8 + e) * kS + j];
    *reinterpret_cast<bf16x8*>(dst + (int64_t)j * hid + c8) = v;
  }
}

// Generic-width triangle multiplication output for pair width 64 and hidden width H (64 or 128):
//   out = z + (LN_out(p) W_out^T) * sigmoid(LN_pair(z) W_g^T)
// with p read straight from the contraction's channel planes, as one streaming kernel (so the
// projection never round-trips through memory). Each workgroup converts both weights to bf16
// once (LDS); every wave then walks tiles of 32 consecutive keys j of one (b, i) on its own,
// loading the next tile's plane segments (H channels x 64 contiguous bytes) and z rows while
// it works on the current one. The plane segments become 32 token rows in a wave-private LDS
// tile; the centre norm reads its statistics from there, then normalises one 8-channel piece
// per k step (hi + lo) into both output tiles, so no token row is held in registers. Lane
// (li, g) owns token li: channels H/2 g .. of p, 32 g .. 32 g + 31 of z. The weight rows are
// stored permuted (row r = 8 v + 4 g + e of output tile t holds channel 32 g + 16 t + 4 v + e),
// so a lane's accumulators hold the output channels of its own z half-row: the two products
// meet each other and z in registers, and the lane writes its 32 output channels as four
// 16-byte pieces.
constexpr int kTmoWaves = 4;
constexpr int kTmoWs = 72;  // LDS row stride of 64-wide rows (elements)
template <int H>
struct __attribute__((aligned(16))) TmoLds {
  bf16 wo[64 * (H + 8)];              // W_out rows (permuted), k = H
  bf16 wg[64 * kTmoWs];               // W_g rows (permuted), k = 64
  bf16 rows[kTmoWaves][32 * (H + 8)];  // per wave: the tile's p as 32 token rows
  float lnow[H], lnob[H], lnw[64], lnb[64];
};

__device__ __forceinline__ int tmo_perm(int row) {
  const int t = row >> 5, r = row & 31;
  return 32 * ((r >> 2) & 1) + 16 * t + 4 * (r >> 3) + (r & 3);
}

template <int H>
__global__ __launch_bounds__(64 * kTmoWaves) void trimul_out_planes(TrimulPlanesArgs a) {
  constexpr int HP = H / 16;  // plane pieces per lane, and 8-channel pieces of a half p row
  constexpr int RS = H + 8;   // LDS row stride of the token rows and the W_out rows
  __shared__ TmoLds<H> lds;
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int idx = tid; idx < 64 * (H / 8); idx += 64 * kTmoWaves) {
    const int row = idx / (H / 8), ch = 8 * (idx % (H / 8));
    *reinterpret_cast<bf16x8*>(lds.wo + row * RS + ch) = cvt8(a.w_out + tmo_perm(row) * H + ch);
  }
  for (int idx = tid; idx < 64 * 8; idx += 64 * kTmoWaves) {
    const int row = idx >> 3, ch = 8 * (idx & 7);
    *reinterpret_cast<bf16x8*>(lds.wg + row * kTmoWs + ch) = cvt8(a.w_gate + tmo_perm(row) * 64 + ch);
  }
  if (tid < H) {
    lds.lnow[tid] = a.lno_w[tid];
    lds.lnob[tid] = a.lno_b[tid];
  }
  if (tid < 64) {
    lds.lnw[tid] = a.ln_w[tid];
    lds.lnb[tid] = a.ln_b[tid];
  }
  __syncthreads();

  const int n = a.n, njt = (n + 31) / 32;
  const int tiles = a.batch * n * njt;
  const int stride = (int)gridDim.x * kTmoWaves;
  int t = (int)blockIdx.x * kTmoWaves + wave;
  if (t >= tiles) return;
  const float eps_out = a.eps_out ? *a.eps_out : a.eps;
  const int64_t gg = (int64_t)a.np * a.np;
  bf16* trow = lds.rows[wave];

  // Tile (b, i, jt): keys j = 32 jt + li. pc: this lane's plane pieces (piece q = lane + 64 u:
  // channel q / 4, keys 8 (q % 4) .. + 7; np % 32 == 0 keeps them inside the plane); zr: z row j
  // (the last real one past n). A tile past the end re-reads the last tile.
  auto fetch = [&](int tile, bf16x8* pc, bf16x8* zr) __attribute__((always_inline)) {
    const int tt = tile < tiles ? tile : tiles - 1;
    const int bi = tt / njt, jt = tt - bi * njt;
    const int b = bi / n, i = bi - b * n;
    const bf16* pl = a.planes + (int64_t)b * H * gg + (int64_t)i * a.np + 32 * jt;
#pragma unroll
    for (int u = 0; u < HP; ++u) {
      const int q = lane + 64 * u;
      pc[u] = ld8(pl + (int64_t)(q >> 2) * gg + 8 * (q & 3));
    }
    const int64_t m = (int64_t)bi * n + min(32 * jt + li, n - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) zr[s] = ld8(a.z + m * 64 + 32 * g + 8 * s);
  };
  auto process = [&](int tile, const bf16x8* pc, const bf16x8* zr) __attribute__((always_inline)) {
    // plane pieces -> token rows (LDS operations of a wave complete in order)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int u = 0; u < HP; ++u) {
      const int q = lane + 64 * u, c = q >> 2, k0 = 8 * (q & 3);
#pragma unroll
      for (int e = 0; e < 8; ++e) trow[(k0 + e) * RS + c] = pc[u][e];
    }
    __builtin_amdgcn_wave_barrier();
    const bf16* prow = trow + li * RS + (H / 2) * g;
    // centre-norm statistics of token li (the row's other half in lane li + 32)
    float s1 = 0.f;
#pragma unroll
    for (int s = 0; s < HP; ++s) {
      const bf16x8 x = ld8(prow + 8 * s);
#pragma unroll
      for (int e = 0; e < 8; ++e) s1 += (float)x[e];
    }
    const float mean = pair_sum(s1) * (1.f / H);
    float s2 = 0.f;
#pragma unroll
    for (int s = 0; s < HP; ++s) {
      const bf16x8 x = ld8(prow + 8 * s);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = (float)x[e] - mean;
        s2 += d * d;
      }
    }
    const float rstd = __builtin_amdgcn_rsqf(pair_sum(s2) * (1.f / H) + eps_out);
    int hb = (H / 2) * g, cb = 32 * g;  // per-channel constants read per tile
    asm volatile("" : "+v"(hb), "+v"(cb));
    f32x16 ay[2] = {zero16(), zero16()}, ag[2] = {zero16(), zero16()};
    // output projection, one normalised 8-channel piece per k step into both output tiles
#pragma unroll
    for (int s = 0; s < HP; ++s) {
      const bf16x8 x = ld8(prow + 8 * s);
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(&lds.lnow[hb + 8 * s]);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(&lds.lnow[hb + 8 * s + 4]);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(&lds.lnob[hb + 8 * s]);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(&lds.lnob[hb + 8 * s + 4]);
      f32x4 y0, y1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y0[e] = ((float)x[e] - mean) * rstd * w0[e] + b0[e];
        y1[e] = ((float)x[4 + e] - mean) * rstd * w1[e] + b1[e];
      }
      bf16x8 hi, lo;
      split8(y0, y1, hi, lo);
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const bf16x8 w8 = ld8(lds.wo + (32 * t2 + li) * RS + (H / 2) * g + 8 * s);
        ay[t2] = mfma32(w8, lo, ay[t2]);
        ay[t2] = mfma32(w8, hi, ay[t2]);
      }
    }
    // gate projection of LN_pair(z)
    {
      float z1 = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) z1 += (float)zr[s][e];
      const float zmean = pair_sum(z1) * (1.f / 64);
      float z2 = 0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = (float)zr[s][e] - zmean;
          z2 += d * d;
        }
      const float zrstd = __builtin_amdgcn_rsqf(pair_sum(z2) * (1.f / 64) + a.eps);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(&lds.lnw[cb + 8 * s]);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(&lds.lnw[cb + 8 * s + 4]);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(&lds.lnb[cb + 8 * s]);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(&lds.lnb[cb + 8 * s + 4]);
        f32x4 y0, y1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          y0[e] = ((float)zr[s][e] - zmean) * zrstd * w0[e] + b0[e];
          y1[e] = ((float)zr[s][4 + e] - zmean) * zrstd * w1[e] + b1[e];
        }
        bf16x8 hi, lo;
        split8(y0, y1, hi, lo);
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const bf16x8 w8 = ld8(lds.wg + (32 * t2 + li) * kTmoWs + 32 * g + 8 * s);
          ag[t2] = mfma32(w8, lo, ag[t2]);
          ag[t2] = mfma32(w8, hi, ag[t2]);
        }
      }
    }
    const int bi = tile / njt, jt = tile - bi * njt;
    const int j = 32 * jt + li;
    const int64_t m = (int64_t)bi * n + j;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      bf16x8 y[2];
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 16 * t2 + 4 * v + e;  // channel within the lane's half
          const float r = a.residual ? (float)zr[c >> 3][c & 7] : 0.f;
          y[v >> 1][4 * (v & 1) + e] =
              (bf16)(ay[t2][4 * v + e] * sigmoid_scaled(-kLog2e * ag[t2][4 * v + e]) + r);
        }
      if (j < n) {
        bf16* dst = a.out + m * 64 + 32 * g + 16 * t2;
        *reinterpret_cast<bf16x8*>(dst) = y[0];
        *reinterpret_cast<bf16x8*>(dst + 8) = y[1];
      }
    }
  };

  if constexpr (H >= 128) {
    // one register buffer (with two, 194 VGPRs left one wave per SIMD and the kernel took 132
    // instead of 98 µs on the Protenix-1 template shape): the next tile's pieces load after the
    // current one, other waves cover the wait
    bf16x8 p0[HP], z0[4];
    fetch(t, p0, z0);
    while (true) {
      process(t, p0, z0);
      t += stride;
      if (t >= tiles) break;
      fetch(t, p0, z0);
    }
  } else {
    // two register buffers used in turn: the next tile's pieces load while the current one is
    // processed
    bf16x8 p0[HP], z0[4], p1[HP], z1[4];
    fetch(t, p0, z0);
    while (true) {
      fetch(t + stride, p1, z1);
      process(t, p0, z0);
      t += stride;
      if (t >= tiles) break;
      fetch(t + stride, p0, z0);
      process(t, p1, z1);
      t += stride;
      if (t >= tiles) break;
    }
  }
}

// Generic-width triangle attention output for pair width 64 and gated width HD (64, 128, 256):
//   out = z + (sigmoid(LN_pair(z) W_g^T + b_g) * o) W_out^T + b_out
// as one streaming kernel (the gate is computed here from z, which the residual reads anyway,
// instead of being stored by the projection and read by the attention core). Same scheme as
// trimul_out_planes64: both weights converted to bf16 once per workgroup; every wave walks
// tiles of 32 consecutive pair positions m on its own, loading the next tile's z and o rows
// while it works on the current one; lane (li, g) holds position li's channels
// 32 g .. 32 g + 31 of z and HD/2 g .. HD/2 g + HD/2 - 1 of o. The gate rows are permuted so
// that a lane's accumulators hold the gate of its own o channels; the gated values are then the
// output product's operand as they stand, and the output rows are permuted so that a lane's
// accumulators hold its own z channels. o is read in the attention's frame: position (b, i, j)
// of z takes o row (b, j, i) for the ending node (transposed).
template <int HD>
struct __attribute__((aligned(16))) TaoLds {
  bf16 wg[HD * kTmoWs];            // gate rows (permuted), k = 64 pair channels
  bf16 wo[64 * (HD + 8)];          // output rows (permuted), k = HD gated channels
  float lnw[64], lnb[64], bg[HD], bo[64];  // bg times -log2(e), as the gate rows
};

template <int HD>
__device__ __forceinline__ int tao_perm(int row, int half) {
  const int t = row >> 5, r = row & 31;
  return half * ((r >> 2) & 1) + 16 * t + 4 * (r >> 3) + (r & 3);
}

template <int HD>
__global__ __launch_bounds__(64 * kTmoWaves) void triattn_out_rows(TriattnRowsArgs a) {
  constexpr int KO = HD / 16;  // 8-channel pieces of a lane's half o row
  constexpr int WOS = HD + 8;
  __shared__ TaoLds<HD> lds;
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int idx = tid; idx < HD * 8; idx += 64 * kTmoWaves) {  // gate: HD rows x 64
    const int row = idx >> 3, ch = 8 * (idx & 7);
    const float* src = a.w_gate + tao_perm<HD>(row, HD / 2) * 64 + ch;
    bf16x8 w;
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = (bf16)(-kLog2e * src[e]);
    *reinterpret_cast<bf16x8*>(lds.wg + row * kTmoWs + ch) = w;
  }
  for (int idx = tid; idx < 64 * (HD / 8); idx += 64 * kTmoWaves) {  // output: 64 rows x HD
    const int row = idx / (HD / 8), ch = 8 * (idx % (HD / 8));
    *reinterpret_cast<bf16x8*>(lds.wo + row * WOS + ch) = cvt8(a.w_out + tao_perm<HD>(row, 32) * HD + ch);
  }
  if (tid < 64) {
    lds.lnw[tid] = a.ln_w[tid];
    lds.lnb[tid] = a.ln_b[tid];
    lds.bo[tid] = a.b_out ? a.b_out[tid] : 0.f;
  }
  if (tid < HD) lds.bg[tid] = a.b_gate ? -kLog2e * a.b_gate[tid] : 0.f;
  __syncthreads();

  const int n = a.n;
  const int64_t rows = (int64_t)a.batch * n * n;
  const int64_t tiles = (rows + 31) / 32;
  const int64_t stride = (int64_t)gridDim.x * kTmoWaves;
  int64_t t = (int64_t)blockIdx.x * kTmoWaves + wave;
  if (t >= tiles) return;

  // the z row and the o row of this lane's position (the last one past the end)
  auto rows_of = [&](int64_t tile, int64_t& mz, int64_t& mo) __attribute__((always_inline)) {
    mz = min(min(tile, tiles - 1) * 32 + li, rows - 1);
    mo = mz;
    if (a.transposed) {
      const int64_t bi = mz / n;
      const int j = (int)(mz - bi * n);
      const int64_t b = bi / n;
      const int i = (int)(bi - b * n);
      mo = (b * n + j) * n + i;
    }
  };
  auto fetch = [&](int64_t tile, bf16x8* zr, bf16x8* orr) __attribute__((always_inline)) {
    int64_t mz, mo;
    rows_of(tile, mz, mo);
#pragma unroll
    for (int s = 0; s < 4; ++s) zr[s] = ld8(a.z + mz * 64 + 32 * g + 8 * s);
#pragma unroll
    for (int s = 0; s < KO; ++s) orr[s] = ld8(a.o + mo * HD + (HD / 2) * g + 8 * s);
  };
  auto process = [&](int64_t tile, const bf16x8* zr, bf16x8* orr) __attribute__((always_inline)) {
    // LayerNorm of z (the row's other 32 channels in lane li + 32) -> bf16 hi / lo
    float s1 = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) s1 += (float)zr[s][e];
    const float mean = pair_sum(s1) * (1.f / 64);
    float s2 = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = (float)zr[s][e] - mean;
        s2 += d * d;
      }
    const float rstd = __builtin_amdgcn_rsqf(pair_sum(s2) * (1.f / 64) + a.eps);
    int cb = 32 * g, hb = (HD / 2) * g;  // read per tile (held, they would take registers)
    asm volatile("" : "+v"(cb), "+v"(hb));
    bf16x8 xh[4], xl[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(&lds.lnw[cb + 8 * s]);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(&lds.lnw[cb + 8 * s + 4]);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(&lds.lnb[cb + 8 * s]);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(&lds.lnb[cb + 8 * s + 4]);
      f32x4 y0, y1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y0[e] = ((float)zr[s][e] - mean) * rstd * w0[e] + b0[e];
        y1[e] = ((float)zr[s][4 + e] - mean) * rstd * w1[e] + b1[e];
      }
      split8(y0, y1, xh[s], xl[s]);
    }
    // gate tiles: gated channel HD/2 g + 16 t + 4 v + e in acc[4 v + e], gated in place in orr
#pragma unroll
    for (int t4 = 0; t4 < HD / 32; ++t4) {
      const bf16* wr = lds.wg + (32 * t4 + li) * kTmoWs + 32 * g;
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 w8 = ld8(wr + 8 * s);
        acc = mfma32(w8, xl[s], acc);
        acc = mfma32(w8, xh[s], acc);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const f32x4 gb = *reinterpret_cast<const f32x4*>(&lds.bg[hb + 16 * t4 + 4 * v]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 16 * t4 + 4 * v + e;  // channel within the lane's half
          orr[c >> 3][c & 7] = (bf16)(sigmoid_scaled(acc[4 * v + e] + gb[e]) * (float)orr[c >> 3][c & 7]);
        }
      }
    }
    // output tiles: pair channel 32 g + 16 t + 4 v + e, plus the bias and the residual
    const int64_t m = tile * 32 + li;
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      const bf16* wr = lds.wo + (32 * t2 + li) * WOS + (HD / 2) * g;
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < KO; ++s) acc = mfma32(ld8(wr + 8 * s), orr[s], acc);
      bf16x8 y[2];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const f32x4 ob = *reinterpret_cast<const f32x4*>(&lds.bo[cb + 16 * t2 + 4 * v]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 16 * t2 + 4 * v + e;
          const float r = a.residual ? (float)zr[c >> 3][c & 7] : 0.f;
          y[v >> 1][4 * (v & 1) + e] = (bf16)(acc[4 * v + e] + ob[e] + r);
        }
      }
      if (m < rows) {
        bf16* dst = a.out + m * 64 + 32 * g + 16 * t2;
        *reinterpret_cast<bf16x8*>(dst) = y[0];
        *reinterpret_cast<bf16x8*>(dst + 8) = y[1];
      }
    }
  };

  if constexpr (HD >= 128) {
    // one register buffer (the o rows of 128 / 256 gated channels take 32 / 64 VGPRs a buffer;
    // with two, the kernel took 124 / 189 instead of 85 / 135 µs on the Protenix-1 / RoseTTAFold3
    // template shapes): the next tile's rows load after the current one, other waves cover the wait
    bf16x8 z0[4], o0[KO];
    fetch(t, z0, o0);
    while (true) {
      process(t, z0, o0);
      t += stride;
      if (t >= tiles) break;
      fetch(t, z0, o0);
    }
  } else {
    // two register buffers used in turn: the next tile's rows load while the current one is
    // processed
    bf16x8 z0[4], o0[KO], z1[4], o1[KO];
    fetch(t, z0, o0);
    while (true) {
      fetch(t + stride, z1, o1);
      process(t, z0, o0);
      t += stride;
      if (t >= tiles) break;
      fetch(t + stride, z0, o0);
      process(t, z1, o1);
      t += stride;
      if (t >= tiles) break;
    }
  }
}

}  // namespace

// out[b][i][j][:] = (base ? base[b][i][j][:] : 0) + t[b][j][i][:]: one thread per 8 channels
// of one output position, so every read and write is 16 contiguous bytes and each output
// entry is read (from base) and written by the same thread (base may be out).
__global__ __launch_bounds__(256) void pair_add_transposed(const bf16* base,
                                                           const bf16* __restrict__ t, bf16* out,
                                                           int64_t batch, int n, int c) {
  const int c8 = c / 8;
  const int64_t nn = (int64_t)n * n, total = batch * nn * c8;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * 256) {
    const int64_t pos = idx / c8;
    const int ch = (int)(idx - pos * c8) * 8;
    const int64_t b = pos / nn, r = pos - b * nn;
    const int i = (int)(r / n), j = (int)(r - (int64_t)i * n);
    const bf16x8 tv = ld8(t + ((b * n + j) * n + i) * c + ch);
    bf16x8 y;
    if (base) {
      const bf16x8 bv = ld8(base + pos * c + ch);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = (bf16)((float)bv[e] + (float)tv[e]);
    } else {
      y = tv;
    }
    *reinterpret_cast<bf16x8*>(out + pos * c + ch) = y;
  }
}

void launch_planes_to_rows(const bf16* planes, bf16* rows, int batch, int hid, int n, int np,
                           hipStream_t stream) {
  const size_t lds = (size_t)hid * (kRowTile + 2) * sizeof(bf16);
  if (lds > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(planes_to_rows),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  planes_to_rows<<<dim3((unsigned)((n + kRowTile - 1) / kRowTile), (unsigned)n, (unsigned)batch),
                   256, lds, stream>>>(planes, rows, hid, n, np);
}

void launch_trimul_out_planes(const TrimulPlanesArgs& a, hipStream_t stream) {
  const int64_t tiles = (int64_t)a.batch * a.n * ((a.n + 31) / 32);
  const int64_t blocks = std::min<int64_t>((tiles + kTmoWaves - 1) / kTmoWaves, (int64_t)cu_count() * 6);
  const dim3 grid((unsigned)std::max<int64_t>(1, blocks));
  if (a.hid == 128)
    trimul_out_planes<128><<<grid, 64 * kTmoWaves, 0, stream>>>(a);
  else
    trimul_out_planes<64><<<grid, 64 * kTmoWaves, 0, stream>>>(a);
}

void launch_triattn_out_rows(const TriattnRowsArgs& a, hipStream_t stream) {
  const int64_t tiles = ((int64_t)a.batch * a.n * a.n + 31) / 32;
  const int64_t blocks = std::min<int64_t>((tiles + kTmoWaves - 1) / kTmoWaves, (int64_t)cu_count() * 6);
  const dim3 grid((unsigned)std::max<int64_t>(1, blocks));
  if (a.hd == 256)
    triattn_out_rows<256><<<grid, 64 * kTmoWaves, 0, stream>>>(a);
  else if (a.hd == 128)
    triattn_out_rows<128><<<grid, 64 * kTmoWaves, 0, stream>>>(a);
  else
    triattn_out_rows<64><<<grid, 64 * kTmoWaves, 0, stream>>>(a);
}

void launch_pair_add_transposed(const bf16* base, const bf16* t, bf16* out, int64_t batch, int n,
                                int c, hipStream_t stream) {
  const int64_t total = batch * n * n * (c / 8);
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = (int64_t)cu_count() * 16;
  blocks = blocks < 1 ? 1 : blocks > cap ? cap : blocks;
  pair_add_transposed<<<dim3((unsigned)blocks), 256, 0, stream>>>(base, t, out, batch, n, c);
}

}  // namespace ffk
