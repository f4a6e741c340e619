// Triangle multiplicative update (outgoing / incoming) on gfx950.
//
// Three kernels per call (equations: src/foldforge/models/checkpoints/legacy/reference/triangle.py:39-49):
//   1. trimul_project  z -> LN_pair -> A = (x W_l^T) * M * sigmoid(x W_lg^T), B likewise,
//                      written channel-major [B][h][np][np] so that the contraction is a
//                      K-contiguous batched GEMM in both directions (incoming tiles walk
//                      columns of z, which stores A^T).
//   2. trimul_contract P[bh] = X[bh] Y[bh]^T on MFMA: 256 x 256 tiles (trimul_contract256,
//                      64-k stages by LDS DMA, two 64 KB buffers) when the padded width is a
//                      multiple of 256, else 128 x 128 tiles; both stop at the last 32-key
//                      stage holding a real key (the operands are zero past it).
//   3. trimul_output   LN_out(P) W_out^T * sigmoid(LN_pair(z) W_g^T) + z, channel-last.
// Kernels 1 and 3 are persistent and weight-stationary: each wave keeps its 32-channel
// slice of every projection in registers (one load per workgroup), loops over 64-position
// tiles, and stages its results through LDS so that every global store is 16 bytes. A
// projection tile whose pairs are all masked stores zeros without its products.
// The output gate is recomputed from z in kernel 3 (z is read there for the residual
// anyway) instead of being stored: 128 channels of gate would cost 2 x 67 MB of HBM
// traffic at N = 512 against 8.6 GFLOP of MFMA work.
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kPT = 64;      // positions per projection / output tile
constexpr int kPS = kPT + 8;  // LDS row stride of a [channel][position] staging tile
constexpr int kCT = 128;      // contraction output tile
constexpr int kCK = 32;       // contraction k step
constexpr int kCKP = kCK + 8; // LDS row stride of a contraction operand tile

// Persistent: tiles are (batch, row r of the padded grid, 64 positions along s); one
// workgroup of 8 waves per CU. wp rows: [0,h) to_left, [h,2h) to_left_gate, [2h,3h)
// to_right, [3h,4h) to_right_gate. Wave w computes output o = w / 4 (0: A, 1: B) for hidden
// channels 32 (w % 4) .. + 31, holding that slice of the projection and of its gate in
// registers.
// Memory stays busy through the compute: the z tiles stream through a ring of three LDS
// buffers by LDS DMA, two tiles ahead, and the stores of a tile are left in flight (a wave
// only waits for its own DMA pieces, never for its stores).
__global__ __launch_bounds__(512, 2) void trimul_project(
    const bf16* __restrict__ z, const float* __restrict__ maskf, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ wp, bf16* __restrict__ a_out,
    bf16* __restrict__ b_out, int batch, int n, int np, int outgoing, float eps) {
  constexpr int H = 128, NB = 3;
  __shared__ __attribute__((aligned(16))) bf16 zt[NB][kPT * 128];  // raw z, then LN(z) (off128)
  __shared__ __attribute__((aligned(16))) bf16 stage[8][32 * kPS];  // [channel][position]
  __shared__ __attribute__((aligned(16))) float msk[NB][8][kPT];    // token mask m[s0 + t], per wave
  __shared__ float mrw[NB][8];                                      // token mask m[r], per wave
  __shared__ __attribute__((aligned(16))) float lnp[2][H];  // LayerNorm affine
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int o = wave >> 2, cb = wave & 3;  // output (A / B), channel block
  if (tid < 2 * H) lnp[tid / H][tid % H] = (tid < H ? ln_w : ln_b)[tid % H];  // published by the first barrier
  WFrag wv, wgt;
  load_wfrag(wv, wp, 2 * H * o + 32 * cb, li, g);
  load_wfrag(wgt, wp, 2 * H * o + H + 32 * cb, li, g);
  settle(wv);
  settle(wgt);
  const int nsb = np / kPT;
  const int64_t plane = (int64_t)np * np;
  auto valid_of = [&](const TileAt& t) { return t.r < n ? max(0, min(kPT, n - t.blk * kPT)) : 0; };
  // This wave's 2 one-KB pieces (positions 8 wave .. 8 wave + 7) of a tile's z rows and its
  // own copies of the tile's token-mask values m[s0 + t] (one float per lane) and m[r] (lane
  // 0) into ring slot buf; positions past the end re-read a real row (zeroed by the
  // LayerNorm). A tile past the end issues the same transfers for tile 0 (kept so that every
  // wave always has the same number of transfers in flight). The mask travels by LDS DMA
  // like z: an ordinary load here would be a vector load (the DMAs' memory clobbers rule out
  // scalar loads), and waiting for it would drain every transfer in flight.
  auto z_dma = [&](TileAt t, int buf) {
    if (t.b >= batch) t = TileAt{0, 0, 0};
    const int s0 = t.blk * kPT, valid = valid_of(t);
    const bf16* base = z;
    uint32_t stride = 256;  // bytes between consecutive positions
    if (valid > 0) {
      if (outgoing) {
        base = z + (((int64_t)t.b * n + t.r) * n + s0) * 128;
      } else {
        base = z + (((int64_t)t.b * n + s0) * n + t.r) * 128;
        stride = (uint32_t)n * 256;
      }
    }
    const int last = valid > 0 ? valid - 1 : 0;
    const uint32_t dst = lds_addr(&zt[buf][0]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int piece = 2 * wave + u, pos = 4 * piece + (lane >> 4);
      const int pe = pos < last ? pos : last;
      dma16_stream(base, pe * stride + 16 * ((lane & 15) ^ (pos & 15)), dst + 1024 * piece);
    }
    const float* mb = maskf + (int64_t)t.b * np;
    dma4(mb + s0, 4u * lane, lds_addr(&msk[buf][wave][0]));
    if (lane == 0) dma4(mb + t.r, 0u, lds_addr(&mrw[buf][wave]));
  };
  if ((int)blockIdx.x >= batch * np * nsb) return;
  const TileAt stride = tile_at(gridDim.x, nsb, np);
  TileAt cur = tile_at(blockIdx.x, nsb, np);
  TileAt nxt = tile_add(cur, stride, nsb, np);
  TileAt far = tile_add(nxt, stride, nsb, np);
  // Software pipeline, one barrier per tile: after the barrier of tile k a wave issues the
  // fetch of tile k + 2, projects and stores tile k (normalised in the previous step), then
  // normalises tile k + 1 (fetched one step earlier) in its own ring slot, so LayerNorm work
  // overlaps the other waves' MFMAs.
  z_dma(cur, 0);
  z_dma(nxt, 1);
  wait_vm_lds<4>();  // this wave's transfers of the first tile landed
  __syncthreads();
  ln_inplace_swz<kPT, 512>(zt[0], valid_of(cur), lnp[0], lnp[1], eps);
  int buf = 0, k = 0;
#pragma unroll 1
  for (; cur.b < batch; ++k, buf = buf == NB - 1 ? 0 : buf + 1) {
    const int b = cur.b, r = cur.r, s0 = cur.blk * kPT;
    const int nbuf = buf == NB - 1 ? 0 : buf + 1, fbuf = nbuf == NB - 1 ? 0 : nbuf + 1;
    // this wave's transfers of tile + step have landed (issued after them: only the previous
    // tile's 4 stores, none before the first step); the barrier publishes everyone's pieces
    // and normalised rows and retires the previous tile's reads of ring slot fbuf
    if (k == 0)
      wait_vm_lds<0>();
    else
      wait_vm_lds<4>();
    __syncthreads();
    z_dma(far, fbuf);
    const bf16* xh = zt[buf];
    // pair mask m[r] m[s]: lane t holds m[s0 + t]; a tile whose 64 pairs are all real takes
    // the unmasked epilogue, a tile whose pairs are all masked (a padded row, or every
    // position past the real length) is zero without any product
    const float mr = mrw[buf][wave];
    const float ms = msk[buf][wave][lane];
    const bool full = mr == 1.f && __builtin_amdgcn_ballot_w64(ms != 1.f) == 0;
    const bool none = mr == 0.f || __builtin_amdgcn_ballot_w64(ms != 0.f) == 0;
    bf16* st = stage[wave];
    if (none) {
      const bf16x4 zero4 = {};
#pragma unroll
      for (int pt = 0; pt < kPT / 32; ++pt)
#pragma unroll
        for (int m4 = 0; m4 < 4; ++m4)
          *reinterpret_cast<bf16x4*>(&st[li * kPS + pt * 32 + 8 * m4 + 4 * g]) = zero4;
    }
#pragma unroll
    for (int pt = 0; pt < kPT / 32 && !none; ++pt) {
      f32x16 av = zero16(), ag = zero16();
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const bf16x8 x = ld8(&xh[off128(pt * 32 + li, 2 * kk + g)]);
        av = mfma32(x, wv.k[kk], av);
        ag = mfma32(x, wgt.k[kk], ag);
      }
      // D[position][channel]: register q is position pt*32 + acc_row(q, g), lane li channel
      if (full) {
#pragma unroll
        for (int m4 = 0; m4 < 4; ++m4) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (bf16)(av[4 * m4 + e] * sigmoid_scaled(ag[4 * m4 + e]));
          *reinterpret_cast<bf16x4*>(&st[li * kPS + pt * 32 + 8 * m4 + 4 * g]) = v;
        }
      } else {
#pragma unroll
        for (int m4 = 0; m4 < 4; ++m4) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int pa = pt * 32 + 8 * m4 + e;  // uniform; lane group 1 takes pa + 4
            const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ms), pa));
            const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ms), pa + 4));
            const float mk = mr * (g ? m1 : m0);
            v[e] = (bf16)(av[4 * m4 + e] * mk * sigmoid_scaled(ag[4 * m4 + e]));
          }
          *reinterpret_cast<bf16x4*>(&st[li * kPS + pt * 32 + 8 * m4 + 4 * g]) = v;
        }
      }
    }
    // the stage is this wave's own: LDS operations of a wave complete in order
    __builtin_amdgcn_wave_barrier();
    // 32 channels x 64 positions: 4 stores of 16 bytes per lane
    bf16* dst = (o == 0 ? a_out : b_out) + ((int64_t)b * H + 32 * cb) * plane + (int64_t)r * np + s0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int chunk = lane + 64 * u;
      const int c = chunk >> 3, p8 = chunk & 7;
      st16<kNtProject>(dst + (int64_t)c * plane + 8 * p8, ld8(&st[c * kPS + 8 * p8]));
    }
    if (nxt.b < batch) ln_inplace_swz<kPT, 512>(zt[nbuf], valid_of(nxt), lnp[0], lnp[1], eps);
    cur = nxt;
    nxt = far;
    far = tile_add(far, stride, nsb, np);
  }
  wait_vm_lds<0>();  // no LDS write may land after exit
}

// P[bh][i][j] = sum_k X[bh][i][k] * Y[bh][j][k]; all planes [np][np] bf16, np % 128 == 0.
// grid: (np / 128)^2 * batch * h workgroups in one dimension, renumbered so that the tiles
// of a channel plane (which share its X rows and Y rows) run on one XCD and hit one L2;
// block 256 = 2 x 2 waves of 64 x 64.
__global__ __launch_bounds__(256) void trimul_contract(const bf16* __restrict__ X,
                                                       const bf16* __restrict__ Y,
                                                       bf16* __restrict__ P, int np,
                                                       const int* __restrict__ kstages,
                                                       int planes_per_batch) {
  // operand tiles during the k loop, then the output tile [128][kCT + 8] for the stores
  __shared__ __attribute__((aligned(16))) bf16 smem[4 * kCT * kCKP];
  static_assert(kCT * (kCT + 8) <= 4 * kCT * kCKP, "output tile exceeds the operand tiles");
  bf16 (*xs)[kCT * kCKP] = reinterpret_cast<bf16 (*)[kCT * kCKP]>(smem);
  bf16 (*ys)[kCT * kCKP] = reinterpret_cast<bf16 (*)[kCT * kCKP]>(smem + 2 * kCT * kCKP);
  const int nt = np / kCT;
  const uint32_t wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / (nt * nt);
  const int j0 = (int)(wg % nt) * kCT, i0 = (int)((wg / nt) % nt) * kCT;
  const int64_t plane = (int64_t)np * np;
  const bf16* Xb = X + bh * plane + (int64_t)i0 * np;
  const bf16* Yb = Y + bh * plane + (int64_t)j0 * np;
  // k past the batch element's last real key: zero operands, left out
  const int kend = kstages ? min(np, kstages[bh / planes_per_batch] * kCK) : np;
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
  for (int k0 = 0; k0 < kend; k0 += kCK) {
    const bool more = k0 + kCK < kend;
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
      // D[j][i]: lane li is row i, its registers 4 t .. 4 t + 3 columns 8 t + 4 g + 0 .. 3
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(bv[ni], av[mi], acc[mi][ni]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  // the k loop ended with a barrier: the operand tiles are free for the output tile
  constexpr int kOS = kCT + 8;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int i = wm * 64 + mi * 32 + li;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)acc[mi][ni][4 * t + e];
        *reinterpret_cast<bf16x4*>(&smem[i * kOS + wn * 64 + ni * 32 + 8 * t + 4 * g]) = v;
      }
    }
  __syncthreads();
  // 128 rows x 256 bytes: 16-byte stores, 16 lanes per row
  bf16* Pb = P + bh * plane + (int64_t)i0 * np + j0;
#pragma unroll
  for (int u = 0; u < kCT * kCT / 8 / 256; ++u) {
    const int chunk = tid + 256 * u;
    const int row = chunk >> 4, c = chunk & 15;
    st16<kNtContract>(Pb + (int64_t)row * np + 8 * c, ld8(&smem[row * kOS + 8 * c]));
  }
}

// The same product with 256 x 256 output tiles for np % 256 == 0: 8 waves of 128 x 64, the
// operand tiles (256 rows x 64 k of X and of Y, 64 KB a stage) arrive by LDS DMA in two stage
// buffers, one stage ahead, so a plane's operands are read twice rather than four times.
// Operand rows are 128 bytes (whole cache lines per DMA piece: with 32-k stages of 64-byte
// rows the trimul op took 3.5% longer) with their 16-byte pieces XOR-swizzled by (row / 2) % 8,
// so the sixteen rows of an MFMA fragment fetch hit distinct banks. The two buffers then hold
// the output tile for the stores (rows of 512 bytes, pieces swizzled by row % 16).
constexpr int kBT = 256;                    // output tile
constexpr int kBK = 64;                     // k per stage (128-byte operand rows)
constexpr int kBStages = 2;
constexpr int kBStage = 2 * kBT * kBK;      // bf16 per stage (X then Y)
__global__ __launch_bounds__(512, 2) void trimul_contract256(const bf16* __restrict__ X,
                                                             const bf16* __restrict__ Y,
                                                             bf16* __restrict__ P, int np,
                                                             const int* __restrict__ kstages,
                                                             int planes_per_batch) {
  __shared__ __attribute__((aligned(16))) bf16 smem[kBStages * kBStage];  // 128 KB
  static_assert(kBT * kBT <= kBStages * kBStage, "output tile exceeds the ring");
  const int nt = np / kBT;
  const uint32_t wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t bh = wg / (nt * nt);
  const int j0 = (int)(wg % nt) * kBT, i0 = (int)((wg / nt) % nt) * kBT;
  const int64_t plane = (int64_t)np * np;
  const bf16* Xb = X + bh * plane + (int64_t)i0 * np;
  const bf16* Yb = Y + bh * plane + (int64_t)j0 * np;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wm = wave >> 2, wn = wave & 3;  // rows 128 wm .., columns 64 wn ..
  // this wave's 8 one-KB pieces of stage s (pieces 0-31 of X, 32-63 of Y, 8 rows of 128 bytes
  // each: whole cache lines); the 16-byte slot c of row r sits at slot c ^ ((r >> 1) & 7), so
  // the 16 rows of an MFMA fragment read hit distinct banks
  auto stage_dma = [&](int s) {
    const uint32_t base = lds_addr(&smem[(s % kBStages) * kBStage]);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int piece = 8 * wave + u, half = piece >> 5;
      const int row = 8 * (piece & 31) + (lane >> 3);
      const int c = (lane & 7) ^ ((row >> 1) & 7);
      const bf16* src = (half ? Yb : Xb) + s * kBK;
      dma16(src, (uint32_t)(row * np * 2 + 16 * c), base + 1024 * piece);
    }
  };
  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int c = 0; c < 2; ++c) acc[a][c] = zero16();
  // 32-key stages past the batch element's last real key: zero operands, left out (a 64-wide
  // stage may end with one of them)
  const int nk32 = kstages ? min(np / kCK, kstages[bh / planes_per_batch]) : np / kCK;
  const int nk = (nk32 + 1) / 2;
  if (nk > 0) stage_dma(0);
#pragma unroll 1
  for (int s = 0; s < nk; ++s) {
    wait_vm_lds<0>();  // this wave's pieces of stage s landed (nothing later is in flight)
    __syncthreads();   // everyone's pieces of stage s; stage s - 1's slot is free
    if (s + 1 < nk) stage_dma(s + 1);
    const bf16* xs = &smem[(s % kBStages) * kBStage];
    const bf16* ys = xs + kBT * kBK;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8 av[4], bv[2];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const int r = 128 * wm + 32 * mi + li;
        av[mi] = ld8(&xs[r * kBK + 8 * ((2 * kk + g) ^ ((r >> 1) & 7))]);
      }
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int r = 64 * wn + 32 * ni + li;
        bv[ni] = ld8(&ys[r * kBK + 8 * ((2 * kk + g) ^ ((r >> 1) & 7))]);
      }
      // D[j][i]: lane li is row i, its registers 4 t .. 4 t + 3 columns 8 t + 4 g + 0 .. 3
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(bv[ni], av[mi], acc[mi][ni]);
    }
  }
  __syncthreads();  // every wave's last fragment reads are done: the ring holds the output
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const int i = 128 * wm + 32 * mi + li;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)acc[mi][ni][4 * t + e];
        const int c = (64 * wn + 32 * ni + 8 * t) >> 3;  // 16-byte piece of the row
        *reinterpret_cast<bf16x4*>(&smem[i * kBT + 8 * (c ^ (i & 15)) + 4 * g]) = v;
      }
    }
  __syncthreads();
  bf16* Pb = P + bh * plane + (int64_t)i0 * np + j0;
#pragma unroll 4
  for (int u = 0; u < kBT * kBT / 8 / 512; ++u) {
    const int chunk = tid + 512 * u;
    const int row = chunk >> 5, c = chunk & 31;
    st16<kNtContract>(Pb + (int64_t)row * np + 8 * c, ld8(&smem[row * kBT + 8 * (c ^ (row & 15))]));
  }
}

// out[b,i,j,:] = z + (LN_out(P[b,:,i,j]) W_out^T) * sigmoid(LN_pair(z[b,i,j]) W_g^T) over tiles
// of 64 consecutive pairs of one z row. Persistent, one workgroup of 8 waves per CU; wave w
// owns output channels 32 (w & 3) .. + 31 of positions 32 (w >> 2) .. + 31 in both
// projections. z tiles (64 positions x 256 bytes) and P tiles (128 channel rows x 128 bytes)
// arrive by LDS DMA two tiles ahead in three-slot rings. Two barriers per tile, and the
// normalisations run ahead of the products: during tile k the workgroup normalises P of
// tile k (statistics gathered over the two previous phases), projects and stores tile k,
// and for tile k + 1 computes LN(z), the gate and both passes of P's statistics.
__global__ __launch_bounds__(512, 2) void trimul_output(
    const bf16* __restrict__ z, const bf16* __restrict__ P, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const float* __restrict__ lno_w,
    const float* __restrict__ lno_b, const bf16* __restrict__ wg, const bf16* __restrict__ wo,
    bf16* __restrict__ out, int batch, int n, int np, int residual, float eps,
    const float* __restrict__ eps_out_dev) {
  constexpr int H = 128, NB = 3;
  __shared__ __attribute__((aligned(16))) bf16 zs[NB][kPT * 128];  // raw z, then out (off128)
  __shared__ __attribute__((aligned(16))) bf16 ps[NB][H * kPT];    // P, [channel][position]
  __shared__ __attribute__((aligned(16))) bf16 xh[kPT * 128];      // LN(z) (off128)
  __shared__ __attribute__((aligned(16))) bf16 y[kPT * 128];       // LN_out(P) (off128)
  __shared__ float red[2][2][8][kPT];  // [tile parity][sum, centred squares][wave][position]
  __shared__ __attribute__((aligned(16))) float lnp[4][H];  // LN_pair and LN_out affine
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cb = wave & 3, pt = wave >> 2;
  const float* const lsrc[4] = {ln_w, ln_b, lno_w, lno_b};
  lnp[tid >> 7][tid & 127] = lsrc[tid >> 7][tid & 127];  // published by the first barrier
  // the centre norm's epsilon: a device value when the contraction is length-divided
  const float eps_out = eps_out_dev ? *eps_out_dev : eps;
  WFrag fg, fo;
  load_wfrag(fg, wg, 32 * cb, li, g);
  load_wfrag(fo, wo, 32 * cb, li, g);
  settle(fg);
  settle(fo);
  const int njb = (n + kPT - 1) / kPT;
  const int64_t plane = (int64_t)np * np;
  const int ntiles = batch * n * njb;
  auto where = [&](int tile, int& b, int& i, int& j0, int& valid) {
    const int jb = tile % njb;
    i = (tile / njb) % n;
    b = tile / (njb * n);
    j0 = jb * kPT;
    valid = min(kPT, n - j0);
  };
  // This wave's 2 one-KB pieces of the tile's z (positions past the end re-read the last
  // real one) and 2 of its P (8 channel rows each; j0 + 63 < np) into ring slot buf; a tile
  // index past the end fetches tile 0 again, so every wave always has the same number of
  // transfers in flight.
  auto dma = [&](int tile, int buf) {
    int b, i, j0, valid;
    where(tile < ntiles ? tile : 0, b, i, j0, valid);
    const bf16* zb = z + (((int64_t)b * n + i) * n + j0) * 128;
    const uint32_t dz = lds_addr(&zs[buf][0]), dp = lds_addr(&ps[buf][0]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int piece = 2 * wave + u, pos = 4 * piece + (lane >> 4);
      const int pe = pos < valid ? pos : valid - 1;
      dma16_stream(zb, pe * 256 + 16 * ((lane & 15) ^ (pos & 15)), dz + 1024 * piece);
      const bf16* pb = P + ((int64_t)b * H + 8 * piece) * plane + (int64_t)i * np + j0;
      dma16_stream(pb, (uint32_t)((lane >> 3) * plane * 2) + 16 * (lane & 7), dp + 1024 * piece);
    }
  };
  // P statistics of this thread's 16 channels 16 wave .. + 15 at position `lane`; every sum is
  // a tree (these run between the tile's barriers, so their latency is on the tile's path)
  auto p_load = [&](int buf, float (&v)[16]) {
    const bf16* col = &ps[buf][(16 * wave) * kPT + lane];
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = (float)col[e * kPT];
  };
  auto sum16v = [](const float (&v)[16]) {
    float a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = (v[4 * q] + v[4 * q + 1]) + (v[4 * q + 2] + v[4 * q + 3]);
    return (a[0] + a[1]) + (a[2] + a[3]);
  };
  auto red8 = [&](int par, int which) {
    float a[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) a[q] = red[par][which][q][lane];
    return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
  };
  auto p_sum = [&](int buf, int par) {
    float v[16];
    p_load(buf, v);
    red[par][0][wave][lane] = sum16v(v);
  };
  auto p_mean = [&](int par) { return red8(par, 0) * (1.f / H); };
  auto p_centred = [&](int buf, int par) {
    float v[16];
    p_load(buf, v);
    const float mean = p_mean(par);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      v[e] -= mean;
      v[e] *= v[e];
    }
    red[par][1][wave][lane] = sum16v(v);
  };
  // the centre norm's affine for this thread's 16 channels, read once (the first barrier
  // publishes lnp)
  float cn_w[16], cn_b[16];
  auto p_normalise = [&](int buf, int par) {
    float v[16];
    p_load(buf, v);
    const float mean = p_mean(par);
    const float rstd = __builtin_amdgcn_rsqf(red8(par, 1) * (1.f / H) + eps_out);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)((v[8 * h + e] - mean) * rstd * cn_w[8 * h + e] + cn_b[8 * h + e]);
      *reinterpret_cast<bf16x8*>(&y[off128(lane, 2 * wave + h)]) = o;
    }
  };
  const int p0 = 32 * pt + li;  // this lane's position in both products
  // gate: D[channel][position], lane position p0, registers channels 32 cb + 8 j + 4 g + e
  auto gate = [&]() {
    f32x16 ag = zero16();
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) ag = mfma32(fg.k[kk], ld8(&xh[off128(p0, 2 * kk + g)]), ag);
#pragma unroll
    for (int r = 0; r < 16; ++r) ag[r] = sigmoid_scaled(ag[r]);
    return ag;
  };
  const int step = gridDim.x;
  if ((int)blockIdx.x >= ntiles) return;
  dma(blockIdx.x, 0);
  dma(blockIdx.x + step, 1);
  wait_vm_lds<4>();  // this wave's transfers of the first tile landed
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    cn_w[e] = lnp[2][16 * wave + e];
    cn_b[e] = lnp[3][16 * wave + e];
  }
  {
    int b, i, j0, valid;
    where(blockIdx.x, b, i, j0, valid);
    ln_swz<kPT, 512>(zs[0], xh, valid, lnp[0], lnp[1], eps);
    p_sum(0, 0);
  }
  __syncthreads();
  f32x16 sg = gate();
  p_centred(0, 0);
  int buf = 0, k = 0, prev_valid = kPT;
#pragma unroll 1
  for (int tile = blockIdx.x; tile < ntiles; tile += step, ++k, buf = buf == NB - 1 ? 0 : buf + 1) {
    int b, i, j0, valid;
    where(tile, b, i, j0, valid);
    const int nbuf = buf == NB - 1 ? 0 : buf + 1, fbuf = nbuf == NB - 1 ? 0 : nbuf + 1;
    const bool has_next = tile + step < ntiles;
    // this wave's transfers of tile + step have landed (issued after them: the previous
    // tile's 2 stores, fewer for a partial tile); the barrier publishes everyone's pieces,
    // LN(z) and statistics, and retires the previous tile's accesses to ring slot fbuf
    if (k == 0 || prev_valid < kPT)
      wait_vm_lds<0>();
    else
      wait_vm_lds<2>();
    __syncthreads();
    dma(tile + 2 * step, fbuf);
    p_normalise(buf, k & 1);
    if (has_next) {
      int nb, ni, nj0, nvalid;
      where(tile + step, nb, ni, nj0, nvalid);
      ln_swz<kPT, 512>(zs[nbuf], xh, nvalid, lnp[0], lnp[1], eps);
      p_sum(nbuf, (k + 1) & 1);
    }
    __syncthreads();
    {
      f32x16 ao = zero16();
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) ao = mfma32(fo.k[kk], ld8(&y[off128(p0, 2 * kk + g)]), ao);
      bf16* zrow = zs[buf];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x4* pz = reinterpret_cast<bf16x4*>(&zrow[off128(p0, 4 * cb + j) + 4 * g]);
        const bf16x4 zv = *pz;
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)(ao[4 * j + e] * sg[4 * j + e] + (residual ? (float)zv[e] : 0.f));
        *pz = v;
      }
      // the block is this wave's own: LDS operations of a wave complete in order
      __builtin_amdgcn_wave_barrier();
      bf16* dst = out + (((int64_t)b * n + i) * n + j0) * 128;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int chunk = lane + 64 * u;
        const int p = 32 * pt + (chunk >> 2), c = 4 * cb + (chunk & 3);
        if (p < valid)
          st16<kNtOutput>(dst + (int64_t)p * 128 + 8 * c, ld8(&zrow[off128(p, c)]));
      }
    }
    if (has_next) {
      sg = gate();
      p_centred(nbuf, (k + 1) & 1);
    }
    prev_valid = valid;
  }
  wait_vm_lds<0>();  // no LDS write may land after exit
}

static int persistent_grid(int ntiles, int per_cu) {
  return max(1, min(ntiles, cu_count() * per_cu));
}

void launch_trimul(const TrimulArgs& a, hipStream_t stream) {
  const int np = a.np;
  const int tiles_p = a.batch * np * (np / kPT);
  trimul_project<<<persistent_grid(tiles_p, 1), 512, 0, stream>>>(
      a.z, a.maskf, a.ln_w, a.ln_b, a.wp, a.A, a.B, a.batch, a.n, np, a.outgoing, a.eps);
  launch_trimul_contract(a.A, a.B, a.P, (int64_t)a.batch * 128, np, stream, a.kstages, 128);
  const int tiles_o = a.batch * a.n * ((a.n + kPT - 1) / kPT);
  trimul_output<<<persistent_grid(tiles_o, 1), 512, 0, stream>>>(
      a.z, a.P, a.ln_w, a.ln_b, a.lno_w, a.lno_b, a.wg, a.wo, a.out, a.batch, a.n, np,
      a.residual, a.eps, a.eps_out);
}

// eps_out[0] = eps * L^2, L = max(1, the number of positions j < n real in any batch element).
// RoseTTAFold3 divides the contraction by L before the centre LayerNorm
// (src/foldforge/models/checkpoints/legacy/routing.py:33-55 with
// legacy/reference/triangle.py:46-48); LN(P / L) with eps is LN(P) with eps L^2, so the
// kernels keep P as it is and take this epsilon. One workgroup; no host read of L.
__global__ __launch_bounds__(256) void length_eps(const uint8_t* __restrict__ mask, int batch,
                                                  int n, float eps, float* __restrict__ eps_out) {
  __shared__ int total;
  if (threadIdx.x == 0) total = 0;
  __syncthreads();
  int count = 0;
  for (int j = threadIdx.x; j < n; j += 256) {
    bool any = false;
    for (int b = 0; b < batch && !any; ++b) any = mask[(int64_t)b * n + j] != 0;
    count += any ? 1 : 0;
  }
  atomicAdd(&total, count);
  __syncthreads();
  if (threadIdx.x == 0) {
    const float l = (float)(total > 1 ? total : 1);
    eps_out[0] = eps * l * l;
  }
}

void launch_length_eps(const uint8_t* mask, int batch, int n, float eps, float* eps_out,
                       hipStream_t stream) {
  length_eps<<<1, 256, 0, stream>>>(mask, batch, n, eps, eps_out);
}

void launch_trimul_contract(const bf16* A, const bf16* B, bf16* P, int64_t planes, int np,
                            hipStream_t stream, const int* kstages, int planes_per_batch) {
  if (np % kBT == 0) {
    const int64_t nt = np / kBT;
    trimul_contract256<<<dim3((unsigned)(nt * nt * planes)), 512, 0, stream>>>(
        A, B, P, np, kstages, planes_per_batch);
    return;
  }
  const int64_t nt = np / kCT;
  trimul_contract<<<dim3((unsigned)(nt * nt * planes)), 256, 0, stream>>>(A, B, P, np, kstages,
                                                                        planes_per_batch);
}

}  // namespace ffk
