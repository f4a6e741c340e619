// Triangle attention around the starting / ending node on gfx950.
//
// Equations: src/foldforge/models/checkpoints/legacy/attention.py:108-163 with the masked
// softmax of legacy/reference/attention.py:77-100. Three kernels per call:
//   1. triattn_project  z -> LN_pair -> q (scaled by d^-1/2 log2 e), k, v^T and the pair
//                       bias (log2 e scaled, fp32, -inf at masked keys). A tile is 128
//                       positions along one attention row: a row of z (starting) or a
//                       column of z (ending), so the q / k / v^T stores are contiguous. The
//                       bias is written in the flash kernel's register order (below).
//   2. flash_attn_bias  the attention core; the N^3 H logits never leave registers.
//   3. triattn_output   out = z + (sigmoid(LN_pair(z) W_g^T) * o) W_out^T.
// The gate is recomputed from z in kernel 3 rather than stored (z is read there for the
// residual anyway).
//
// Flash core (one wave = 32 queries of up to 4 attention rows; 4 waves per workgroup, two
// workgroups per CU):
//  * S^T (32 keys x 32 queries) is one MFMA accumulator. Its initial value is the pair-bias
//    tile (fp32, stored by kernel 1 in the accumulator's register order), shared by the 4
//    attention rows of the workgroup (the bias does not depend on the row).
//  * Offsets without a running maximum: one offset m per query, shared by the wave's 4 rows,
//    is the largest bias of the first key tile (computed before the loop from the bias alone,
//    so padded rows cannot change a valid row's rounding). It is subtracted from the bias
//    tile once per key block (the accumulator's initial value), so the common key loop has
//    no per-logit work beyond two MFMAs, exp2, bf16 packing and a v_dot2 row sum, and one
//    test of the partial sums per pair of rows. A tile whose partial sum reaches 2^64 gives
//    its row an extra offset (the tile maximum, rounded up to bf16) and rescales the row's
//    l and O: the lazy form of a running maximum, paid only where logits outgrow the offset
//    (large q . k), and the extra offset then enters the row's S accumulation through one
//    more MFMA with constant operands. A row whose final sum still leaves [2^-100, 2^100]
//    (every logit far below the offset) is recomputed exactly at the end with a two-pass
//    softmax (true maximum first).
//  * Every operand tile reaches LDS by LDS DMA (no registers, no VALU): K and V^T of the 4
//    rows in stages of 32 keys (double-buffered, shared by the 4 waves) and each wave's bias
//    tiles (double-buffered), all one step ahead, with explicit waits on the wave's own
//    transfers. V^T is stored by kernel 1 blocked by 32 keys, with the keys of each 16-key
//    group permuted (0-3, 8-11, 4-7, 12-15), so that a lane's 8 keys of the P V product are
//    one 16-byte read.
//  * Each lane owns one query; P^T comes out of the S^T accumulator already in the
//    B-operand order of the P V product.
#include <math.h>

#include <type_traits>

#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kFR = 4;      // attention rows per flash workgroup (share the bias tile)
constexpr int kFW = 4;      // waves per flash workgroup, 32 queries each (two workgroups per
                            // CU: the waves sharing a SIMD belong to different workgroups, so
                            // their barriers do not hold them in step)
constexpr int kFK = 32;     // keys per LDS stage
constexpr float kSumHigh = 1.2676506002282294e30f;  // 2^100
constexpr float kSumLow = 7.888609052210118e-31f;    // 2^-100
constexpr float kSumRescale = 1.8446744073709552e19f; // 2^64: a tile's partial sum that raises m

constexpr int kPT = 64;        // positions per projection / output tile

// Persistent, weight-stationary, one barrier per tile. Tiles are (batch, row r of the padded
// grid, 64 positions along the attention row). Waves 0-3 hold the query and key rows of
// head w, waves 4-7 the value rows of head w - 4; waves 4 and 5 also project the pair bias
// of the tile's first and second 32 positions (4 heads padded to 32 rows). The z tiles
// arrive by LDS DMA two tiles ahead in a three-slot ring and are normalised in place one
// tile ahead, so the LayerNorm and the loads overlap the MFMAs and stores of other waves.
// Each wave stages its outputs in LDS of its own and writes 16 bytes per lane: q and k as
// 64-byte position rows, v^T as 128-byte runs of the 64 positions of one channel.
__global__ __launch_bounds__(512, 2) void triattn_project(
    const bf16* __restrict__ z, const float* __restrict__ maskf, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ wqkv, const bf16* __restrict__ wb,
    bf16* __restrict__ qo, bf16* __restrict__ ko, bf16* __restrict__ vto, float* __restrict__ bo,
    int batch, int n, int np, int starting, int transposed_bias, float eps) {
  constexpr int NB = 3, H = 4;
  __shared__ __attribute__((aligned(16))) bf16 zt[NB][kPT * 128];  // raw z, then LN(z) (off128)
  __shared__ __attribute__((aligned(16))) bf16 sqk[4][32 * 32];    // [position][d], q then k
  __shared__ __attribute__((aligned(16))) bf16 svt[4][32 * kPT];   // [d][key slot]
  __shared__ __attribute__((aligned(16))) float keep[NB][kPT];     // key mask per position
  __shared__ __attribute__((aligned(16))) bf16 wbl[H * 128];       // the pair-bias rows
  __shared__ __attribute__((aligned(16))) float lnp[2][128];        // LayerNorm affine
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool qk = wave < 4;
  const int head = wave & 3;
  if (tid < 256) lnp[tid >> 7][tid & 127] = (tid < 128 ? ln_w : ln_b)[tid & 127];
  for (int e = tid; e < H * 128; e += 512) wbl[e] = wb[e];  // published by the first barrier
  WFrag w0, w1;
  load_wfrag(w0, wqkv, qk ? 32 * head : 256 + 32 * head, li, g);
  settle(w0);
  if (qk) {
    load_wfrag(w1, wqkv, 128 + 32 * head, li, g);
    settle(w1);
  }
  // The bias entry at tile position t is (query r, key s0 + t), except for the AF3 ending
  // node (bias from the un-transposed pair), where it is (query s0 + t, key r).
  const bool key_major = !starting && !transposed_bias;
  const int nsb = np / kPT;
  const int64_t nb = np / 32;
  const int ntiles = batch * np * nsb;
  auto where = [&](int tile, int& b, int& r, int& s0, int& valid) {
    const int sb = tile % nsb;
    r = (tile / nsb) % np;
    b = tile / (nsb * np);
    s0 = sb * kPT;
    valid = (r < n) ? max(0, min(kPT, n - s0)) : 0;
  };
  // This wave's 2 one-KB pieces (positions 8 wave .. 8 wave + 7) of a tile's z rows into ring
  // slot buf (positions past the end re-read a real row, zeroed by the LayerNorm); wave 7
  // also fetches the tile's 64 key-mask values. A tile index past the end fetches tile 0
  // again, so that every wave always has the same number of transfers in flight.
  auto z_dma = [&](int tile, int buf) {
    int b, r, s0, valid;
    where(tile < ntiles ? tile : 0, b, r, s0, valid);
    const bf16* base = z;
    uint32_t stride = 256;  // bytes between consecutive positions
    if (valid > 0) {
      if (starting) {
        base = z + (((int64_t)b * n + r) * n + s0) * 128;
      } else {
        base = z + (((int64_t)b * n + s0) * n + r) * 128;
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
    if (wave == 7) {
      const float* mrow = maskf + (int64_t)b * np + (key_major ? r : s0);
      dma4(mrow, key_major ? 0u : 4u * lane, lds_addr(&keep[buf][0]));
    }
  };
  const int step = gridDim.x;
  if ((int)blockIdx.x >= ntiles) return;
  z_dma(blockIdx.x, 0);
  z_dma(blockIdx.x + step, 1);
  if (wave == 7)
    wait_vm_lds<3>();  // this wave's transfers of the first tile landed
  else
    wait_vm_lds<2>();
  __syncthreads();
  {
    int b, r, s0, valid;
    where(blockIdx.x, b, r, s0, valid);
    ln_inplace_swz<kPT, 512>(zt[0], valid, lnp[0], lnp[1], eps);
  }
  const int sw = (li >> 2) & 3;  // 16-byte column swizzle of a staged q / k row
  const int swv = (li >> 1) & 7;  // of a staged v^T row
  int buf = 0, k = 0;
#pragma unroll 1
  for (int tile = blockIdx.x; tile < ntiles; tile += step, ++k, buf = buf == NB - 1 ? 0 : buf + 1) {
    int b, r, s0, valid;
    where(tile, b, r, s0, valid);
    const int nbuf = buf == NB - 1 ? 0 : buf + 1, fbuf = nbuf == NB - 1 ? 0 : nbuf + 1;
    // this wave's transfers of tile + step have landed (issued after them: only the previous
    // tile's stores, 8 on waves 0-5 and 4 on waves 6-7); the barrier publishes everyone's
    // pieces and normalised rows and retires the previous tile's reads of ring slot fbuf
    if (k == 0)
      wait_vm_lds<0>();
    else if (wave < 6)
      wait_vm_lds<8>();
    else
      wait_vm_lds<4>();
    __syncthreads();
    z_dma(tile + 2 * step, fbuf);
    const bf16* xh = zt[buf];
    const int64_t bh = (int64_t)b * H + head;
    if (qk) {
      bf16* st = sqk[head];
      bf16* qd = qo + ((bh * np + r) * np + s0) * 32;
      bf16* kd = ko + ((bh * np + r) * np + s0) * 32;
#pragma unroll
      for (int pt = 0; pt < kPT / 32; ++pt) {
        f32x16 aq = zero16(), ak = zero16();
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const bf16x8 x = ld8(&xh[off128(pt * 32 + li, 2 * kk + g)]);
          aq = mfma32(w0.k[kk], x, aq);  // D[d][position]: lane position li, register d
          ak = mfma32(w1.k[kk], x, ak);
        }
#pragma unroll
        for (int which = 0; which < 2; ++which) {
          const f32x16& acc = which ? ak : aq;
          // d = 8 j + 4 g + e: row li, 16-byte column j (swizzled), 8 bytes at 4 g
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            bf16x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (bf16)acc[4 * j + e];
            *reinterpret_cast<bf16x4*>(&st[li * 32 + 8 * (j ^ sw) + 4 * g]) = v;
          }
          // the stage is this wave's own: LDS operations of a wave complete in order
          __builtin_amdgcn_wave_barrier();
          bf16* dst = (which ? kd : qd) + pt * 32 * 32;
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int chunk = lane + 64 * u;
            const int p = chunk >> 2, c = chunk & 3;
            st16<kNtProject>(dst + p * 32 + 8 * c, ld8(&st[p * 32 + 8 * (c ^ ((p >> 2) & 3))]));
          }
          __builtin_amdgcn_wave_barrier();
        }
      }
    } else {
      bf16* st = svt[head];
#pragma unroll
      for (int pt = 0; pt < kPT / 32; ++pt) {
        f32x16 av = zero16();
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
          av = mfma32(ld8(&xh[off128(pt * 32 + li, 2 * kk + g)]), w0.k[kk], av);  // D[position][d]
        // position 8 j + 4 g + e sits at key slot 16 (j >> 1) + 8 g + 4 (j & 1) + e: row d = li,
        // 16-byte column 4 pt + 2 (j >> 1) + g (swizzled), 8 bytes at 4 (j & 1)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (bf16)av[4 * j + e];
          const int c = 4 * pt + 2 * (j >> 1) + g;
          *reinterpret_cast<bf16x4*>(&st[li * kPT + 8 * (c ^ swv) + 4 * (j & 1)]) = v;
        }
        if (wave == 4 + pt) {
          f32x16 ab = zero16();
          const bf16x8 zero8 = {};
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) {
            const bf16x8 wrow = li < H ? ld8(&wbl[li * 128 + 16 * kk + 8 * g]) : zero8;
            ab = mfma32(wrow, ld8(&xh[off128(pt * 32 + li, 2 * kk + g)]), ab);
          }
          // D[head][position]: heads are rows 0..3 = registers 0..3 of lane group 0
          const float kp = keep[buf][pt * 32 + li];
          const int64_t s = s0 + pt * 32 + li;
          const int64_t query = key_major ? s : r;
          const int64_t key = key_major ? r : s;
          if (g == 0) {
#pragma unroll
            for (int q = 0; q < H; ++q)
              bo[bias_index((int64_t)b * H + q, nb, query, key)] = kp != 0.f ? ab[q] : -INFINITY;
          }
        }
      }
      __builtin_amdgcn_wave_barrier();
      // 32 rows of d x 64 key slots = two key blocks of [32 d][32 keys] (v^T blocked by 32 keys:
      // each block 2 contiguous KB)
      bf16* vd = vto + ((bh * np + r) * 32) * np + s0 * 32;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int chunk = lane + 64 * u;
        const int d = chunk >> 3, c = chunk & 7;
        st16<kNtProject>(vd + (c >> 2) * 1024 + d * 32 + 8 * (c & 3),
                         ld8(&st[d * kPT + 8 * (c ^ ((d >> 1) & 7))]));
      }
    }
    if (tile + step < ntiles) {
      int nb2, nr, ns0, nvalid;
      where(tile + step, nb2, nr, ns0, nvalid);
      ln_inplace_swz<kPT, 512>(zt[nbuf], nvalid, lnp[0], lnp[1], eps);
    }
  }
  wait_vm_lds<0>();  // no LDS write may land after exit
}

// DQ = head width / 16 (1: 16-wide heads, 2: 32-wide heads, 4: 64-wide heads). 64-wide heads
// take 2 attention rows per workgroup (the stage buffers of 4 would halve the occupancy); a stage
// then carries as many K / V^T pieces and MFMAs as a 32-wide one of 4 rows.
template <int DQ>
constexpr int flash_rows() { return DQ == 4 ? 2 : kFR; }
template <int DQ>
struct __attribute__((aligned(16))) FlashLds {
  static constexpr int FR = flash_rows<DQ>();
  bf16 k[2][FR][kFK * 16 * DQ];  // [key][d], 16-byte pieces at koff
  bf16 v[2][FR][16 * DQ * kFK];  // [d][key], 16-byte pieces at voff
  float bias[kFW][2][1024];      // per wave, two bias tiles (the blocked layout, copied as is)
};

// Element offsets of 16-byte piece p of K row `key` (2 DQ pieces: 32 DQ bytes, 8 / DQ rows
// fill the 64 banks) and of V^T row d (4 pieces of a 32-key stage), XOR-swizzled so that the
// MFMA operand reads of 16 consecutive rows hit distinct banks.
template <int DQ>
__device__ __forceinline__ int koff(int key, int p) {
  constexpr int sh = DQ == 1 ? 3 : DQ == 2 ? 2 : 1;
  return key * 16 * DQ + 8 * (p ^ ((key >> sh) & (2 * DQ - 1)));
}
__device__ __forceinline__ int voff(int d, int p) { return d * kFK + 8 * (p ^ ((d >> 2) & 3)); }

// exp2 of the 32 logits a lane holds for its query, packed into the bf16 P^T operands of
// the P V product; returns the lane's partial row sum (v_dot2 over the packed pairs).
__device__ __forceinline__ float exp_pack(const f32x16& S, bf16x8& p0, bf16x8& p1) {
  const bf16x2 ones = {(bf16)1.f, (bf16)1.f};
  float ts = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const bf16x2 a = {(bf16)fast_exp2(S[i]), (bf16)fast_exp2(S[i + 1])};
    const bf16x2 c = {(bf16)fast_exp2(S[i + 8]), (bf16)fast_exp2(S[i + 9])};
    p0[i] = a[0];
    p0[i + 1] = a[1];
    p1[i] = c[0];
    p1[i + 1] = c[1];
    ts = __builtin_amdgcn_fdot2_f32_bf16(a, ones, ts, false);
    ts = __builtin_amdgcn_fdot2_f32_bf16(c, ones, ts, false);
  }
  return ts;
}

// Scheduling of one pipelined region of the flash stage: its NR operand reads from LDS first,
// then NM times one MFMA followed by NV VALU instructions (the exponentials, packing and sums
// of the other row pair).
template <int NR, int NM, int NV>
__device__ __forceinline__ void flash_interleave() {
  __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
  }
}

// grid (ceil(np / 128) * (rows / FR) * batch * heads) workgroups, renumbered per XCD;
// block 256 = 4 waves x 32 queries, FR attention rows. GATED: the output is og = gate * o,
// else o (bf16 either way).
template <int DQ, bool GATED>
__global__ __launch_bounds__(256, 2) void flash_attn_bias(FlashArgs a) {
  constexpr int D = 16 * DQ;            // head width
  constexpr int FR = flash_rows<DQ>();  // attention rows of the workgroup
  constexpr int DH = DQ == 4 ? 2 : 1;   // 32-row halves of V^T (and of O^T)
  __shared__ FlashLds<DQ> lds;
  const int64_t np = a.np, rows = a.rows;
  const int heads = a.heads;
  const uint32_t nqb = (uint32_t)((np + 32 * kFW - 1) / (32 * kFW));
  const uint32_t nrg = (uint32_t)(rows / FR);
  const uint32_t total = gridDim.x;
  const uint32_t wg = xcd_remap(blockIdx.x, total);
  const uint32_t qb = wg % nqb;
  const uint32_t rg = (wg / nqb) % nrg;
  const int64_t bh = wg / (nqb * nrg);
  const int64_t j0 = (int64_t)qb * 32 * kFW;
  const int64_t r0 = (int64_t)rg * FR;
  if (r0 >= a.rows_valid || j0 >= a.n_valid) return;  // whole workgroup outside the output
  const int64_t bidx = bh / heads;
  const int h = (int)(bh % heads);
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int dl = DQ == 1 ? li & 15 : li;  // V^T row (of each half) of this lane (16-wide heads: rows repeat)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t jw = j0 + 32 * wave;  // first query of this wave
  const bool active = jw < np;        // the last query block may be partial
  const int64_t j = jw + li;
  const int64_t nb = np / 32;
  const int64_t nstage = np / kFK;
  // key stages past the batch element's last real key hold bias -inf only: exp2 gives exact
  // zeros there, so leaving them out changes no bit of l or O
  const int64_t nrun =
      a.kstages ? min(nstage, ((int64_t)a.kstages[bidx] * 32 + kFK - 1) / kFK) : nstage;

  // Transfers (each one 1 KB LDS DMA per wave): stage s of K / V^T = 2 FR DQ pieces, FR DQ / 2
  // per wave (piece P = (FR DQ / 2) wave + u: K pieces first, DQ per row, each 32 / DQ keys;
  // then V^T pieces, DQ per row, each 16 rows d); bias tile kb of this wave = 4 pieces. Past the
  // last stage / tile a transfer repeats a real one into a buffer that is no longer read, so
  // every wave always has the same transfers in flight.
  const bf16* kbase = a.k + (bh * rows + r0) * np * D;
  const bf16* vbase = a.vt + (bh * rows + r0) * D * np;
  const uint32_t k_lds = lds_addr(&lds.k[0][0][0]), v_lds = lds_addr(&lds.v[0][0][0]);
  auto kv_dma = [&](int64_t s, int buf) {
    const int64_t key0 = (s < nstage ? s : nstage - 1) * kFK;
    constexpr int PW = FR * DQ / 2;  // pieces per wave
#pragma unroll
    for (int u = 0; u < PW; ++u) {
      const int P = PW * wave + u;  // wave-uniform
      if (P < FR * DQ) {
        const int rr = P / DQ, i = P % DQ;
        const int key = (32 / DQ) * i + lane / (2 * DQ);
        const int p = (lane % (2 * DQ)) ^ ((key >> (DQ == 1 ? 3 : DQ == 2 ? 2 : 1)) & (2 * DQ - 1));
        dma16(kbase, (uint32_t)((((int64_t)rr * np + key0 + key) * D + 8 * p) * 2),
              k_lds + (uint32_t)(((buf * FR + rr) * kFK * D + 512 * i) * 2));
      } else {
        const int rr = (P - FR * DQ) / DQ, i = (P - FR * DQ) % DQ;
        // (v^T blocked by 32 keys: the stage's 16 rows d are one contiguous KB)
        const int d = 16 * i + (lane >> 2), p = (lane & 3) ^ ((d >> 2) & 3);
        dma16(vbase, (uint32_t)(((int64_t)rr * D * np + key0 * D + d * 32 + 8 * p) * 2),
              v_lds + (uint32_t)(((buf * FR + rr) * D * kFK + 16 * i * kFK) * 2));
      }
    }
  };
  const float* bias_w = a.bias + (bh * nb + (active ? jw / 32 : 0)) * nb * 1024;
  const uint32_t b_lds = lds_addr(&lds.bias[wave][0][0]);
  auto bias_dma = [&](int64_t kb) {
    const int64_t kt = kb < nb ? kb : nb - 1;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dma16(bias_w, (uint32_t)((kt * 1024 + 256 * i + 4 * lane) * 4),
            b_lds + (uint32_t)(((kb & 1) * 1024 + 256 * i) * 4));
  };

  kv_dma(0, 0);
  bias_dma(0);
  bf16x8 qa[FR][DQ];
  float l[FR];
  f32x16 O[FR][DH];
  const bf16x8 zero8 = {};
#pragma unroll
  for (int rr = 0; rr < FR; ++rr) {
#pragma unroll
    for (int f = 0; f < DQ; ++f)
      qa[rr][f] = active ? ld8(a.q + ((bh * rows + r0 + rr) * np + j) * D + 16 * f + 8 * g) : zero8;
    l[rr] = 0.f;
#pragma unroll
    for (int h = 0; h < DH; ++h) O[rr][h] = zero16();
  }
  // the q loads complete here, not inside the key loop (see settle)
#pragma unroll
  for (int rr = 0; rr < FR; ++rr)
#pragma unroll
    for (int f = 0; f < DQ; ++f) asm volatile("" ::"v"(qa[rr][f]));
  wait_vm_lds<0>();
  __syncthreads();

  // Offsets. Each query starts from one offset shared by the wave's rows: the largest bias of
  // its first key tile (0 when that tile is fully masked), subtracted from the bias tile once
  // per stage, so the key loop needs no subtraction of its own. A tile whose partial sum
  // reaches 2^64 (logits more than 64 log2 units above the offset, e.g. large q.k) gives that
  // row an extra offset of its own: the tile's maximum rounded up to bf16, while the row's
  // l and O so far are scaled down by the increase and the tile is recomputed (a uniform
  // branch the common case never takes). From then on the extra offset enters the row's S
  // accumulation through one more MFMA with constant operands (A: 1 at k = 0 of every key
  // row; B: minus the offset at k = 0 of the lane's query). Every offset depends on the row's
  // and query's own logits, so no row of the workgroup (a padded one included) changes another
  // row's rounding.
  float msh = 0.f;
  if (active) {
    const float* bt = &lds.bias[wave][0][4 * lane];
    float tm = -INFINITY;
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(bt + 256 * v4);
#pragma unroll
      for (int e = 0; e < 4; ++e) tm = fmaxf(tm, x[e]);
    }
    tm = pair_max(tm);
    msh = tm > -INFINITY ? tm : 0.f;
  }
  const bf16x8 ones8 = g == 0 ? bf16x8{(bf16)1.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f} : zero8;
  bf16x8 moff[FR];  // minus the row's extra offset at k = 0 of this lane's query (half 1: zeros)
  float xoff[FR];   // the extra offset (a bf16 value), the same in both lanes of a query
#pragma unroll
  for (int rr = 0; rr < FR; ++rr) {
    moff[rr] = zero8;
    xoff[rr] = 0.f;
  }

  // One stage; XOFF: with the rows' extra offsets. The key loop runs without them until some
  // row of the wave needs one (never, for moderate logits), then with them to the end: two
  // straight loops rather than a test per row and tile.
  bool xrows = false;  // some row of the wave has an extra offset (wave-uniform)
  auto stage = [&](int64_t st, auto xo) {
    constexpr bool XOFF = decltype(xo)::value;
    const int sb = (int)(st & 1);
    // this wave's bias tile st and everyone's K / V^T stage st have landed (waited for and
    // published at the end of the last stage)
    wait_vm_lds<0>();
    f32x16 bcur;
    {
      const float* bt = &lds.bias[wave][st & 1][4 * lane];
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(bt + 256 * v4);
#pragma unroll
        for (int e = 0; e < 4; ++e) bcur[4 * v4 + e] = x[e] - msh;
      }
    }
    kv_dma(st + 1, sb ^ 1);  // the other stage buffer, read last stage
    bias_dma(st + 1);        // the other tile buffer, read last stage (issued last: see below)
    if (active) {
      // Rows in pairs: S^T = (bias - m) + K Q^T, the exponentials, one check of the partial
      // sums, then O^T += V^T P^T. With two pairs the stage is software-pipelined inside the
      // wave: the exponentials of one pair are issued between the MFMAs of the other (the
      // logits of pair 2 under the exponentials of pair 0, then the P V products of pair 0
      // under those of pair 2), since a SIMD overlaps a wave's VALU work with that wave's own
      // MFMAs but not with another wave's.
      auto qk_pair = [&](int rp, f32x16 (&S)[2]) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int rr = rp + u;
          const bf16* kt = lds.k[sb][rr];
          S[u] = XOFF ? mfma32(ones8, moff[rr], bcur) : bcur;
#pragma unroll
          for (int f = 0; f < DQ; ++f) S[u] = mfma32(ld8(kt + koff<DQ>(li, 2 * f + g)), qa[rr][f], S[u]);
        }
      };
      auto exp_pair = [&](const f32x16 (&S)[2], bf16x8 (&p0)[2], bf16x8 (&p1)[2], float (&ts)[2]) {
#pragma unroll
        for (int u = 0; u < 2; ++u) ts[u] = exp_pack(S[u], p0[u], p1[u]);
      };
      auto check_pair = [&](int rp, f32x16 (&S)[2], bf16x8 (&p0)[2], bf16x8 (&p1)[2], float (&ts)[2]) {
        if (__builtin_amdgcn_ballot_w64(!(ts[0] < kSumRescale) || !(ts[1] < kSumRescale)) != 0) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int rr = rp + u;
            if (__builtin_amdgcn_ballot_w64(!(ts[u] < kSumRescale)) == 0) continue;
            // logits far above the offset: the row's extra offset rises to the tile's maximum
            // (rounded up to bf16), its sum and output so far are scaled by 2^-(increase), and
            // the tile is recomputed
            float tm = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) tm = fmaxf(tm, S[u][e]);
            tm = pair_max(tm);
            const float xn = tm > 0.f ? bf16_ceil(xoff[rr] + tm) : xoff[rr];
            const float dm = xn - xoff[rr];
            const float f = fast_exp2(-dm);
#pragma unroll
            for (int e = 0; e < 16; ++e) S[u][e] -= dm;
            l[rr] *= f;
#pragma unroll
            for (int h = 0; h < DH; ++h)
#pragma unroll
              for (int e = 0; e < 16; ++e) O[rr][h][e] *= f;
            xoff[rr] = xn;
            if (g == 0) moff[rr][0] = (bf16)(-xn);
            xrows = true;
            ts[u] = exp_pack(S[u], p0[u], p1[u]);
          }
        }
      };
      auto pv_pair = [&](int rp, const bf16x8 (&p0)[2], const bf16x8 (&p1)[2], const float (&ts)[2]) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int rr = rp + u;
          l[rr] += ts[u];
          const bf16* vtile = lds.v[sb][rr];
#pragma unroll
          for (int h = 0; h < DH; ++h) {
            O[rr][h] = mfma32(ld8(vtile + voff(dl + 32 * h, g)), p0[u], O[rr][h]);
            O[rr][h] = mfma32(ld8(vtile + voff(dl + 32 * h, 2 + g)), p1[u], O[rr][h]);
          }
        }
      };
      f32x16 SA[2], SB[2];
      bf16x8 pA0[2], pA1[2], pB0[2], pB1[2];
      float tsA[2], tsB[2];
      if constexpr (FR == 2) {
        qk_pair(0, SA);
        exp_pair(SA, pA0, pA1, tsA);
        check_pair(0, SA, pA0, pA1, tsA);
        pv_pair(0, pA0, pA1, tsA);
      } else {
        static_assert(FR == 4, "flash rows per workgroup");
        constexpr int NQK = 2 * (DQ + (XOFF ? 1 : 0));  // MFMAs of one pair's logits
        qk_pair(0, SA);
        __builtin_amdgcn_sched_barrier(0);  // (each pipelined region is scheduled on its own)
        // the logits of rows 2, 3 under the exponentials of rows 0, 1
        qk_pair(2, SB);
        exp_pair(SA, pA0, pA1, tsA);
        flash_interleave<2 * DQ, NQK, 64 / NQK>();
        __builtin_amdgcn_sched_barrier(0);
        check_pair(0, SA, pA0, pA1, tsA);
        // the P V products of rows 0, 1 under the exponentials of rows 2, 3
        pv_pair(0, pA0, pA1, tsA);
        exp_pair(SB, pB0, pB1, tsB);
        flash_interleave<4 * DH, 4 * DH, 64 / (4 * DH)>();
        __builtin_amdgcn_sched_barrier(0);
        check_pair(2, SB, pB0, pB1, tsB);
        pv_pair(2, pB0, pB1, tsB);
      }
    }
    // this wave's pieces of the next K / V^T stage have landed (only its 4 bias pieces, issued
    // after them, may still be in flight); the barrier publishes everyone's and retires this
    // stage's reads of the buffer the next transfers overwrite
    wait_vm_lds<4>();
    __syncthreads();
    };
  int64_t st = 0;
#pragma unroll 1
  for (; st < nrun && !xrows; ++st) stage(st, std::false_type{});
#pragma unroll 1
  for (; st < nrun; ++st) stage(st, std::true_type{});
  wait_vm_lds<0>();  // no LDS write may land after exit
  if (!active) return;

  // Exact two-pass softmax of one attention row for this wave's 32 queries, reading K, V^T
  // and the bias tiles straight from global memory (the rare path: rows whose sums left the
  // safe range of the fixed offset).
  auto exact_row = [&](int rr, f32x16 (&Orow)[DH], float& lrow) {
    const bf16* krow = kbase + (int64_t)rr * np * D + li * D;
    const bf16* vrow = vbase + (int64_t)rr * D * np + dl * 32;  // key block kb at kb * 32 D
    auto logits = [&](int64_t kb) {
      f32x16 st;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(bias_w + kb * 1024 + 256 * v4 + 4 * lane);
#pragma unroll
        for (int e = 0; e < 4; ++e) st[4 * v4 + e] = x[e];
      }
#pragma unroll
      for (int f = 0; f < DQ; ++f) st = mfma32(ld8(krow + kb * 32 * D + 16 * f + 8 * g), qa[rr][f], st);
      return st;
    };
    float mx = -INFINITY;
    for (int64_t kb = 0; kb < nb; ++kb) {
      const f32x16 st = logits(kb);
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[i]);
    }
    mx = pair_max(mx);
    const float off = mx > -INFINITY ? mx : 0.f;
    f32x16 o[DH];
#pragma unroll
    for (int h = 0; h < DH; ++h) o[h] = zero16();
    float ls = 0.f;
    for (int64_t kb = 0; kb < nb; ++kb) {
      f32x16 st = logits(kb);
#pragma unroll
      for (int i = 0; i < 16; ++i) st[i] -= off;
      bf16x8 p0, p1;
      ls += exp_pack(st, p0, p1);
#pragma unroll
      for (int h = 0; h < DH; ++h) {
        o[h] = mfma32(ld8(vrow + kb * 32 * D + 32 * h * 32 + 8 * g), p0, o[h]);
        o[h] = mfma32(ld8(vrow + kb * 32 * D + 32 * h * 32 + 16 + 8 * g), p1, o[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < DH; ++h) Orow[h] = o[h];
    lrow = ls;
  };

  const bool qvalid = j < a.n_valid;
#pragma unroll
  for (int rr = 0; rr < FR; ++rr) {
    const int64_t r = r0 + rr;
    if (r >= a.rows_valid) continue;  // a padded row: nothing to store
    float lt = pair_sum(l[rr]);
    // padded queries (past n) take no part in the choice
    if (__builtin_amdgcn_ballot_w64(qvalid && (!(lt < kSumHigh) || !(lt > kSumLow))) != 0) {
      exact_row(rr, O[rr], l[rr]);
      lt = pair_sum(l[rr]);
    }
    if (!qvalid) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int64_t off = bidx * a.o_sb + r * a.o_sr + j * a.o_sj + h * D;
#pragma unroll
    for (int hh = 0; hh < DH; ++hh) {
      // 16-byte pieces of 8 head channels (half the store instructions of 8-byte ones): half g
      // ends with pieces g and 2 + g of the tile's 32 rows
      float y[2][8];
      acc_pieces(O[rr][hh], g, y);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int d0 = 32 * hh + 8 * (2 * k + g);
        if (d0 >= D) continue;  // 16-wide heads: rows 16-31 repeat rows 0-15
        bf16x8 w;
        if (GATED) {
          const bf16x8 gv = *reinterpret_cast<const bf16x8*>(a.gate + off + d0);
#pragma unroll
          for (int t = 0; t < 8; ++t) w[t] = (bf16)(y[k][t] * inv * (float)gv[t]);
          *reinterpret_cast<bf16x8*>(a.og + off + d0) = w;
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) w[t] = (bf16)(y[k][t] * inv);
          st16<kNtFlash>(a.o + off + d0, w);
        }
      }
    }
  }
}

// out = z + (sigmoid(LN(z) W_g^T) * o) W_out^T over tiles of 64 consecutive pairs of one z row
// (z, o and out share the [b][i][j][128] layout, so a tile is 16 contiguous KB of each).
// Persistent, one workgroup of 8 waves per CU; wave w owns output channels 32 (w & 3) ..
// + 31 of positions 32 (w >> 2) .. + 31, for the gate and for the output projection. z and o
// tiles arrive by LDS DMA two tiles ahead (three-slot rings); LN(z) of the next tile is
// computed during the current one. A step: the gate times o, in place in the o slot; LN of
// the next tile; a barrier; the output projection plus the residual, in place in the z slot.
// After the next step's first barrier, the finished rows leave as whole 256-byte rows (16
// bytes per lane), before that slot is refilled.
__global__ __launch_bounds__(512, 2) void triattn_output(
    const bf16* __restrict__ z, const bf16* __restrict__ o, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ wg, const bf16* __restrict__ wo,
    const float* __restrict__ bg, const float* __restrict__ bo, bf16* __restrict__ out,
    int batch, int n, int residual, float eps) {
  constexpr int NB = 3;
  __shared__ __attribute__((aligned(16))) bf16 zs[NB][kPT * 128];  // raw z, then out (off128)
  __shared__ __attribute__((aligned(16))) bf16 os[NB][kPT * 128];  // o, then gate * o (off128)
  __shared__ __attribute__((aligned(16))) bf16 xh[2][kPT * 128];   // LN(z) (off128)
  __shared__ __attribute__((aligned(16))) float lnp[2][128];
  __shared__ float pbias[2][128];  // gate bias (times -log2 e, as the packed gate), output bias
  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cb = wave & 3, pt = wave >> 2;
  if (tid < 256) lnp[tid >> 7][tid & 127] = (tid < 128 ? ln_w : ln_b)[tid & 127];
  if (tid >= 256) {  // published by the first barrier; absent biases are zeros
    const int c = tid & 127;
    pbias[(tid >> 7) & 1][c] = tid < 384 ? (bg ? -kLog2e * bg[c] : 0.f) : (bo ? bo[c] : 0.f);
  }
  WFrag fg, fo;
  load_wfrag(fg, wg, 32 * cb, li, g);
  load_wfrag(fo, wo, 32 * cb, li, g);
  settle(fg);
  settle(fo);
  const int njb = (n + kPT - 1) / kPT;
  const int ntiles = batch * n * njb;
  auto where = [&](int tile, int& valid) -> int64_t {
    const int jb = tile % njb;
    const int i = (tile / njb) % n;
    const int b = tile / (njb * n);
    const int j0 = jb * kPT;
    valid = min(kPT, n - j0);
    return (((int64_t)b * n + i) * n + j0) * 128;
  };
  // This wave's 2 one-KB pieces of the tile's z and of its o into ring slot buf (positions
  // past the end re-read the last real one); a tile index past the end fetches tile 0 again,
  // so every wave always has the same number of transfers in flight.
  auto dma = [&](int tile, int buf) {
    int valid;
    const int64_t off = where(tile < ntiles ? tile : 0, valid);
    const uint32_t dz = lds_addr(&zs[buf][0]), dov = lds_addr(&os[buf][0]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int piece = 2 * wave + u, pos = 4 * piece + (lane >> 4);
      const int pe = pos < valid ? pos : valid - 1;
      const uint32_t voff = pe * 256 + 16 * ((lane & 15) ^ (pos & 15));
      dma16_stream(z + off, voff, dz + 1024 * piece);
      dma16_stream(o + off, voff, dov + 1024 * piece);
    }
  };
  const int step = gridDim.x;
  if ((int)blockIdx.x >= ntiles) return;
  dma(blockIdx.x, 0);
  dma(blockIdx.x + step, 1);
  wait_vm_lds<4>();  // this wave's transfers of the first tile landed
  __syncthreads();
  {
    int valid;
    where(blockIdx.x, valid);
    ln_swz<kPT, 512>(zs[0], xh[0], valid, lnp[0], lnp[1], eps);
  }
  const int p0 = 32 * pt + li;  // this lane's position in both products
  int buf = 0, k = 0, prev_valid = kPT, last_buf = 0;
  int64_t prev_off = 0;
  // the output rows of a finished tile (all 128 channels, in place in its z slot) as whole
  // 256-byte rows: wave w stores positions 8 w .. 8 w + 7, 16 lanes a position
  auto store_rows = [&](const bf16* zrow, int64_t o_off, int o_valid) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int p = 8 * wave + 4 * u + (lane >> 4), c = lane & 15;
      if (p < o_valid) st16<kNtOutput>(out + o_off + (int64_t)p * 128 + 8 * c, ld8(&zrow[off128(p, c)]));
    }
  };
#pragma unroll 1
  for (int tile = blockIdx.x; tile < ntiles; tile += step, ++k, buf = buf == NB - 1 ? 0 : buf + 1) {
    int valid;
    const int64_t off = where(tile, valid);
    const int nbuf = buf == NB - 1 ? 0 : buf + 1, fbuf = nbuf == NB - 1 ? 0 : nbuf + 1;
    // this wave's transfers of tile + step have landed (nothing was issued after them); the
    // barrier publishes everyone's pieces, LN(z) and the previous tile's output rows, and
    // retires the previous tile's other accesses to ring slot fbuf
    wait_vm_lds<0>();
    __syncthreads();
    if (k > 0) {
      store_rows(zs[fbuf], prev_off, prev_valid);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the rows are read before the slot is refilled
    }
    dma(tile + 2 * step, fbuf);
    // gate: D[channel][position], lane position p0, registers channels 32 cb + 8 j + 4 g + e
    {
      const bf16* xr = xh[k & 1];
      f32x16 ag = zero16();
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) ag = mfma32(fg.k[kk], ld8(&xr[off128(p0, 2 * kk + g)]), ag);
      bf16* orow = os[buf];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x4* po = reinterpret_cast<bf16x4*>(&orow[off128(p0, 4 * cb + j) + 4 * g]);
        const bf16x4 ov = *po;
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (bf16)(sigmoid_scaled(ag[4 * j + e] + pbias[0][32 * cb + 8 * j + 4 * g + e]) * (float)ov[e]);
        *po = v;
      }
    }
    if (tile + step < ntiles) {
      int nvalid;
      where(tile + step, nvalid);
      ln_swz<kPT, 512>(zs[nbuf], xh[(k + 1) & 1], nvalid, lnp[0], lnp[1], eps);
    }
    __syncthreads();
    // output projection: D[channel][position] over the gated o of all 128 channels
    {
      const bf16* gr = os[buf];
      f32x16 ao = zero16();
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) ao = mfma32(fo.k[kk], ld8(&gr[off128(p0, 2 * kk + g)]), ao);
      bf16* zrow = zs[buf];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bf16x4* pz = reinterpret_cast<bf16x4*>(&zrow[off128(p0, 4 * cb + j) + 4 * g]);
        const bf16x4 zv = *pz;
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (bf16)(ao[4 * j + e] + pbias[1][32 * cb + 8 * j + 4 * g + e] + (residual ? (float)zv[e] : 0.f));
        *pz = v;
      }
    }
    prev_valid = valid;
    prev_off = off;
    last_buf = buf;
  }
  __syncthreads();  // every wave's part of the last tile's output rows
  store_rows(zs[last_buf], prev_off, prev_valid);
  wait_vm_lds<0>();  // no LDS write may land after exit
}

static int persistent_grid(int ntiles, int per_cu) {
  return max(1, min(ntiles, cu_count() * per_cu));
}

void launch_flash(const FlashArgs& a, hipStream_t stream) {
  const int64_t nqb = (a.np + 32 * kFW - 1) / (32 * kFW);
  const int fr = a.dh == 64 ? flash_rows<4>() : kFR;
  const dim3 grid((unsigned)(nqb * (a.rows / fr) * a.batch * a.heads));
  const bool gated = a.og != nullptr;
  if (a.dh == 64) {
    if (gated)
      flash_attn_bias<4, true><<<grid, 64 * kFW, 0, stream>>>(a);
    else
      flash_attn_bias<4, false><<<grid, 64 * kFW, 0, stream>>>(a);
  } else if (a.dh == 16) {
    if (gated)
      flash_attn_bias<1, true><<<grid, 64 * kFW, 0, stream>>>(a);
    else
      flash_attn_bias<1, false><<<grid, 64 * kFW, 0, stream>>>(a);
  } else {
    if (gated)
      flash_attn_bias<2, true><<<grid, 64 * kFW, 0, stream>>>(a);
    else
      flash_attn_bias<2, false><<<grid, 64 * kFW, 0, stream>>>(a);
  }
}

void launch_triattn(const TriattnArgs& a, hipStream_t stream) {
  const int np = a.np;
  const int tiles_p = a.batch * np * (np / kPT);
  triattn_project<<<persistent_grid(tiles_p, 1), 512, 0, stream>>>(
      a.z, a.maskf, a.ln_w, a.ln_b, a.wqkv, a.wb, a.q, a.k, a.vt, a.bias, a.batch, a.n, np,
      a.starting, a.transposed_bias, a.eps);
  FlashArgs f{};
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
  f.kstages = a.kstages;
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
  if (a.project_only) return;
  const int tiles_o = a.batch * a.n * ((a.n + kPT - 1) / kPT);
  auto output = [&](const bf16* wo, const float* bo, bf16* dst, int residual) {
    triattn_output<<<persistent_grid(tiles_o, 1), 512, 0, stream>>>(
        a.z, a.o, a.ln_w, a.ln_b, a.wg, wo, a.bg, bo, dst, a.batch, a.n, residual, a.eps);
  };
  if (a.form == kTriattnUntransposed) {
    // the update in the attention's orientation: the z-frame update, transposed
    output(a.wo, a.bo, a.tbuf, 0);
    launch_pair_add_transposed(a.residual ? a.z : nullptr, a.tbuf, a.out, a.batch, a.n, 128, stream);
  } else if (a.form == kTriattnDual) {
    output(a.wo_t, a.bo_t, a.tbuf, 0);
    output(a.wo, a.bo, a.out, a.residual);
    launch_pair_add_transposed(a.out, a.tbuf, a.out, a.batch, a.n, 128, stream);
  } else {
    output(a.wo, a.bo, a.out, a.residual);
  }
}

}  // namespace ffk
