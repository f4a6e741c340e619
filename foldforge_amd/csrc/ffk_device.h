// Device-side building blocks shared by the pair-stack kernels (gfx950 / CDNA4 only).
//
// MFMA: v_mfma_f32_32x32x16_bf16 (one wave64 computes a 32x32 fp32 tile from a
// 32x16 A slice and a 16x32 B slice). Operand layout used throughout:
//   lane l = 32*g + i (g = 0, 1): A operand = 8 bf16 of row i at k = 8g..8g+7 of the
//   16-wide k slice; B operand = 8 bf16 of column i at the same k. Because A and B use
//   the same k <-> (lane group, element) pairing, any consistent permutation of k
//   inside a slice gives the same sum.
//   D (16 fp32 per lane): acc[r] is row 8*(r/4) + 4*g + (r%4), column i.
// Every matrix operand here is "K-contiguous": A rows and B columns are contiguous
// along k, so one 16-byte load fetches a lane's operand.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ffk {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(bf16))));
typedef bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(bf16))));
typedef bf16 bf16x2 __attribute__((__vector_size__(2 * sizeof(bf16))));
typedef f16 f16x4 __attribute__((__vector_size__(4 * sizeof(f16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.f;
  return z;
}

// Row (within a 32x32 MFMA tile) held by accumulator register r of lane group g.
__device__ __forceinline__ int acc_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// Index of pair-bias entry (query, key) in the flash core's blocked layout
//   [bh][query / 32][key / 32][v][lane][e] (a 32 x 32 tile = 1024 fp32),
//   lane = 32 g + query % 32, key % 32 = 8 v + 4 g + e:
// accumulator register 4 v + e of lane `lane` of the S^T tile; a lane's 4 registers of one v
// are 16 contiguous bytes and consecutive lanes are consecutive, so a DMA'd tile reads back
// from LDS without bank conflicts.
__device__ __forceinline__ int64_t bias_index(int64_t bh, int64_t nb, int64_t query, int64_t key) {
  const int kk = (int)(key & 31);
  const int v = kk >> 3, g = (kk >> 2) & 1, e = kk & 3;
  const int lane = 32 * g + (int)(query & 31);
  return ((((bh * nb + (query >> 5)) * nb + (key >> 5)) * 4 + v) * 64 + lane) * 4 + e;
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// 8 fp32 values -> bf16 hi + lo (hi + lo carries the value to about 16 bits of mantissa).
__device__ __forceinline__ void split8(const f32x4& a, const f32x4& b, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (bf16)a[e];
    hi[4 + e] = (bf16)b[e];
    lo[e] = (bf16)(a[e] - (float)hi[e]);
    lo[4 + e] = (bf16)(b[e] - (float)hi[4 + e]);
  }
}

// 8 consecutive fp32 values (16-byte aligned) -> one bf16 MFMA operand.
__device__ __forceinline__ bf16x8 cvt8(const float* p) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = (bf16)a[e];
    r[4 + e] = (bf16)b[e];
  }
  return r;
}

// Stores of intermediates that the next kernel reads once. Bit k of FFK_NT_MASK makes family k
// use non-temporal (streaming) stores: 1 projections (A, B, q, k, v^T), 2 contraction (P),
// 4 output kernels (z), 8 flash core (o). Only the output kernels stream by default: streaming
// the projections' outputs sped a ragged N = 512 block up by 2% but slowed a full-mask trunk by
// 2% (their consumers then read from HBM instead of the last-level cache), and streaming P or o
// (the flash core writes 8-byte pieces) cost 3-20%.
#ifndef FFK_NT_MASK
#define FFK_NT_MASK 4
#endif
constexpr int kNtProject = 1, kNtContract = 2, kNtOutput = 4, kNtFlash = 8;
template <int Family>
__device__ __forceinline__ void st16(bf16* p, bf16x8 v) {
  if constexpr ((FFK_NT_MASK & Family) != 0)
    __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(p));
  else
    *reinterpret_cast<bf16x8*>(p) = v;
}
template <int Family>
__device__ __forceinline__ void st8(bf16* p, bf16x4 v) {
  if constexpr ((FFK_NT_MASK & Family) != 0)
    __builtin_nontemporal_store(v, reinterpret_cast<bf16x4*>(p));
  else
    *reinterpret_cast<bf16x4*>(p) = v;
}

// Four values rounded to bf16, one 8-byte store.
__device__ __forceinline__ void store4(bf16* p, float a, float b, float c, float d) {
  bf16x4 v;
  v[0] = (bf16)a;
  v[1] = (bf16)b;
  v[2] = (bf16)c;
  v[3] = (bf16)d;
  *reinterpret_cast<bf16x4*>(p) = v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.f + fast_exp2(-x * kLog2e));
}

__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }

// sigmoid(x) from y = -log2(e) x (gate weights packed pre-multiplied by -log2(e)).
__device__ __forceinline__ float sigmoid_scaled(float y) {
  return __builtin_amdgcn_rcpf(1.f + fast_exp2(y));
}

// acc += A(32 x K) * B(K x 32); a_row / b_row point at k = 0 of this lane's A row and
// B column (lane l%32), K a multiple of 16.
template <int K>
__device__ __forceinline__ void mma_rows(const bf16* a_row, const bf16* b_row, int g, f32x16& acc) {
#pragma unroll
  for (int k0 = 0; k0 < K; k0 += 16) {
    acc = mfma32(ld8(a_row + k0 + 8 * g), ld8(b_row + k0 + 8 * g), acc);
  }
}

// The hardware deals workgroup w to XCD w % 8 (each XCD has its own L2). Renumber so that
// every XCD receives one contiguous range of logical workgroup ids: neighbours in the
// logical order (which share operands) then share an L2. Identity when total % 8 != 0.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t wg, uint32_t total) {
  if (total % 8u != 0u) return wg;
  return (wg % 8u) * (total / 8u) + wg / 8u;
}

// A persistent workgroup's tile in a (batch, row, block) grid, tile = (b * rows + r) * nblk +
// blk. The walk advances by the grid stride with adds and carries: the stride is split into
// the same three digits once, so the tile loop does no integer division (a runtime 32-bit
// division is a long scalar sequence, and a tile loop needs the digits of three tiles).
struct TileAt {
  int blk, r, b;
};
__device__ __forceinline__ TileAt tile_at(int tile, int nblk, int rows) {
  TileAt t;
  t.blk = tile % nblk;
  t.r = (tile / nblk) % rows;
  t.b = tile / (nblk * rows);
  return t;
}
// t + step, where step = tile_at(stride, nblk, rows) (each digit below its radix).
__device__ __forceinline__ TileAt tile_add(TileAt t, const TileAt& step, int nblk, int rows) {
  t.blk += step.blk;
  int carry = t.blk >= nblk ? 1 : 0;
  t.blk -= carry * nblk;
  t.r += step.r + carry;
  carry = t.r >= rows ? 1 : 0;
  t.r -= carry * rows;
  t.b += step.b + carry;
  return t;
}

// Smallest bf16-representable value >= x (x finite).
__device__ __forceinline__ float bf16_ceil(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0xffffu) != 0u) u = (u & 0xffff0000u) + (x > 0.f ? 0x10000u : 0u);
  return __uint_as_float(u);
}

// Combine x with the value of lane l ^ 32 (one v_permlane32_swap). After the swap of x
// with itself each lane holds {x, partner} in the two results, in an order that depends
// on the half, so only symmetric combinations are formed.
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A 32-row x 128-k slice of a K-contiguous bf16 weight matrix held in registers: entry kk
// is this lane's MFMA operand for k = 16 kk .. 16 kk + 15 of row (first + lane % 32).
struct WFrag {
  bf16x8 k[8];
};

__device__ __forceinline__ void load_wfrag(WFrag& w, const bf16* __restrict__ W, int first_row,
                                           int li, int g) {
  const bf16* row = W + (int64_t)(first_row + li) * 128 + 8 * g;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) w.k[kk] = ld8(row + 16 * kk);
}

// Force the loads of a fragment to complete here. Weight fragments are loaded once before a
// persistent tile loop; without this the compiler's wait bookkeeping cannot prove them done at
// the loop head and re-waits on them inside every iteration (down to vmcnt(0)), which also
// drains every DMA and store the loop keeps in flight.
__device__ __forceinline__ void settle(const WFrag& w) {
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) asm volatile("" ::"v"(w.k[kk]));
}

// Lane permutes inside rows of 16 lanes (DPP, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}
constexpr int kDppXor1 = 0xb1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4e;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each 16

// Sum over groups of 4 / 16 consecutive lanes (every lane of the group gets the total): pair
// and quad sums by quad permutes, then the two quads of an 8 joined by the half-row mirror
// and the two 8s of a 16 by the row mirror.
__device__ __forceinline__ float sum4(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  return v;
}

__device__ __forceinline__ float sum16(float v) {
  v = sum4(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Row stride (elements) of a 128-channel bf16 tile in LDS: 16 bytes of padding per row.
constexpr int kRow = 136;

// A tile of TM positions of a 128-channel bf16 pair tensor in registers, NT threads
// (256 or 512): 16 lanes per position, 8 channels per lane, NT / 16 positions per pass.
template <int TM, int NT = 256>
struct LnTile {
  static constexpr int kPer = NT / 16;
  static constexpr int kPass = TM / kPer;
  bf16x8 v[kPass];
};

// Issue the loads of a tile: position t lives at base + t * stride (elements) and is real
// when t < valid; other positions read as zeros.
template <int TM, int NT>
__device__ __forceinline__ void ln_load(LnTile<TM, NT>& tile, const bf16* __restrict__ base,
                                        int64_t stride, int valid) {
  const int sub = threadIdx.x & 15, pos0 = threadIdx.x >> 4;
#pragma unroll
  for (int it = 0; it < LnTile<TM, NT>::kPass; ++it) {
    const int t = pos0 + LnTile<TM, NT>::kPer * it;
    if (t < valid) {
      tile.v[it] = ld8(base + (int64_t)t * stride + 8 * sub);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) tile.v[it][e] = (bf16)0.f;
    }
  }
}

// LayerNorm a loaded tile (fp32 statistics, fp32 affine) into LDS as bf16 [TM][kRow]; invalid
// positions are written as zeros. When raw is non-null the input is stored there too.
template <int TM, int NT>
__device__ __forceinline__ void ln_finish(const LnTile<TM, NT>& tile, int valid,
                                          const float* __restrict__ w, const float* __restrict__ b,
                                          float eps, bf16* xh, bf16* raw) {
  const int sub = threadIdx.x & 15, pos0 = threadIdx.x >> 4;
  float wv[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wv[e] = w[8 * sub + e];
    bv[e] = b ? b[8 * sub + e] : 0.f;
  }
#pragma unroll
  for (int it = 0; it < LnTile<TM, NT>::kPass; ++it) {
    const int t = pos0 + LnTile<TM, NT>::kPer * it;
    float x[8];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = (float)tile.v[it][e];
      s += x[e];
    }
    const float mean = sum16(s) * (1.f / 128.f);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] -= mean;
      q += x[e] * x[e];
    }
    const float rstd = __builtin_amdgcn_rsqf(sum16(q) * (1.f / 128.f) + eps);
    bf16x8 o;
    const bool real = t < valid;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = real ? (bf16)(x[e] * rstd * wv[e] + bv[e]) : (bf16)0.f;
    *reinterpret_cast<bf16x8*>(xh + t * kRow + 8 * sub) = o;
    if (raw) *reinterpret_cast<bf16x8*>(raw + t * kRow + 8 * sub) = tile.v[it];
  }
}

// An opaque copy of a pointer: loads through it cannot be hoisted out of the enclosing loop
// (used where keeping loop-invariant values in registers would cost occupancy).
template <typename T>
__device__ __forceinline__ const T* opaque(const T* p) {
  asm volatile("" : "+s"(p));
  return p;
}

typedef __attribute__((address_space(3))) void lds_void;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void*)p;
}

// gfx950 LDS: 64 banks of 4 bytes; a 16-byte-per-lane access serves 16 lanes per cycle.
// Element offset of 16-byte piece k8 of row r in an unpadded 128-channel bf16 tile, pieces
// XOR-swizzled with r % 16: sixteen lanes reading sixteen consecutive rows at one k (an MFMA
// operand fetch) or the sixteen pieces of one row hit distinct banks.
__device__ __forceinline__ int off128(int r, int k8) { return r * 128 + 8 * (k8 ^ (r & 15)); }

// One wave-wide LDS DMA: lane L copies 16 bytes from sbase + voff (bytes) to LDS byte address
// m0 + 16 L; sbase and m0 are wave-uniform. Issued as inline assembly so that the compiler's
// wait insertion does not treat every later LDS read as dependent on it: each use is paired
// with an explicit s_waitcnt vmcnt (vector-memory operations of a wave complete in order)
// before the data is read, and a kernel waits for its last transfers before it exits.
// The compiler does not look inside inline assembly for hazards, so the transfer is preceded
// by the wait states the ISA requires of its operands: 5 after a VALU instruction writes an
// SGPR that a VMEM instruction reads (the compiler materialises sbase with v_readlane or
// v_readfirstlane when scalar registers run short), which also covers the 1 after an SALU
// write of M0 before a global load with LDS = 1.
#define FFK_DMA_HAZARD "s_nop 4\n"
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t m0) {
  asm volatile(FFK_DMA_HAZARD "global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0)
               : "memory");
}
// Same for data read once (the pair tensor): non-temporal, so the stream does not evict
// reused data (weights) from L2.
__device__ __forceinline__ void dma16_stream(const void* sbase, uint32_t voff, uint32_t m0) {
  asm volatile(FFK_DMA_HAZARD "global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase),
               "{m0}"(m0)
               : "memory");
}
// Same for 4 bytes per lane: lane L copies sbase + voff to LDS byte address m0 + 4 L.
__device__ __forceinline__ void dma4(const void* sbase, uint32_t voff, uint32_t m0) {
  asm volatile(FFK_DMA_HAZARD "global_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0)
               : "memory");
}
// Wait until at most N vector-memory operations of this wave are in flight and its LDS
// operations are done.
template <int N>
__device__ __forceinline__ void wait_vm_lds() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}

// Sum of 8 values as a tree (depth 3 rather than a chain of 8 dependent adds).
__device__ __forceinline__ float sum8(const float (&x)[8]) {
  return ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
}

// LayerNorm (fp32 statistics and affine) of the rows 0 .. TM - 1 of an off128 tile src into
// the off128 tile dst (which may be src), NT threads, 16 lanes per row; rows >= valid become
// zeros. A thread's rows are all read before any is written (in place, the compiler could not
// otherwise issue a later row's read ahead of an earlier row's write), and the rows' sums and
// reductions are independent, so their latencies overlap: this runs between two barriers of
// every tile of the persistent pair kernels, so its length is on their critical path.
template <int TM, int NT>
__device__ __forceinline__ void ln_swz(const bf16* src, bf16* dst, int valid, const float* w,
                                       const float* b, float eps) {
  constexpr int IT = TM / (NT / 16);
  const int sub = threadIdx.x & 15, pos0 = threadIdx.x >> 4;
  bf16x8 raw[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it)
    raw[it] = *reinterpret_cast<const bf16x8*>(&src[off128(pos0 + (NT / 16) * it, sub)]);
  float wv[8], bv[8];
  {
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(w + 8 * sub);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(w + 8 * sub + 4);
    f32x4 b0 = {0.f, 0.f, 0.f, 0.f}, b1 = b0;
    if (b) {
      b0 = *reinterpret_cast<const f32x4*>(b + 8 * sub);
      b1 = *reinterpret_cast<const f32x4*>(b + 8 * sub + 4);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wv[e] = w0[e];
      wv[e + 4] = w1[e];
      bv[e] = b0[e];
      bv[e + 4] = b1[e];
    }
  }
  float x[IT][8], mean[IT], rstd[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[it][e] = (float)raw[it][e];
    mean[it] = sum8(x[it]);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) mean[it] = sum16(mean[it]) * (1.f / 128.f);
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    float d2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[it][e] -= mean[it];
      d2[e] = x[it][e] * x[it][e];
    }
    rstd[it] = sum8(d2);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) rstd[it] = __builtin_amdgcn_rsqf(sum16(rstd[it]) * (1.f / 128.f) + eps);
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int t = pos0 + (NT / 16) * it;
    bf16x8 o;
    const bool real = t < valid;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = real ? (bf16)(x[it][e] * rstd[it] * wv[e] + bv[e]) : (bf16)0.f;
    *reinterpret_cast<bf16x8*>(&dst[off128(t, sub)]) = o;
  }
}
template <int TM, int NT>
__device__ __forceinline__ void ln_inplace_swz(bf16* buf, int valid, const float* w, const float* b,
                                               float eps) {
  ln_swz<TM, NT>(buf, buf, valid, w, b, eps);
}

// Load and LayerNorm in one step (see ln_load / ln_finish).
template <int TM, int NT = 256>
__device__ __forceinline__ void ln_tile_128(const bf16* __restrict__ base, int64_t stride, int valid,
                                            const float* __restrict__ w, const float* __restrict__ b,
                                            float eps, bf16* xh, bf16* raw) {
  LnTile<TM, NT> tile;
  ln_load(tile, base, stride, valid);
  ln_finish(tile, valid, w, b, eps, xh, raw);
}

// The 32 rows of a 32 x 32 accumulator tile in 16-byte pieces: lanes l and l ^ 32 hold rows
// 8 v + 4 g + 0..3 of piece v in acc[4 v ..]; one exchange of 8 values leaves half g with the
// whole pieces g and 2 + g (y[k][0..7] = rows 8 (2 k + g) + 0..7). Both lanes of a pair must run
// it together.
__device__ __forceinline__ void acc_pieces(const f32x16& acc, int g, float (&y)[2][8]) {
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = acc[8 * k + e], hi = acc[8 * k + 4 + e];
      const uint32_t send = __float_as_uint(g ? lo : hi);
      const auto sw = __builtin_amdgcn_permlane32_swap(send, send, false, false);
      const float recv = __uint_as_float(g ? sw[0] : sw[1]);
      y[k][e] = g ? recv : lo;
      y[k][4 + e] = g ? hi : recv;
    }
}

}  // namespace ffk
