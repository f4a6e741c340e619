// Fused pair transition on gfx950: x + squeeze(silu(expand_a(LN(x))) * expand_b(LN(x))).
//
// Equations: src/foldforge/models/checkpoints/legacy/reference/transition.py:40-41 and
// src/foldforge/modules/dense/diffusion_transformer.py:36-44 (SwiGLU). The 4c-wide hidden
// layer never leaves registers: x is read once and the output written once.
//
// Persistent over tiles of 128 positions; 4 waves per workgroup and two workgroups per CU (two
// waves per SIMD from different workgroups, so one wave's silu VALU work fills the other's MFMA
// gaps without a shared barrier; each tile start lowers the waves' priority with the
// workgroup's progress so that neither workgroup finishes far ahead of its partner). Wave w
// owns positions 32 w .. 32 w + 31 of the tile for the whole tile:
//   * its LN'd operand x^ (32 positions x 128 channels) sits in registers as the B operand;
//   * the expand GEMMs are computed transposed, D = W_a,b (hidden x k) * x^ (k x positions),
//     so a lane holds one position and 16 hidden channels of a 32-hidden block;
//   * h = silu(a) * b, rounded to bf16, is then directly the B operand of the squeeze GEMM
//     (k = hidden, in the order the accumulator registers hold it; the squeeze weight is
//     packed in that same order);
//   * the squeeze accumulates out^T (128 channels x 32 positions) in registers, initialised
//     with the residual x, across all 512 hidden channels.
// expand_a is packed pre-multiplied by -log2(e), so a' = -log2(e) a feeds exp2 directly and
// h' = a' b / (1 + 2^a') = -log2(e) h; squeeze is packed pre-multiplied by -ln(2), which
// undoes that factor (out = squeeze h = (-ln 2 squeeze) h').
// Every global-to-LDS transfer is a direct LDS DMA (global_load_lds_dwordx4), so no VGPRs
// stage data. The 384 KB of bf16 weights are packed once per call (pack_transition) into 16
// contiguous 24 KB chunks of 32 hidden channels (expand_a rows, expand_b rows, squeeze
// columns), each already in the byte order the kernel wants in LDS, so streaming a chunk is a
// plain linear copy; chunks are double-buffered, one barrier per chunk, and the next tile's
// raw x arrives behind the first chunk's compute. LDS tiles are unpadded and XOR-swizzled.
// attention_output_transition runs the triangle attention's gate / output projection in front
// of the same tile (three lead chunks of weights ahead of the 16), see there.
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kXC = 32;   // hidden channels per chunk

struct __attribute__((aligned(16))) TransitionChunk {
  bf16 wa[kXC * 128];  // expand_a rows h0 .. h0 + 31, k = 0 .. 127 (16-byte pieces swizzled)
  bf16 wb[kXC * 128];  // expand_b rows
  bf16 ws[128 * kXC];  // squeeze [out channel][hidden h0 .. h0 + 31] (pieces swizzled)
};

// Element offset of 16-byte piece p of row r of the 32-wide squeeze chunk (the analogue of
// off128: 4 pieces per row, four consecutive rows fill the 64 banks, so the piece is swizzled
// with (r / 4) % 4).
__device__ __forceinline__ int off32(int r, int p) { return r * 32 + 8 * (p ^ ((r >> 2) & 3)); }

constexpr int kChunkElems = 3 * kXC * 128;  // 12288 bf16 = 24 KB per chunk

// The attention-output variant (attention_output_transition) streams three lead chunks in
// front of the 16 transition chunks. Each lead chunk is three slabs of 32 rows x 128 k in
// off128 order (a slab fills one of the wa / wb / ws fields): slabs 0-3 hold the gate weight
// rows 32 s .. 32 s + 31 (times -log2 e, as sigmoid_scaled wants), slabs 4-7 the output
// projection rows 32 (s - 4) .., slab 8 is unused.
constexpr int kLeadChunks = 3;

__device__ __forceinline__ const bf16* lead_slab(const TransitionChunk* ch, int s) {
  return reinterpret_cast<const bf16*>(ch) + kXC * 128 * s;
}

// expand_a [512][128], expand_b [512][128], squeeze [128][512] (fp32) -> 16 chunks of the LDS
// image TransitionChunk: expand rows with 16-byte pieces at off128 positions, squeeze rows
// (output channels) holding the chunk's 32 hidden channels in accumulator order (inside each
// 16-block: 0-3, 8-11, 4-7, 12-15) with pieces at off32 positions; scaled as described above.
// With wg / wo ([128][128] gate and output projection of the triangle attention in front),
// the kLeadChunks lead chunks come first.
__global__ __launch_bounds__(256) void pack_transition(const float* __restrict__ wa,
                                                       const float* __restrict__ wb,
                                                       const float* __restrict__ ws,
                                                       const float* __restrict__ wg,
                                                       const float* __restrict__ wo,
                                                       bf16* __restrict__ dst) {
  const int lead = wg ? kLeadChunks : 0;
  const int total = (16 + lead) * kChunkElems;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    int c = i / kChunkElems;
    const int rem = i % kChunkElems, part = rem >> 12, o = rem & 4095;
    float v;
    if (c < lead) {
      const int slab = 3 * c + part, r = o >> 7, slot = (o >> 3) & 15, e = o & 7;
      const int src = (32 * (slab & 3) + r) * 128 + 8 * (slot ^ (r & 15)) + e;
      v = slab < 4 ? -kLog2e * wg[src] : slab < 8 ? wo[src] : 0.f;
      dst[i] = (bf16)v;
      continue;
    }
    c -= lead;
    if (part < 2) {
      const int r = o >> 7, slot = (o >> 3) & 15, e = o & 7;
      const int src = (kXC * c + r) * 128 + 8 * (slot ^ (r & 15)) + e;
      v = part == 0 ? -kLog2e * wa[src] : wb[src];
    } else {
      const int r = o >> 5, slot = (o >> 3) & 3, e = o & 7;
      const int q = 8 * (slot ^ ((r >> 2) & 3)) + e;            // accumulator-order position
      const int hid = (q & ~12) | ((q & 4) << 1) | ((q & 8) >> 1);  // its hidden channel
      v = (-1.f / kLog2e) * ws[r * 512 + kXC * c + hid];
    }
    dst[i] = (bf16)v;
  }
}

// This wave's share (24 / NW of the 24 one-KB pieces) of chunk c of the packed weights into
// the chunk buffer at LDS byte address buf.
template <int NW>
__device__ __forceinline__ void weight_dma(const bf16* wpack, int c, uint32_t buf, int wave,
                                           int lane) {
  constexpr int per = 24 / NW;
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int q = per * wave + u;
    dma16(wpack + c * kChunkElems, 1024 * q + 16 * lane, buf + 1024 * q);
  }
}

// One chunk: issue the DMA of the weights NB - 1 chunks ahead (and, in the first chunk of a
// tile, of this wave's rows of the next tile's x), then expand (a', b) -> h' -> squeeze into
// acc using cur.
template <int NW, typename XDma>
__device__ __forceinline__ void transition_chunk(const TransitionChunk* cur, uint32_t ahead_buf,
                                                 int c_ahead, bool first, const XDma& xdma,
                                                 const bf16* wpack, int wave, int lane,
                                                 const bf16x8 (&xb)[8], f32x16 (&acc)[4]) {
  const int g = lane >> 5, li = lane & 31;
  weight_dma<NW>(wpack, c_ahead, ahead_buf, wave, lane);
  f32x16 a = zero16(), b = zero16();
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    a = mfma32(ld8(&cur->wa[off128(li, 2 * kk + g)]), xb[kk], a);
    b = mfma32(ld8(&cur->wb[off128(li, 2 * kk + g)]), xb[kk], b);
  }
  if (first) xdma();
  // a', b: hidden h0 + 8 (r/4) + 4 g + r%4, position li. Slice s of h' (registers 8 s ..
  // 8 s + 7) covers hidden 16 s + {4 g .. 4 g + 3, 8 + 4 g .. 8 + 4 g + 3}: the packed
  // squeeze weight holds each 16-block as 0-3, 8-11 | 4-7, 12-15, so piece 2 s + g of an
  // output row is exactly that k set.
  bf16x8 hb[2];
#pragma unroll
  for (int r = 0; r < 16; ++r)
    hb[r >> 3][r & 7] = (bf16)(a[r] * b[r] * __builtin_amdgcn_rcpf(1.f + fast_exp2(a[r])));
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int ot = 0; ot < 4; ++ot)
      acc[ot] = mfma32(ld8(&cur->ws[off32(32 * ot + li, 2 * s + g)]), hb[s], acc[ot]);
  }
}

// Two workgroups share each SIMD of a CU. At equal priority the older wave wins every issue
// conflict, so the workgroup dispatched first runs ahead and the other finishes its last tiles
// alone, one wave per SIMD. A workgroup's waves therefore drop one priority level per quarter
// of its tiles done (done of total): the workgroup ahead yields to its partner.
__device__ __forceinline__ void progress_priority(int64_t done, int64_t total) {
  const int64_t q = 4 * done / total;
  if (q == 0)
    __builtin_amdgcn_s_setprio(3);
  else if (q == 1)
    __builtin_amdgcn_s_setprio(2);
  else if (q == 2)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
}

// The rows of one wave: this wave's 32 rows of the tile at row0 of src straight into its rows
// of the LDS tile (xr_lds: the wave's first row): piece j = rows 4 j .. 4 j + 3, lane L fills
// bytes 16 L of it. Rows past the end re-read the last row (finite values, never stored:
// positions do not interact). row0 < rows, so the scalar base is a real row and every offset
// is non-negative.
__device__ __forceinline__ void rows_dma(const bf16* src, int64_t row0, int64_t rows, int rw,
                                         uint32_t xr_lds, int lane) {
  const bf16* base = src + row0 * 128;
  const int64_t last = rows - 1 - row0;  // >= 0
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = rw + 4 * j + (lane >> 4);  // tile row
    const int rr = r < last ? r : (int)last;
    dma16_stream(base, 256 * rr + 16 * ((lane & 15) ^ (r & 15)), xr_lds + 4 * j * 256);
  }
}

// One tile of the transition from its rows x in the wave's rows of XR (landed and published):
// residual and LayerNorm, then the stream chunks C0 .. NCH - 1 (k: the stream position of
// chunk C0, advanced past the tile), with the next tile's rows (xdma) fetched in chunk C0 once
// x^ is in registers; the output rows are stored from registers.
template <int NW, int NB, int C0, int NCH, typename XDma>
__device__ __forceinline__ void transition_tile(bf16* XR, const TransitionChunk* W, uint32_t w_lds,
                                                const bf16* wpack, const float* ln_w,
                                                const float* ln_b, bf16* out, int64_t rows,
                                                int64_t row0, int residual, float eps, int& k,
                                                const XDma& xdma, int wave, int lane) {
  constexpr int C = 128;
  const int g = lane >> 5, li = lane & 31;
  const int sub = lane & 15, p16 = lane >> 4;  // LayerNorm layout: 16 lanes per position
  const int rw = 32 * wave;                    // this wave's first tile row
  bf16x8 xv[8];
#pragma unroll
  for (int it = 0; it < 8; ++it) xv[it] = ld8(&XR[off128(rw + 4 * it + p16, sub)]);
  // out^T accumulators: acc[ot] = channels 32 ot + (8 (r/4) + 4 g + r%4), position li
  f32x16 acc[4];
#pragma unroll
  for (int ot = 0; ot < 4; ++ot) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bf16x4 v = *reinterpret_cast<const bf16x4*>(&XR[off128(rw + li, 4 * ot + m) + 4 * g]);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[ot][4 * m + e] = residual ? (float)v[e] : 0.f;
    }
  }
  __syncthreads();
  // LayerNorm (fp32 statistics and affine), written back over the raw rows; the affine is
  // re-read per tile rather than held in registers through the chunk loop
  float lw[8], lb[8];
  {
    const float* w_ = opaque(ln_w);
    const float* b_ = opaque(ln_b);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lw[e] = w_[8 * sub + e];
      lb[e] = b_[8 * sub + e];
    }
  }
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    float v[8];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = (float)xv[it][e];
      s += v[e];
    }
    const float mean = sum16(s) * (1.f / 128.f);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] -= mean;
      q += v[e] * v[e];
    }
    const float rstd = __builtin_amdgcn_rsqf(sum16(q) * (1.f / 128.f) + eps);
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (bf16)(v[e] * rstd * lw[e] + lb[e]);
    *reinterpret_cast<bf16x8*>(&XR[off128(rw + 4 * it + p16, sub)]) = o;
  }
  __syncthreads();
  bf16x8 xb[8];  // B operand: position li, k = 16 kk + 8 g .. + 7
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) xb[kk] = ld8(&XR[off128(rw + li, 2 * kk + g)]);
  // x^ must be in registers before the next tile's x overwrites its rows
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

#pragma unroll 1
  for (int c = C0; c < NCH; ++c, ++k) {
    // chunks wrap around into the next tile; buffer (k + NB - 1) % NB was last read in
    // chunk k - 1
    transition_chunk<NW>(&W[k % NB], w_lds + ((k + NB - 1) % NB) * sizeof(TransitionChunk),
                         (c + NB - 1) % NCH, c == C0, xdma, wpack, wave, lane, xb, acc);
    // this wave's pieces of chunk k + 1 have landed (after them only the pieces of chunks up
    // to k + NB - 1 and, in the tile's first transition chunk, the 8 x pieces were issued); the
    // barrier then publishes every wave's pieces and retires the reads of W[k % NB]
    constexpr int later = (NB - 2) * (24 / NW);
    if (c == C0)
      wait_vm_lds<later + 8>();
    else
      wait_vm_lds<later>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  // Store from registers: lanes l and l ^ 32 hold channels 8 m + 0..3 and 8 m + 4..7 of one
  // position; one swap gives lane group 0 the 8 channels of m = 0, 2 and group 1 those of
  // m = 1, 3, so every lane writes 16 contiguous bytes.
  const int64_t r = row0 + rw + li;
#pragma unroll
  for (int ot = 0; ot < 4; ++ot) {
#pragma unroll
    for (int mp = 0; mp < 2; ++mp) {
      uint32_t own[2][2];  // [m - 2 mp][dword]: channels 32 ot + 8 m + 4 g + 0..3
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int base = 4 * (2 * mp + t);
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          bf16x2 p;
          p[0] = (bf16)acc[ot][base + 2 * d];
          p[1] = (bf16)acc[ot][base + 2 * d + 1];
          own[t][d] = __builtin_bit_cast(uint32_t, p);
        }
      }
      uint32_t recv[2];
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const uint32_t send = g ? own[0][d] : own[1][d];
        const auto sw = __builtin_amdgcn_permlane32_swap(send, send, false, false);
        recv[d] = g ? sw[0] : sw[1];
      }
      uint32_t v[4];
      v[0] = g ? recv[0] : own[0][0];
      v[1] = g ? recv[1] : own[0][1];
      v[2] = g ? own[1][0] : recv[0];
      v[3] = g ? own[1][1] : recv[1];
      // (regular stores: L2 merges the eight 32-byte pieces of a row into full lines)
      if (r < rows)
        *reinterpret_cast<u32x4*>(out + r * C + 32 * ot + 8 * (2 * mp + g)) =
            u32x4{v[0], v[1], v[2], v[3]};
    }
  }
}

// grid: persistent; block 64 NW (NW waves, 32 positions each, tile = 32 NW positions); NB
// weight-chunk buffers. wpack: see pack_transition.
template <int NW, int NB, int WG_PER_CU>
__global__ __launch_bounds__(64 * NW, WG_PER_CU) void transition_swiglu(
    const bf16* __restrict__ x, const float* __restrict__ ln_w, const float* __restrict__ ln_b,
    const bf16* __restrict__ wpack, bf16* __restrict__ out, int64_t rows, int residual,
    float eps) {
  constexpr int C = 128, NCH = 512 / kXC, XT = 32 * NW;
  __shared__ TransitionChunk W[NB];  // chunk k of the stream lives in W[k % NB]
  __shared__ bf16 XR[XT * C];        // x tile: raw, then x^; wave w owns rows 32 w .. 32 w + 31
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rw = 32 * wave;  // this wave's first tile row
  const uint32_t w_lds = lds_addr(W), xr_lds = lds_addr(XR + rw * C);

  const int64_t ntiles = (rows + XT - 1) / XT;
  if ((int64_t)blockIdx.x >= ntiles) return;
  rows_dma(x, (int64_t)blockIdx.x * XT, rows, rw, xr_lds, lane);
#pragma unroll
  for (int b = 0; b < NB - 1; ++b) weight_dma<NW>(wpack, b, w_lds + b * sizeof(TransitionChunk), wave, lane);
  int k = 0;  // position in the chunk stream (16 chunks per tile)

#pragma unroll 1
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * XT;
    progress_priority((tile - blockIdx.x) / gridDim.x, (ntiles - 1 - blockIdx.x) / gridDim.x + 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // own x rows and chunk-0 pieces landed
    __syncthreads();                                   // everyone's chunk-0 pieces landed
    // the last tile re-reads its own rows instead of a next tile's
    const int64_t next0 = tile + gridDim.x < ntiles ? row0 + (int64_t)gridDim.x * XT : row0;
    auto xdma = [&]() { rows_dma(x, next0, rows, rw, xr_lds, lane); };
    transition_tile<NW, NB, 0, NCH>(XR, W, w_lds, wpack, ln_w, ln_b, out, rows, row0, residual,
                                    eps, k, xdma, wave, lane);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS write may land after exit
}

// Triangle attention's output projection fused in front of the pair transition (the block
// order of AF3 and its descendants: the transition reads exactly that output):
//   y = z + (sigmoid(LN_pair(z) W_g^T) * o) W_out^T,   out = y + transition(y),
// y rounded to bf16 as the separate output kernel stores it, so the result is the two ops'
// (src/foldforge/models/checkpoints/legacy/pairformer.py:200-202: the ending node's
// attention residual, then the transition residual). z and o (the attention output, z frame) are read once and y never
// reaches HBM. Same workgroup, tiles and transition chunks as transition_swiglu; a tile first
// runs kLeadChunks lead chunks of the gate / output weights (see kLeadChunks), wave-private
// in the wave's own 32 rows of the tile:
//   z rows landed -> z kept as the residual (accumulator layout), LN_pair(z) in place -> its
//   B operands in registers -> o rows DMA'd over them;
//   lead chunk 0: gate rows 0-95 (D[channel][position], lanes = positions, as the transition's
//   accumulators), sigmoid times o, in place over o;
//   lead chunk 1: gate rows 96-127, then the gated rows read back as B operands (natural k
//   order) and the output projection rows 0-63;
//   lead chunk 2: output rows 64-127; y = z + projection into the rows, where the transition
//   tile (transition_tile) picks it up as its x.
// Neither projection carries a bias (the lineages with biases run the separate kernels).
template <int NW, int NB, int WG_PER_CU>
__global__ __launch_bounds__(64 * NW, WG_PER_CU) void attention_output_transition(
    const bf16* __restrict__ z, const bf16* __restrict__ o, const float* __restrict__ lnp_w,
    const float* __restrict__ lnp_b, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, const bf16* __restrict__ wpack, bf16* __restrict__ out,
    int64_t rows, float eps_pair, float eps) {
  constexpr int C = 128, NCH = kLeadChunks + 512 / kXC, XT = 32 * NW, per = 24 / NW;
  __shared__ TransitionChunk W[NB];  // chunk k of the stream lives in W[k % NB]
  __shared__ bf16 XR[XT * C];        // z, LN(z), o, gated o, y, LN(y); wave w owns rows 32 w ..
  const int lane = threadIdx.x & 63, g = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & 15, p16 = lane >> 4;  // LayerNorm layout: 16 lanes per position
  const int rw = 32 * wave;                    // this wave's first tile row
  const uint32_t w_lds = lds_addr(W), xr_lds = lds_addr(XR + rw * C);

  const int64_t ntiles = (rows + XT - 1) / XT;
  if ((int64_t)blockIdx.x >= ntiles) return;
  rows_dma(z, (int64_t)blockIdx.x * XT, rows, rw, xr_lds, lane);
#pragma unroll
  for (int b = 0; b < NB - 1; ++b) weight_dma<NW>(wpack, b, w_lds + b * sizeof(TransitionChunk), wave, lane);
  int k = 0;  // position in the chunk stream (NCH chunks per tile)

  // Lead chunk epilogue: its buffer's reads retire, the next chunk's pieces are published.
  auto lead_end = [&]() {
    wait_vm_lds<0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    ++k;
  };
  // rows of the gated values: sigmoid of the gate accumulator of rows 32 cb .. times o, in
  // place over o (both in the accumulator layout: position li, channels 32 cb + 8 j + 4 g + e)
  auto gate_rows = [&](const f32x16& ag, int cb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x4* po = reinterpret_cast<bf16x4*>(&XR[off128(rw + li, 4 * cb + j) + 4 * g]);
      const bf16x4 ov = *po;
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)(sigmoid_scaled(ag[4 * j + e]) * (float)ov[e]);
      *po = v;
    }
  };
  auto project = [&](const bf16* slab, const bf16x8 (&b)[8]) {
    f32x16 d = zero16();
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) d = mfma32(ld8(&slab[off128(li, 2 * kk + g)]), b[kk], d);
    return d;
  };

#pragma unroll 1
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * XT;
    progress_priority((tile - blockIdx.x) / gridDim.x, (ntiles - 1 - blockIdx.x) / gridDim.x + 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // own z rows and chunk-0 pieces landed
    __syncthreads();                                   // everyone's chunk-0 pieces landed
    // z in the accumulator layout (the residual of y)
    bf16x4 zres[4][4];
#pragma unroll
    for (int ot = 0; ot < 4; ++ot)
#pragma unroll
      for (int m = 0; m < 4; ++m)
        zres[ot][m] = *reinterpret_cast<const bf16x4*>(&XR[off128(rw + li, 4 * ot + m) + 4 * g]);
    // LN_pair(z) in place: the statistics and rounding of ln_swz, position by position
    {
      float pw[8], pb[8];
      const float* w_ = opaque(lnp_w);
      const float* b_ = opaque(lnp_b);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pw[e] = w_[8 * sub + e];
        pb[e] = b_[8 * sub + e];
      }
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        bf16* piece = &XR[off128(rw + 4 * it + p16, sub)];
        const bf16x8 raw = ld8(piece);
        float x[8], d2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (float)raw[e];
        const float mean = sum16(sum8(x)) * (1.f / 128.f);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[e] -= mean;
          d2[e] = x[e] * x[e];
        }
        const float rstd = __builtin_amdgcn_rsqf(sum16(sum8(d2)) * (1.f / 128.f) + eps_pair);
        bf16x8 y;
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = (bf16)(x[e] * rstd * pw[e] + pb[e]);
        *reinterpret_cast<bf16x8*>(piece) = y;
      }
    }
    bf16x8 xb[8];  // LN_pair(z) as the B operand: position li, k = 16 kk + 8 g .. + 7
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) xb[kk] = ld8(&XR[off128(rw + li, 2 * kk + g)]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // read before o overwrites the rows
    rows_dma(o, row0, rows, rw, xr_lds, lane);

    // lead chunk 0: gate rows 0-95
    {
      const TransitionChunk* cur = &W[k % NB];
      weight_dma<NW>(wpack, (0 + NB - 1) % NCH, w_lds + ((k + NB - 1) % NB) * sizeof(TransitionChunk), wave,
                     lane);
      f32x16 ag[3];
#pragma unroll
      for (int cb = 0; cb < 3; ++cb) ag[cb] = project(lead_slab(cur, cb), xb);
      wait_vm_lds<per>();  // the o rows landed (only the next chunk's pieces were issued after)
#pragma unroll
      for (int cb = 0; cb < 3; ++cb) gate_rows(ag[cb], cb);
      lead_end();
    }
    // lead chunk 1: gate rows 96-127, output rows 0-63
    bf16x8 gb[8];
    f32x16 ao[4];
    {
      const TransitionChunk* cur = &W[k % NB];
      weight_dma<NW>(wpack, (1 + NB - 1) % NCH, w_lds + ((k + NB - 1) % NB) * sizeof(TransitionChunk), wave,
                     lane);
      gate_rows(project(lead_slab(cur, 0), xb), 3);
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) gb[kk] = ld8(&XR[off128(rw + li, 2 * kk + g)]);
      ao[0] = project(lead_slab(cur, 1), gb);
      ao[1] = project(lead_slab(cur, 2), gb);
      lead_end();
    }
    // lead chunk 2: output rows 64-127, then y = z + projection into the rows
    {
      const TransitionChunk* cur = &W[k % NB];
      weight_dma<NW>(wpack, (2 + NB - 1) % NCH, w_lds + ((k + NB - 1) % NB) * sizeof(TransitionChunk), wave,
                     lane);
      ao[2] = project(lead_slab(cur, 0), gb);
      ao[3] = project(lead_slab(cur, 1), gb);
#pragma unroll
      for (int ot = 0; ot < 4; ++ot)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (bf16)(ao[ot][4 * m + e] + (float)zres[ot][m][e]);
          *reinterpret_cast<bf16x4*>(&XR[off128(rw + li, 4 * ot + m) + 4 * g]) = v;
        }
      lead_end();
    }
    // the last tile re-reads its own rows instead of a next tile's
    const int64_t next0 = tile + gridDim.x < ntiles ? row0 + (int64_t)gridDim.x * XT : row0;
    auto xdma = [&]() { rows_dma(z, next0, rows, rw, xr_lds, lane); };
    transition_tile<NW, NB, kLeadChunks, NCH>(XR, W, w_lds, wpack, ln_w, ln_b, out, rows, row0,
                                              1, eps, k, xdma, wave, lane);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS write may land after exit
}

// Workgroup shape: kTransNW waves of 32 positions, kTransNB chunk buffers, kTransWG
// workgroups per CU (LDS: kTransNB * 24 KB + kTransNW * 8 KB per workgroup).
#ifndef FFK_TRANSITION_SHAPE
#define FFK_TRANSITION_SHAPE 4, 2, 2
#endif
constexpr int kTransShape[3] = {FFK_TRANSITION_SHAPE};
constexpr int kTransNW = kTransShape[0], kTransNB = kTransShape[1], kTransWG = kTransShape[2];
static_assert(24 % kTransNW == 0 && kTransNB >= 2, "transition workgroup shape");

void launch_transition_pack(const float* wa, const float* wb, const float* ws, bf16* dst,
                            hipStream_t stream) {
  pack_transition<<<dim3(16 * kChunkElems / 256), 256, 0, stream>>>(wa, wb, ws, nullptr, nullptr,
                                                                    dst);  // one element per thread
}

void launch_attention_transition_pack(const float* wg, const float* wo, const float* wa,
                                      const float* wb, const float* ws, bf16* dst,
                                      hipStream_t stream) {
  pack_transition<<<dim3((16 + kLeadChunks) * kChunkElems / 256), 256, 0, stream>>>(wa, wb, ws, wg,
                                                                                   wo, dst);
}

void launch_transition(const TransitionArgs& a, hipStream_t stream) {
  constexpr int XT = 32 * kTransNW;
  const int64_t ntiles = (a.rows + XT - 1) / XT;
  const int64_t slots = (int64_t)cu_count() * kTransWG;
  const int grid = (int)(ntiles < slots ? ntiles : slots);
  transition_swiglu<kTransNW, kTransNB, kTransWG><<<dim3(grid), 64 * kTransNW, 0, stream>>>(
      a.x, a.ln_w, a.ln_b, a.w, a.out, a.rows, a.residual, a.eps);
}

void launch_attention_output_transition(const AttnTransitionArgs& a, hipStream_t stream) {
  constexpr int XT = 32 * kTransNW;
  const int64_t ntiles = (a.rows + XT - 1) / XT;
  const int64_t slots = (int64_t)cu_count() * kTransWG;
  const int grid = (int)(ntiles < slots ? ntiles : slots);
  attention_output_transition<kTransNW, kTransNB, kTransWG><<<dim3(grid), 64 * kTransNW, 0, stream>>>(
      a.z, a.o, a.lnp_w, a.lnp_b, a.ln_w, a.ln_b, a.w, a.out, a.rows, a.eps_pair, a.eps);
}

}  // namespace ffk
