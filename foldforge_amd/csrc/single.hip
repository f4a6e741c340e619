// Single-track kernels: attention with pair bias and the wide (non-128) SwiGLU transition.
//
// Shapes: tokens m = b * n + i (M = batch * n rows), single width cs (a multiple of 64),
// heads x dh with dh a multiple of 8 and at most 32. The pair input z is [batch, n, n, 128].
//
// Attention with pair bias (legacy/transformer.py:93-137 of the reference):
//   x = LN_single(s); q = (x W_q^T + b_q), k = x W_k^T, v = x W_v^T, g = sigmoid(x W_g^T + gb)
//   bias[h, i, j] = LN_pair(z[i, j]) . W_b[h]   (the pair norm has no offset)
//   o = softmax_j(q_i . k_j / sqrt(dh) + bias[h, i, j]) over valid keys j, 0 for an empty row
//   out = s + (g * o) W_out^T
// is run as: row_gemm<kEpiApb, kXLn> (LayerNorm prologue; q, k, v^T, gate) -> apb_pair_bias
// -> apb_attention (gate applied) -> row_gemm<kEpiResid>.
// The wide transition is row_gemm<kEpiSwiglu, kXLn> -> row_gemm<kEpiResid>.
// The same file holds row_stream, the streaming LayerNorm-fed token-row GEMM that the
// generic pair widths (template stacks, Chai-1's pair 256) run their projections on.
//
// Logits are carried in log2 units: q is scaled by log2(e) / sqrt(dh) and the pair-bias
// weights by log2(e), so the softmax uses exp2. Masked keys (and the padding keys past n)
// get the finite logit kMaskedLogit: their weight is exactly 0 once any valid key is seen.
#include <algorithm>
#include <type_traits>

#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

namespace {

constexpr float kMaskedLogit = -1e30f;

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)0.f;
  return r;
}

// Position of key `key` inside the v^T rows: index bits 2 and 3 exchanged, so that the 8
// consecutive positions a lane loads are the 8 keys its P^T operand holds.
__device__ __forceinline__ int vkey_pos(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

// ---------------------------------------------------------------------------- row GEMM
// D[o][m] = sum_k W[o][k] X[m][k] over 32 rows of X per workgroup: A = W rows (fp32 parameters,
// converted in registers), B = X rows. The workgroup's 8 waves cover NO output tiles of 32
// with KS waves each (NO * KS = 8): the KS waves of a tile split k in groups of 64 (part p
// takes groups p, p + KS, ...), keep the next group's global loads in flight while
// multiplying the current one, and add their partial tiles through LDS; part 0 runs the
// epilogue. For MFMA step t of a group, lane half g supplies k = 64 kg + 32 g + 8 t + (0..7)
// of both operands.
// Precision: activations enter as fp32 and are split into bf16 hi + lo (two MFMAs); the weights
// are rounded to bf16, or with w_split also split into hi + lo (a third MFMA, lo x hi: the
// products then carry about fp32 accuracy, the lo x lo term below it dropped). The single-track
// ops set w_split: their GEMMs are small and latency-bound, and a bf16 rounding of a weight is
// the same perturbation at every application of the block, so it moves the trunk's trajectory
// rather than averaging out.
// X sources: kXLn = LayerNorm of bf16 rows (ln_x [M][K], statistics and affine in fp32, the
// normalised tile staged in LDS once per workgroup as hi / lo rows); kXF32 = fp32 rows
// streamed from x32 [M][K].
// Epilogue: lane (li, g) holds token m0 + li and outputs o = 32 ot + 8 v + 4 g + e
// (acc[4 v + e]).

constexpr int kGemmWaves = 8;

size_t row_gemm_lds(int xsrc, int K, int no) {
  const size_t red = (size_t)(kGemmWaves - no) * 64 * 16 * sizeof(float);
  return xsrc == kXLn ? red + (size_t)2 * 32 * (K + 8) * sizeof(bf16) : red;
}

// The input row of logical row m under the row map a.tmap (see kMap* in ffk_kernels.h).
// The last workgroup's rows past M (the grid covers M rounded up to 32) read row M - 1: they
// are never stored, and an unclamped transposed map would read past the end of the input.
__device__ inline int64_t mapped_row(const RowGemmArgs& a, int64_t m) {
  m = min(m, a.M - 1);
  if (a.tmap == kMapPairT) {
    const int64_t nn = (int64_t)a.n * a.n;
    const int64_t b = m / nn, rem = m - b * nn;
    const int r = (int)(rem / a.n), j = (int)(rem - (int64_t)r * a.n);
    return (b * a.n + j) * a.n + r;
  }
  if (a.tmap == kMapPadKeys || a.tmap == kMapPadKeysT) {
    const int64_t bn = m / a.np;
    const int j = min((int)(m - bn * a.np), a.n - 1);
    if (a.tmap == kMapPadKeys) return bn * a.n + j;
    const int64_t b = bn / a.n;
    return (b * a.n + j) * a.n + (bn - b * a.n);
  }
  if (a.tmap == kMapGridOut || a.tmap == kMapGridIn) {
    const int64_t gg = (int64_t)a.npm * a.npm;
    const int64_t b = m / gg, rem = m - b * gg;
    const int i = min((int)(rem / a.npm), a.n - 1), k = min((int)(rem % a.npm), a.n - 1);
    return a.tmap == kMapGridOut ? (b * a.n + i) * a.n + k : (b * a.n + k) * a.n + i;
  }
  return m;
}

// kEpiOpm: the MSA row read by logical row m = (b n + j) sp + s (rows past the depth repeat
// the last one; their projection is zeroed).
__device__ inline int64_t opm_msa_row(const RowGemmArgs& a, int64_t m) {
  m = min(m, a.M - 1);
  const int64_t bj = m / a.sp;
  const int s = min((int)(m - bj * a.sp), a.depth - 1);
  const int64_t b = bj / a.n;
  const int j = (int)(bj - b * a.n);
  return (b * a.depth + s) * a.n + j;
}

// kEpiApb's width of one projection (q, k, v and, with apb_no_gate == 0, the gate).
__device__ __forceinline__ int apb_width(const RowGemmArgs& a) { return a.O / (a.apb_no_gate ? 3 : 4); }

// The weight row (fp32, K values) multiplied by row li of output tile ot, and the tile's
// segment and first channel as the epilogue reads them (packed tiles: see kEpiTrimul and
// kEpiSwiglu below).
template <int EPI>
__device__ inline const float* tile_weight_row(const RowGemmArgs& a, int ot, int li, int& seg, int& cbase) {
  const float* wr;
  seg = 0;
  cbase = 0;
  if (EPI == kEpiApb) {
    const int cs = apb_width(a);
    seg = (ot * 32) / cs;
    cbase = ot * 32 - seg * cs;
    const float* base = seg == 0 ? a.w0 : seg == 1 ? a.w1 : seg == 2 ? a.w2 : a.w3;
    wr = base + (int64_t)(cbase + li) * a.K;
  } else if (EPI == kEpiPwa || EPI == kEpiOpm) {
    const int hd = a.O / 2;
    seg = (ot * 32) / hd;
    cbase = ot * 32 - seg * hd;
    wr = (seg == 0 ? a.w0 : a.w1) + (int64_t)(cbase + li) * a.K;
  } else if (EPI == kEpiTrimul) {
    // packed tile: rows 0-15 are projection rows cbase .. cbase + 15 of one side, rows 16-31 the
    // matching gate rows
    const int tps = a.O / 64;  // tiles per side: hid / 16
    seg = ot / tps;
    cbase = (ot - seg * tps) * 16;
    const float* base = li < 16 ? (seg == 0 ? a.w0 : a.w1) : (seg == 0 ? a.w2 : a.w3);
    wr = base + (int64_t)(cbase + (li & 15)) * a.K;
  } else if (EPI == kEpiSwiglu) {
    // packed tile: rows 0-15 are expand_a rows 16 ot .., rows 16-31 the expand_b rows alike
    wr = (li < 16 ? a.w0 : a.w1) + (int64_t)(ot * 16 + (li & 15)) * a.K;
  } else {
    wr = a.w0 + (int64_t)(ot * 32 + li) * a.K;
  }
  return wr;
}

__device__ __forceinline__ int stage_row(int r) { return r ^ ((r >> 2) & 1); }

// A 32-row tile inside one run of an epilogue's row decomposition m = q L + rem (kEpiApb's flash
// layout: L = np, q = b n + r, rem = the key j; kEpiTrimul: L = npm^2, q = b), computed once per
// tile from its first row (uniform across the wave) instead of per lane and output tile.
struct TileRun {
  int64_t m0, q, rem0, b;
  int r;
};
template <int EPI>
__device__ __forceinline__ TileRun tile_run(const RowGemmArgs& a, int64_t m0) {
  TileRun t{};
  t.m0 = m0;
  const int64_t len = EPI == kEpiTrimul ? (int64_t)a.npm * a.npm
                      : EPI == kEpiOpm   ? (int64_t)a.sp
                      : EPI == kEpiPwa   ? (int64_t)a.n
                                         : (int64_t)a.np;
  t.q = m0 / len;
  t.rem0 = m0 - t.q * len;
  if (EPI == kEpiApb) {
    t.b = t.q / a.n;
    t.r = (int)(t.q - t.b * a.n);
  }
  return t;
}

// The per-row value an epilogue reads from memory, once per row rather than per output tile:
// kEpiTrimul's pair mask factor m_i m_k (symmetric, so the same for the transposed read).
template <int EPI>
__device__ __forceinline__ float row_pre(const RowGemmArgs& a, const int64_t m) {
  if (EPI == kEpiTrimul) {
    const int64_t gg = (int64_t)a.npm * a.npm;
    const int64_t b = m / gg, rem = m - b * gg;
    const int i = (int)(rem / a.npm), k = (int)(rem - (int64_t)i * a.npm);
    return i < a.n && k < a.n && a.mask[b * a.n + i] && a.mask[b * a.n + k] ? 1.f : 0.f;
  }
  return 0.f;
}

// Epilogue of output tile ot for logical row m (< M): lane half g holds outputs
// 32 ot + 8 v + 4 g + e in acc[4 v + e]. lb: the per-output biases (q_bias / gate_b of kEpiApb,
// bias_out of kEpiResid) staged in LDS by output index, or NULL to read them from the arguments.
// The loads an epilogue needs are all issued before its first store.
// stage: a wave-private LDS tile of 32 x 32 bf16 (NULL: none), through which the
// position-contiguous outputs (kEpiApb's flash-layout v^T, kEpiTrimul's channel planes) are
// transposed and written as 16-byte pieces of 64-byte runs; tr: the tile's run (tile_run),
// required with stage, whose 32 rows must then be consecutive positions of one run
// (np % 32 == 0), so those epilogues take both only from the streaming kernel. ypre: the yin
// values of kEpiGateResid, loaded by the caller (NULL: loaded here). rpre: the
// residual values of kEpiResid and kEpiGateResid, loaded by the caller (NULL: loaded here); both
// as the two 16-byte pieces (acc_pieces) of the lane. Channel row r of the tile sits at LDS row
// stage_row(r), which puts the rows the two lane halves write at once (r, r + 4) on different
// banks.
template <int EPI>
__device__ __forceinline__ void row_epilogue(const RowGemmArgs& a, const f32x16& acc, const int64_t m, const int ot,
                                    const int seg, const int cbase, const int g, const float* lb,
                                    const float pre, bf16* stage = nullptr,
                                    const TileRun* tr = nullptr, const bf16x8* rpre = nullptr,
                                    const bf16x8* ypre = nullptr) {
  // the bias of output o (global index gi of src when not staged)
  auto obias = [&](int o, const float* src, int gi) { return lb ? lb[o] : (src ? src[gi] : 0.f); };
  if (EPI == kEpiApb && a.flash_rows > 0) {
    const int cs = apb_width(a);
    int64_t bn, b;
    int j, r;
    if (tr) {
      bn = tr->q;
      j = (int)(tr->rem0 + (m - tr->m0));
      b = tr->b;
      r = tr->r;
    } else {
      bn = m / a.np;
      j = (int)(m - bn * a.np);
      b = bn / a.n;
      r = (int)(bn - b * a.n);
    }
    if (seg != 2) {
      // q, k (the flash layouts) and the gate (token rows) as 16-byte pieces of 8 channels of
      // one head (dh % 8 == 0)
      float y[2][8];
      acc_pieces(acc, g, y);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int c = cbase + 8 * (2 * k + g);
        const int o0 = 32 * ot + 8 * (2 * k + g);
        const int hh = c / a.dh, d0 = c - hh * a.dh;
        const int64_t blk = (b * a.heads + hh) * a.flash_rows + r;  // the (b, h, r) block
        bf16x8 o;
        if (seg == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (bf16)((y[k][e] + obias(o0 + e, a.q_bias, c + e)) * a.q_scale);
          *reinterpret_cast<bf16x8*>(a.q + (blk * a.np + j) * a.dh + d0) = o;
        } else if (seg == 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (bf16)y[k][e];
          *reinterpret_cast<bf16x8*>(a.k + (blk * a.np + j) * a.dh + d0) = o;
        } else if (j < a.n) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            o[e] = (bf16)sigmoid_scaled((y[k][e] + obias(o0 + e, a.gate_b, c + e) + a.gate_bias) * -kLog2e);
          *reinterpret_cast<bf16x8*>(a.gate + (bn * a.n + j) * cs + c) = o;
        }
      }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int c = cbase + 8 * v + 4 * g;  // 4 channels of one head (dh % 4 == 0)
      const int hh = c / a.dh, d0 = c - hh * a.dh;
      const int64_t blk = (b * a.heads + hh) * a.flash_rows + r;  // the (b, h, r) block
      float y[4] = {acc[4 * v], acc[4 * v + 1], acc[4 * v + 2], acc[4 * v + 3]};
      if (seg == 2) {
        const int pos = vkey_pos(j);
        if (stage) {
#pragma unroll
          for (int e = 0; e < 4; ++e) stage[stage_row(8 * v + 4 * g + e) * 32 + (pos & 31)] = (bf16)y[e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            a.vt[blk * a.dh * a.np + (pos >> 5) * 32 * a.dh + (d0 + e) * 32 + (pos & 31)] = (bf16)y[e];
        }
      }
    }
    if (seg == 2 && stage) {
      // the tile's 32 v^T rows (tile-local channel r) of this run of 32 positions: lane L
      // writes pieces L and L + 64 (row piece / 4, 8 positions each)
      __builtin_amdgcn_wave_barrier();
      const int lane = 32 * g + (int)(m - tr->m0);
      const int jt = (int)tr->rem0;
      const int64_t bt = tr->b;
      const int rt = tr->r;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int piece = lane + 64 * u, r = piece >> 2, part = piece & 3;
        const int c = cbase + r, hh = c / a.dh, d = c - hh * a.dh;
        const int64_t blk = (bt * a.heads + hh) * a.flash_rows + rt;
        // (v^T blocked by 32 keys; jt is a multiple of 32)
        *reinterpret_cast<bf16x8*>(a.vt + blk * a.dh * a.np + jt * a.dh + d * 32 + 8 * part) =
            *reinterpret_cast<const bf16x8*>(stage + stage_row(r) * 32 + 8 * part);
      }
      __builtin_amdgcn_wave_barrier();
    }
  } else if (EPI == kEpiApb) {
    const int cs = apb_width(a);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int c = cbase + 8 * v + 4 * g;
      const int o0 = 32 * ot + 8 * v + 4 * g;
      float y0 = acc[4 * v], y1 = acc[4 * v + 1], y2 = acc[4 * v + 2], y3 = acc[4 * v + 3];
      if (seg == 0) {
        y0 += obias(o0, a.q_bias, c);
        y1 += obias(o0 + 1, a.q_bias, c + 1);
        y2 += obias(o0 + 2, a.q_bias, c + 2);
        y3 += obias(o0 + 3, a.q_bias, c + 3);
        y0 *= a.q_scale;
        y1 *= a.q_scale;
        y2 *= a.q_scale;
        y3 *= a.q_scale;
        store4(a.q + m * cs + c, y0, y1, y2, y3);
      } else if (seg == 1) {
        store4(a.k + m * cs + c, y0, y1, y2, y3);
      } else if (seg == 2) {
        const int64_t b = m / a.n;
        const int key = (int)(m - b * a.n);
        const int pos = vkey_pos(key);
        const float ys[4] = {y0, y1, y2, y3};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int hh = (c + e) / a.dh, d = (c + e) - hh * a.dh;
          a.vt[((b * a.heads + hh) * a.dh + d) * a.np + pos] = (bf16)ys[e];
        }
      } else {
        const float nb = -kLog2e;
        y0 += obias(o0, a.gate_b, c);
        y1 += obias(o0 + 1, a.gate_b, c + 1);
        y2 += obias(o0 + 2, a.gate_b, c + 2);
        y3 += obias(o0 + 3, a.gate_b, c + 3);
        y0 = sigmoid_scaled((y0 + a.gate_bias) * nb);
        y1 = sigmoid_scaled((y1 + a.gate_bias) * nb);
        y2 = sigmoid_scaled((y2 + a.gate_bias) * nb);
        y3 = sigmoid_scaled((y3 + a.gate_bias) * nb);
        store4(a.gate + m * cs + c, y0, y1, y2, y3);
      }
    }
  } else if (EPI == kEpiPwa) {
    const int hd = a.O / 2;
    const int64_t bs = m / a.n;  // b S + s
    const int j = (int)(m - bs * a.n);
    const int64_t b = bs / a.depth, srow = bs - b * a.depth;
    if (seg == 0 && stage) {
      // v^T: the tile's 32 channel rows of this run of 32 tokens (n % 32 == 0), transposed
      // through the wave's LDS tile and written as 16-byte pieces of 64-byte runs
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int e = 0; e < 4; ++e) stage[stage_row(8 * v + 4 * g + e) * 32 + (j & 31)] = (bf16)acc[4 * v + e];
      __builtin_amdgcn_wave_barrier();
      const int lane = 32 * g + (int)(m - tr->m0);
      const int64_t bt = tr->q / a.depth, st = tr->q - bt * a.depth;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int piece = lane + 64 * u, r = piece >> 2, part = piece & 3;
        const int c = cbase + r, hh = c / a.dh, d = c - hh * a.dh;
        *reinterpret_cast<bf16x8*>(a.vt + (((bt * a.heads + hh) * a.depth + st) * a.dh + d) * a.np +
                                   tr->rem0 + 8 * part) =
            *reinterpret_cast<const bf16x8*>(stage + stage_row(r) * 32 + 8 * part);
      }
      __builtin_amdgcn_wave_barrier();
      return;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int c = cbase + 8 * v + 4 * g;  // 4 channels of one head (dh % 4 == 0)
      float y[4] = {acc[4 * v], acc[4 * v + 1], acc[4 * v + 2], acc[4 * v + 3]};
      if (seg == 0) {
        const int hh = c / a.dh, d0 = c - hh * a.dh;
        bf16* dst = a.vt + (((b * a.heads + hh) * a.depth + srow) * a.dh + d0) * a.np + j;
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(int64_t)e * a.np] = (bf16)y[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = sigmoid_scaled(-kLog2e * y[e]);
        store4(a.gate + m * hd + c, y[0], y[1], y[2], y[3]);
      }
    }
  } else if (EPI == kEpiOpm) {
    const int64_t bj = m / a.sp;
    const int s = (int)(m - bj * a.sp);
    const int64_t b = bj / a.n;
    const int j = (int)(bj - b * a.n);
    const float keep = s < a.depth && a.rows_mask[(b * a.depth + s) * a.n + j] ? 1.f : 0.f;
    const float* bias = seg == 0 ? a.bias0 : a.bias1;
    const int hd = a.O / 2;  // channels a side (32; Chai-1's grouped form 64)
    bf16* dst = (seg == 0 ? a.lt : a.rt) + bj * hd * a.sp + s;
    if (stage) {
      // the tile's 32 channel rows of this run of 32 MSA rows, transposed through the wave's
      // LDS tile and written as 16-byte pieces of 64-byte runs (lane L: pieces L and L + 64)
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = cbase + 8 * v + 4 * g + e;
          stage[stage_row(8 * v + 4 * g + e) * 32 + (s & 31)] =
              (bf16)((acc[4 * v + e] + (bias ? bias[c] : 0.f)) * keep);
        }
      __builtin_amdgcn_wave_barrier();
      const int lane = 32 * g + (int)(m - tr->m0);
      bf16* run = (seg == 0 ? a.lt : a.rt) + tr->q * hd * a.sp + tr->rem0;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int piece = lane + 64 * u, r = piece >> 2, part = piece & 3;
        *reinterpret_cast<bf16x8*>(run + (int64_t)(cbase + r) * a.sp + 8 * part) =
            *reinterpret_cast<const bf16x8*>(stage + stage_row(r) * 32 + 8 * part);
      }
      __builtin_amdgcn_wave_barrier();
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = cbase + 8 * v + 4 * g + e;
          dst[(int64_t)c * a.sp] = (bf16)((acc[4 * v + e] + (bias ? bias[c] : 0.f)) * keep);
        }
    }
    if (seg == 0 && cbase == 0 && g == 0) a.mt[bj * a.sp + s] = (bf16)keep;
  } else if (EPI == kEpiTrimul) {
    const int hid = a.O / 4;
    const int64_t gg = (int64_t)a.npm * a.npm;
    const int64_t b = tr ? tr->q : m / gg;
    const int64_t rem = tr ? tr->rem0 + (m - tr->m0) : m - b * gg;
    const float keep = pre;  // the pair mask factor (row_pre)
    bf16* plane = (seg == 0 ? a.pa : a.pb) + b * hid * gg + rem;
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = cbase + 8 * v + 4 * g + e;
        const float proj = acc[4 * v + e] * keep;  // masked before the gate, as the reference
        const bf16 y = (bf16)(proj * sigmoid_scaled(-kLog2e * acc[8 + 4 * v + e]));
        if (stage)
          stage[stage_row(8 * v + 4 * g + e) * 32 + (int)(m - tr->m0)] = y;
        else
          plane[(int64_t)c * gg] = y;
      }
    if (stage) {
      // the tile's 16 channel rows of 32 positions: lane L writes piece L (row L / 4)
      __builtin_amdgcn_wave_barrier();
      const int lane = 32 * g + (int)(m - tr->m0);
      const int r = lane >> 2, part = lane & 3;
      const int64_t bt = tr->q, remt = tr->rem0;
      *reinterpret_cast<bf16x8*>((seg == 0 ? a.pa : a.pb) + bt * hid * gg + (int64_t)(cbase + r) * gg + remt +
                                 8 * part) = *reinterpret_cast<const bf16x8*>(stage + stage_row(r) * 32 + 8 * part);
      __builtin_amdgcn_wave_barrier();
    }
  } else if (EPI == kEpiStoreY) {
    float y[2][8];
    acc_pieces(acc, g, y);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)y[k][e];
      *reinterpret_cast<bf16x8*>(a.hy + m * a.O + ot * 32 + 8 * (2 * k + g)) = o;
    }
  } else if (EPI == kEpiGateResid) {
    bf16x8 yv[2], rv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int c = ot * 32 + 8 * (2 * k + g);
      yv[k] = ypre ? ypre[k] : *reinterpret_cast<const bf16x8*>(a.yin + m * a.O + c);
      if (a.residual) rv[k] = rpre ? rpre[k] : *reinterpret_cast<const bf16x8*>(a.res + m * a.O + c);
    }
    float y[2][8];
    acc_pieces(acc, g, y);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = (float)yv[k][e] * sigmoid_scaled(-kLog2e * y[k][e]);
        if (a.residual) t += (float)rv[k][e];
        o[e] = (bf16)t;
      }
      *reinterpret_cast<bf16x8*>(a.out + m * a.O + ot * 32 + 8 * (2 * k + g)) = o;
    }
  } else if (EPI == kEpiLinear) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int c = ot * 32 + 8 * v + 4 * g;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = acc[4 * v + e] + (a.bias_out ? a.bias_out[c + e] : 0.f);
        if (a.act == kActSigmoid)
          t = sigmoid_scaled(-kLog2e * t);
        else if (a.act == kActSilu)
          t = t * sigmoid_scaled(-kLog2e * t);
        else if (a.act == kActRelu)
          t = fmaxf(t, 0.f);
        y[e] = t;
      }
      if (a.y_f32) {
        const f32x4 yv = {y[0], y[1], y[2], y[3]};
        *reinterpret_cast<f32x4*>(static_cast<float*>(a.y) + m * a.O + c) = yv;
      } else {
        store4(static_cast<bf16*>(a.y) + m * a.O + c, y[0], y[1], y[2], y[3]);
      }
    }
  } else if (EPI == kEpiSwiglu) {
    const int hid = a.O / 2;
    f32x4 y[2];
#pragma unroll
    for (int v = 0; v < 2; ++v)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float av = acc[4 * v + e], bv = acc[8 + 4 * v + e];
        y[v][e] = av * sigmoid_scaled(-kLog2e * av) * bv;
      }
    if (a.h16) {
      // hidden 8 v + 4 g + 0..3 in y[v]: one exchange gives half g the 8 channels 8 g .. 8 g + 7
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t send = __float_as_uint(g ? y[0][e] : y[1][e]);
        const auto sw = __builtin_amdgcn_permlane32_swap(send, send, false, false);
        const float recv = __uint_as_float(g ? sw[0] : sw[1]);
        o[e] = (bf16)(g ? recv : y[0][e]);
        o[4 + e] = (bf16)(g ? y[1][e] : recv);
      }
      *reinterpret_cast<bf16x8*>(a.h16 + m * hid + ot * 16 + 8 * g) = o;
    } else {
#pragma unroll
      for (int v = 0; v < 2; ++v)
        *reinterpret_cast<f32x4*>(a.h32 + m * hid + ot * 16 + 8 * v + 4 * g) = y[v];
    }
  } else {
    bf16x8 rv[2];
    if (a.residual) {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        rv[k] = rpre ? rpre[k] : *reinterpret_cast<const bf16x8*>(a.res + m * a.O + ot * 32 + 8 * (2 * k + g));
    }
    float y[2][8];
    acc_pieces(acc, g, y);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int c = ot * 32 + 8 * (2 * k + g);
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = y[k][e] + obias(c + e, a.bias_out, c + e);
        if (a.residual) t += (float)rv[k][e];
        o[e] = (bf16)t;
      }
      *reinterpret_cast<bf16x8*>(a.out + m * a.O + c) = o;
    }
  }
}

template <int EPI, int XSRC, int NO>
__global__ __launch_bounds__(512) void row_gemm(RowGemmArgs a) {
  constexpr int KS = kGemmWaves / NO;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  float* red = reinterpret_cast<float*>(smem);  // [NO][KS - 1][64][16]
  bf16* xs_hi = reinterpret_cast<bf16*>(smem + (kGemmWaves - NO) * 64 * 16 * sizeof(float));
  const int xstride = a.K + 8;  // [32][K + 8]: rows 16 bytes apart modulo 256, conflict-free
  bf16* xs_lo = xs_hi + 32 * xstride;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, g = lane >> 5;
  const int osub = wave / KS, part = wave % KS;
  const int ot = blockIdx.y * NO + osub;
  const bool active = ot * 32 < a.O;
  const int64_t m0 = (int64_t)blockIdx.x * 32;
  const int G = a.K / 64;

  int seg, cbase;
  const float* wr = tile_weight_row<EPI>(a, ot, li, seg, cbase);
  wr += 32 * g;
  const float* x32 = a.x32 + mapped_row(a, m0 + li) * a.K + 32 * g;

  f32x16 acc = zero16();
  f32x4 wc[8], wn[8], xc[8], xn[8];
  auto fetch = [&](int kg, f32x4* w, f32x4* x) {
#pragma unroll
    for (int q = 0; q < 8; ++q) w[q] = *reinterpret_cast<const f32x4*>(wr + 64 * kg + 4 * q);
    if (XSRC == kXF32) {
#pragma unroll
      for (int q = 0; q < 8; ++q) x[q] = *reinterpret_cast<const f32x4*>(x32 + 64 * kg + 4 * q);
    }
  };
  if (active && part < G) fetch(part, wc, xc);

  if (XSRC == kXLn) {
    // thread t normalises row t / 16, chunks (t % 16) + 16 i of 8 channels, held in registers;
    // the 16 threads of a row are consecutive lanes, joined by DPP sums
    constexpr int kMaxChunks = kLnGemmMaxK / 128;
    const int r = tid >> 4, pc = tid & 15;
    const int nc = a.K / 8;
    const bf16* xr = a.ln_x + (EPI == kEpiOpm ? opm_msa_row(a, m0 + r) : mapped_row(a, m0 + r)) * a.K;
    bf16x8 xv[kMaxChunks];
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i)
      if (pc + 16 * i < nc) xv[i] = ld8(xr + 8 * (pc + 16 * i));
    float s1 = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i)
      if (pc + 16 * i < nc)
#pragma unroll
        for (int e = 0; e < 8; ++e) s1 += (float)xv[i][e];
    const float mean = a.ln_plain ? 0.f : sum16(s1) / (float)a.K;
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i)
      if (pc + 16 * i < nc)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = (float)xv[i][e] - mean;
          s2 += d * d;
        }
    const float eps = a.eps_dev ? *a.eps_dev : a.eps;
    const float rstd = a.ln_plain ? 1.f : __builtin_amdgcn_rsqf(sum16(s2) / (float)a.K + eps);
    const f32x4 one4 = {1.f, 1.f, 1.f, 1.f}, zero4 = {0.f, 0.f, 0.f, 0.f};
    const bool has_w = a.ln_w != nullptr && !a.ln_plain, has_b = a.ln_b != nullptr && !a.ln_plain;
#pragma unroll
    for (int i = 0; i < kMaxChunks; ++i) {
      if (pc + 16 * i < nc) {
        const int c = 8 * (pc + 16 * i);
        const f32x4 w0 = has_w ? *reinterpret_cast<const f32x4*>(a.ln_w + c) : one4;
        const f32x4 w1 = has_w ? *reinterpret_cast<const f32x4*>(a.ln_w + c + 4) : one4;
        const f32x4 b0 = has_b ? *reinterpret_cast<const f32x4*>(a.ln_b + c) : zero4;
        const f32x4 b1 = has_b ? *reinterpret_cast<const f32x4*>(a.ln_b + c + 4) : zero4;
        f32x4 y0, y1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          y0[e] = ((float)xv[i][e] - mean) * rstd * w0[e] + b0[e];
          y1[e] = ((float)xv[i][4 + e] - mean) * rstd * w1[e] + b1[e];
        }
        bf16x8 hi, lo;
        split8(y0, y1, hi, lo);
        *reinterpret_cast<bf16x8*>(xs_hi + r * xstride + c) = hi;
        *reinterpret_cast<bf16x8*>(xs_lo + r * xstride + c) = lo;
      }
    }
    __syncthreads();
  }

  if (active) {
    for (int kg = part; kg < G; kg += KS) {
      const bool more = kg + KS < G;
      if (more) fetch(kg + KS, wn, xn);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x8 whi, wlo, xhi, xlo;
        split8(wc[2 * t], wc[2 * t + 1], whi, wlo);
        if (XSRC == kXLn) {
          const int k = 64 * kg + 32 * g + 8 * t;
          xhi = *reinterpret_cast<const bf16x8*>(xs_hi + li * xstride + k);
          xlo = *reinterpret_cast<const bf16x8*>(xs_lo + li * xstride + k);
        } else {
          split8(xc[2 * t], xc[2 * t + 1], xhi, xlo);
        }
        acc = mfma32(whi, xlo, acc);
        acc = mfma32(whi, xhi, acc);
        if (a.w_split) acc = mfma32(wlo, xhi, acc);
      }
      if (more) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          wc[q] = wn[q];
          xc[q] = xn[q];
        }
      }
    }
  }
  if (KS > 1) {
    if (part > 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((osub * (KS - 1) + part - 1) * 64 + lane) * 16 + r] = acc[r];
    }
    __syncthreads();
    if (part != 0) return;
#pragma unroll
    for (int w = 0; w < KS - 1; ++w)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += red[((osub * (KS - 1) + w) * 64 + lane) * 16 + r];
  }

  const int64_t m = m0 + li;
  if (!active || m >= a.M) return;
  row_epilogue<EPI>(a, acc, m, ot, seg, cbase, g, nullptr, row_pre<EPI>(a, m));
}

// ---------------------------------------------------------------------------- streaming row GEMM
// The products and epilogues of row_gemm for rows of K = 64 to 512 channels, as a persistent
// kernel: each workgroup converts the weights to bf16 once (LDS, in output-tile order, rows
// K + 8 elements apart so that the operand reads of 16 rows hit distinct banks), then every
// wave walks whole 32-row tiles on its own, with no barrier in the loop. With gridDim.y > 1 the
// output tiles are split into that many equal parts, one per grid row (wide outputs: each
// workgroup then holds a part of the weights and more workgroups fit on a CU). The next tile's input
// rows are loaded while the current one is normalised, multiplied for all O / 32 output tiles
// and stored by the epilogue of each output tile. Rows of up to 128 channels enter the MFMAs as
// bf16 hi + lo (as row_gemm); LayerNorm-fed rows of 256 as the rounded bf16 normalisation (as
// the reference's bf16 LayerNorm output), and 512-channel (plain bf16) rows are held in one
// register buffer, loaded after the last product of the previous tile.
// Lane (li, g) holds row li's channels (K / 2) g .. (K / 2) g + K / 2 - 1; MFMA step s takes
// channels (K / 2) g + 8 s .. + 7 of both operands.
// Waves per workgroup: 4, and 8 (two per SIMD, sharing a weight image of up to 154 KiB, one
// workgroup per CU) for rows of 256 channels or more.
__host__ __device__ constexpr int stream_waves(int K) { return K >= 256 ? 8 : 4; }

// LDS of one workgroup holding the weight rows of Op of the O outputs.
size_t row_stream_lds(int K, int O, int Op) {
  return (size_t)Op * (K + 8) * sizeof(bf16) + (size_t)(2 * K + O) * sizeof(float) +
         (size_t)stream_waves(K) * 32 * 32 * sizeof(bf16);
}

template <int EPI, int XSRC, int K>
__global__ __launch_bounds__(64 * stream_waves(K)) void row_stream(RowGemmArgs a) {
  constexpr int kStreamWaves = stream_waves(K);
  constexpr int KS = K / 16;  // MFMA steps
  constexpr int KH = K / 2;   // channels per lane
  constexpr int WS = K + 8;   // LDS row stride of the weight image (elements)
  constexpr bool BF = XSRC != kXF32;                // bf16 input rows
  constexpr int NX = BF ? KS : 2 * KS;              // 16-byte input pieces per lane
  constexpr bool LO = XSRC != kXBf16 && K <= 128;   // activations as bf16 hi + lo
  // the gate / residual epilogue of wide rows loads every output tile's operands (up to 128
  // VGPRs) at the start of a row tile instead of a second input buffer
  constexpr bool GR = EPI == kEpiGateResid && K >= 256;
  constexpr bool DB = NX <= 16 && !GR;              // two input buffers (64 VGPRs each at most)
  using XT = typename std::conditional<BF, bf16x8, f32x4>::type;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int nt = a.O / 32 / (int)gridDim.y;  // output tiles of this workgroup's part
  const int ot0 = (int)blockIdx.y * nt;
  bf16* wl = reinterpret_cast<bf16*>(smem);  // [nt][32][WS]: output tiles ot0 ..
  float* lnp = reinterpret_cast<float*>(smem + (size_t)nt * 32 * WS * sizeof(bf16));  // weight, offset
  float* lb = lnp + 2 * K;  // per-output biases (row_epilogue)
  // this wave's transpose tile (row_epilogue), for the epilogues that write position runs
  bf16* stage = reinterpret_cast<bf16*>(lb + a.O) + (threadIdx.x >> 6) * 32 * 32;
  const bool staged = (EPI == kEpiTrimul || EPI == kEpiOpm || (EPI == kEpiApb && a.flash_rows > 0) ||
                       (EPI == kEpiPwa && a.n % 32 == 0)) &&
                      a.M % 32 == 0;
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (int idx = tid; idx < nt * 32 * (K / 8); idx += 64 * kStreamWaves) {
    const int row = idx / (K / 8), ch = 8 * (idx % (K / 8));
    int seg, cbase;
    const float* wr = tile_weight_row<EPI>(a, ot0 + (row >> 5), row & 31, seg, cbase);
    *reinterpret_cast<bf16x8*>(wl + row * WS + ch) = cvt8(wr + ch);
  }
  for (int o = tid; o < a.O; o += 64 * kStreamWaves) {
    float v = 0.f;
    if (EPI == kEpiApb) {
      const int cs = apb_width(a), seg = o / cs, c = o - seg * cs;
      if (seg == 0 && a.q_bias) v = a.q_bias[c];
      if (seg == 3 && a.gate_b) v = a.gate_b[c];
    } else if (EPI == kEpiResid && a.bias_out) {
      v = a.bias_out[o];
    }
    lb[o] = v;
  }
  if (XSRC == kXLn) {
    const bool plain = a.ln_plain != 0;
    for (int c = tid; c < K; c += 64 * kStreamWaves) {
      lnp[c] = a.ln_w && !plain ? a.ln_w[c] : 1.f;
      lnp[K + c] = a.ln_b && !plain ? a.ln_b[c] : 0.f;
    }
  }
  __syncthreads();

  const int64_t tiles = (a.M + 31) / 32;
  const int64_t stride = (int64_t)gridDim.x * kStreamWaves;
  int64_t t = (int64_t)blockIdx.x * kStreamWaves + wave;
  if (t >= tiles) return;
  const float eps = XSRC == kXLn && a.eps_dev ? *a.eps_dev : a.eps;

  // the input rows of a tile (a tile past the end re-reads the last one, so every load stays
  // inside the input)
  auto fetch = [&](XT* x, int64_t tile) __attribute__((always_inline)) {
    const int64_t tt = tile < tiles ? tile : tiles - 1;
    const int64_t row = EPI == kEpiOpm ? opm_msa_row(a, tt * 32 + li) : mapped_row(a, tt * 32 + li);
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      if (BF)
        x[i] = *reinterpret_cast<const XT*>(a.ln_x + row * K + KH * g + 8 * i);
      else
        x[i] = *reinterpret_cast<const XT*>(a.x32 + row * K + KH * g + 4 * i);
    }
  };
  auto process = [&](XT* x, int64_t tile) __attribute__((always_inline)) {
    // GR: the epilogue operands of the first GRS output tiles, loaded first: their wait then
    // comes after the normalisation and the first products, not right behind the previous
    // tile's stores (vmcnt counts stores too). Tiles GRS .. 7 reuse the slots of tiles 0, 1,
    // loaded once those are consumed (all 8 at once would exceed the register file).
    constexpr int GRS = 6;
    bf16x8 gy[GR ? GRS : 1][2], gr[GR ? GRS : 1][2];
    const int64_t mg = tile * 32 + li < a.M ? tile * 32 + li : a.M - 1;
    auto gr_load = [&](int u, bf16x8 (&yv)[2], bf16x8 (&rv)[2]) __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int64_t at = mg * a.O + (ot0 + u) * 32 + 8 * (2 * k + g);
        yv[k] = *reinterpret_cast<const bf16x8*>(a.yin + at);
        if (a.residual) rv[k] = *reinterpret_cast<const bf16x8*>(a.res + at);
      }
    };
    if constexpr (GR) {
#pragma unroll
      for (int u = 0; u < GRS; ++u)
        if (u < nt) gr_load(u, gy[u], gr[u]);
    }
    // the MFMA operands: hi + lo of the activations (LO), else the rows of x themselves
    // (kXLn: normalised in place)
    bf16x8 xh[LO ? KS : 1], xl[LO ? KS : 1];
    if (XSRC == kXBf16) {
    } else if (XSRC == kXLn) {
      float s1 = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) s1 += (float)x[s][e];
      const bool plain = a.ln_plain != 0;
      const float mean = plain ? 0.f : pair_sum(s1) * (1.f / K);
      // (K = 256: each pass converts the bf16 rows again; 128 converted values per lane held
      // from one pass to the next would not fit in registers)
      if constexpr (!LO)
#pragma unroll
        for (int s = 0; s < KS; ++s) asm volatile("" : "+v"(x[s]));
      float s2 = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = (float)x[s][e] - mean;
          s2 += d * d;
        }
      const float rstd = plain ? 1.f : __builtin_amdgcn_rsqf(pair_sum(s2) * (1.f / K) + eps);
      if constexpr (!LO)
#pragma unroll
        for (int s = 0; s < KS; ++s) asm volatile("" : "+v"(x[s]));
      const float mr = -mean * rstd;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        // read per tile: held across the loop, the affine would take K registers (K = 256: the
        // offset also waits for the previous step's values, so that the scheduler cannot issue
        // every step's affine reads at once)
        int c = KH * g + 8 * s;
        if constexpr (!LO) {
          if (s > 0)
            asm volatile("" : "+v"(c) : "v"(x[s - 1]));
          else
            asm volatile("" : "+v"(c));
        } else {
          asm volatile("" : "+v"(c));
        }
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(lnp + c);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(lnp + c + 4);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(lnp + K + c);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(lnp + K + c + 4);
        f32x4 y0, y1;
        if constexpr (LO) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            y0[e] = ((float)x[s][e] - mean) * rstd * w0[e] + b0[e];
            y1[e] = ((float)x[s][4 + e] - mean) * rstd * w1[e] + b1[e];
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            y0[e] = fmaf(fmaf((float)x[s][e], rstd, mr), w0[e], b0[e]);
            y1[e] = fmaf(fmaf((float)x[s][4 + e], rstd, mr), w1[e], b1[e]);
          }
        }
        if constexpr (LO) {
          split8(y0, y1, xh[s], xl[s]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x[s][e] = (bf16)y0[e];
            x[s][4 + e] = (bf16)y1[e];
          }
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) split8(x[2 * s], x[2 * s + 1], xh[s], xl[s]);
    }
    const int64_t m = tile * 32 + li;
    const float pre = m < a.M ? row_pre<EPI>(a, m) : 0.f;
    const TileRun tr = staged ? tile_run<EPI>(a, tile * 32) : TileRun{};
    auto out_tile = [&](int ot, const bf16x8* rpre, const bf16x8* ypre = nullptr) __attribute__((always_inline)) {
      const bf16* wt = wl + ((ot - ot0) * 32 + li) * WS + KH * g;
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 w = *reinterpret_cast<const bf16x8*>(wt + 8 * s);
        if constexpr (LO) {
          acc = mfma32(w, xl[s], acc);
          acc = mfma32(w, xh[s], acc);
        } else {
          acc = mfma32(w, x[s], acc);
        }
      }
      int seg, cbase;
      (void)tile_weight_row<EPI>(a, ot, li, seg, cbase);
      if (m < a.M)
        row_epilogue<EPI>(a, acc, m, ot, seg, cbase, g, lb, pre, staged ? stage : nullptr,
                          staged ? &tr : nullptr, rpre, ypre);
    };
    if (EPI == kEpiResid && a.residual && nt <= 4) {
      // the residual of every output tile is loaded before the tile's first store: a wait
      // for a load issued after stores would wait for those stores too (vmcnt counts both)
      bf16x8 rv[4][2];
      const int64_t mm = m < a.M ? m : a.M - 1;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (u < nt)
#pragma unroll
          for (int k = 0; k < 2; ++k)
            rv[u][k] = *reinterpret_cast<const bf16x8*>(a.res + mm * a.O + (ot0 + u) * 32 + 8 * (2 * k + g));
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (u < nt) out_tile(ot0 + u, rv[u]);
    } else if constexpr (GR) {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (u < nt) {
          out_tile(ot0 + u, gr[u % GRS], gy[u % GRS]);
          if (u + GRS < 8 && u + GRS < nt) gr_load(u + GRS, gy[u % GRS], gr[u % GRS]);
        }
    } else if (K >= 256 && ((EPI == kEpiResid && a.residual) || EPI == kEpiGateResid)) {
      // the epilogue operands of each output tile (yin, the residual) are loaded one tile
      // ahead, before the previous tile's stores, into two register sets used in turn (rows
      // of 256 channels or more: shorter rows keep the registers for more waves per SIMD)
      const int64_t mm = m < a.M ? m : a.M - 1;
      const int last = ot0 + nt - 1;
      auto epi_load = [&](int ot, bf16x8 (&rv)[2], bf16x8 (&yv)[2]) __attribute__((always_inline)) {
        ot = ot < last ? ot : last;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int64_t at = mm * a.O + ot * 32 + 8 * (2 * k + g);
          if (EPI == kEpiGateResid) yv[k] = *reinterpret_cast<const bf16x8*>(a.yin + at);
          if (a.residual) rv[k] = *reinterpret_cast<const bf16x8*>(a.res + at);
        }
      };
      bf16x8 ra[2], rb[2], ya[2], yb[2];
      epi_load(ot0, ra, ya);
#pragma unroll 1
      for (int ot = ot0; ot <= last; ot += 2) {
        epi_load(ot + 1, rb, yb);
        out_tile(ot, ra, ya);
        if (ot == last) break;
        epi_load(ot + 2, ra, ya);
        out_tile(ot + 1, rb, yb);
      }
    } else {
#pragma unroll 1
      for (int ot = ot0; ot < ot0 + nt; ++ot) out_tile(ot, nullptr);
    }
  };

  if constexpr (DB) {
    // two register buffers used in turn: the next tile's rows load while the current one is
    // processed
    XT x0[NX], x1[NX];
    fetch(x0, t);
    while (true) {
      fetch(x1, t + stride);
      process(x0, t);
      t += stride;
      if (t >= tiles) break;
      fetch(x0, t + stride);
      process(x1, t);
      t += stride;
      if (t >= tiles) break;
    }
  } else {
    XT x0[NX];
    fetch(x0, t);
    while (true) {
      process(x0, t);
      t += stride;
      if (t >= tiles) break;
      fetch(x0, t);
    }
  }
}

// ---------------------------------------------------------------------------- pair bias
// bias[b, h, i, j] = rstd_ij * (z_ij . W'_h - mean_ij * sum_c W'_h[c]) with
// W'_h[c] = log2(e) * gamma[c] * W_b[h][c]; this equals LN_pair(z_ij) . W_b[h] * log2(e) for
// the offset-free pair norm. z is exact in bf16 and W' is carried as a bf16 pair
// hi + lo (two MFMA passes), so the bias keeps fp32 accuracy: its error does not grow with
// the logit size (large pair logits would otherwise shift the softmax weights).
// One wave handles a tile of 32 consecutive keys j of one (b, i): lane (li, g) loads its
// row's channels 16 t + 8 g .. 16 t + 8 g + 7 for t < C / 16, so each load instruction reads
// 32 contiguous bytes per row (lanes l and l ^ 32 together), the statistics come from those
// registers (two passes, halves joined across lane l ^ 32), and the heads x keys block is
// one 32 x 32 MFMA tile (A = W' rows, B = the z rows; channels 16 t .. 16 t + 15 feed step t).
template <int C>
__global__ __launch_bounds__(256) void apb_pair_bias(PairBiasArgs a) {
  constexpr int kU = C / 16;  // 8-channel chunks per lane (each lane half holds C / 2)
  __shared__ float wsum_s[4][32];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 31, g = lane >> 5;
  const int n = a.n;
  const int njt = a.np / 32;
  const int64_t stride = (int64_t)gridDim.x * 4;

  // Tiles are fetched one ahead (two register buffers used alternately); a fetch past the
  // last tile re-reads the last tile, so every load stays inside z.
  auto fetch = [&](bf16x8* zf, int64_t tile) {
    const int64_t tt = tile < a.tiles ? tile : a.tiles - 1;
    const int64_t bi = tt / njt;
    const int j0 = (int)(tt - bi * njt) * 32;
    const int key = min(j0 + li, n - 1);
    int64_t row = bi * n + key;  // pair position (query i, key): z[b, i, key]
    if (a.transposed) {          // z[b, key, i]
      const int64_t b = bi / n;
      row = (b * n + key) * n + (bi - b * n);
    }
    const bf16* zr = a.z + row * C + 8 * g;
#pragma unroll
    for (int u = 0; u < kU; ++u) zf[u] = ld8(zr + 16 * u);
  };
  int64_t t = (int64_t)blockIdx.x * 4 + wave;
  bf16x8 z0[kU], z1[kU];
  fetch(z0, t);

  bf16x8 wf[kU], wl[kU];
  float rs = 0.f;
  const float* wrow = a.w_bias + min(li, a.heads - 1) * C + 8 * g;
  const float* lrow = a.ln_w + 8 * g;
  const float keep = li < a.heads ? kLog2e : 0.f;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(wrow + 16 * u);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(wrow + 16 * u + 4);
    const f32x4 l0 = *reinterpret_cast<const f32x4*>(lrow + 16 * u);
    const f32x4 l1 = *reinterpret_cast<const f32x4*>(lrow + 16 * u + 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = keep * (e < 4 ? l0[e] * w0[e] : l1[e - 4] * w1[e - 4]);
      wf[u][e] = (bf16)v;
      wl[u][e] = (bf16)(v - (float)wf[u][e]);
      rs += v;
    }
  }
  rs = pair_sum(rs);
  if (g == 0) wsum_s[wave][li] = rs;
  __syncthreads();

  auto process = [&](const bf16x8* zf, int64_t tile) {
    float s1 = 0.f;
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) s1 += (float)zf[u][e];
    const float mean = pair_sum(s1) * (1.f / C);
    float s2 = 0.f;
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = (float)zf[u][e] - mean;
        s2 += d * d;
      }
    const float rstd = __builtin_amdgcn_rsqf(pair_sum(s2) * (1.f / C) + a.eps);
    f32x16 acc = zero16();
#pragma unroll
    for (int u = 0; u < kU; ++u) acc = mfma32(wl[u], zf[u], acc);
#pragma unroll
    for (int u = 0; u < kU; ++u) acc = mfma32(wf[u], zf[u], acc);

    const int64_t bi = tile / njt;
    const int key = (int)(tile - bi * njt) * 32 + li;
    const int64_t b = bi / n;
    const int64_t i = bi - b * n;
    const bool valid = key < n && a.mask[b * n + key] != 0;
    float* out = a.bias + (b * a.heads * n + i) * a.np + key;
    // blocked: entry (query i, key) of head h at bias_index(b heads + h, ...), a whole number
    // of head strides (np^2) apart
    if (a.blocked) out = a.bias + bias_index(b * a.heads, a.np / 32, i, key);
    const int64_t hstride = a.blocked ? (int64_t)a.np * a.np : (int64_t)n * a.np;
    const float masked = a.blocked ? -INFINITY : kMaskedLogit;
    const int64_t xe = b * a.extra_sb + i * a.extra_si + key;  // head 0's extra logit
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int h = acc_row(r, g);
      if (h < a.heads) {
        float y = rstd * (acc[r] - mean * wsum_s[wave][h]);
        if (a.extra && valid) {
          const int64_t at = xe + h * a.extra_sh;
          y += kLog2e * (a.extra_bf16 ? (float)static_cast<const bf16*>(a.extra)[at]
                                      : static_cast<const float*>(a.extra)[at]);
        }
        out[h * hstride] = valid ? y : masked;
      }
    }
  };
  while (t < a.tiles) {
    fetch(z1, t + stride);
    process(z0, t);
    t += stride;
    if (t >= a.tiles) break;
    fetch(z0, t + stride);
    process(z1, t);
    t += stride;
  }
}

// The same bias at pair width 128 with the z rows staged through LDS: each wave owns two 8 KB
// tile buffers that its own LDS DMA fills (each transfer is 4 whole rows, 1 KB contiguous for
// the un-transposed orientation, swizzled by off128), one tile ahead of the one it processes, so
// the rows arrive as full lines instead of 32-byte pieces of 32 rows per load; a wave's buffers
// are its own, so the loop has no barrier. Persistent: every wave walks tiles t0, t0 + stride, ...
// (stride = 4 gridDim.x). The waits count this wave's vector-memory operations, which on gfx950
// include its stores: waiting for tile k's rows also waits for the stores of tile k - 1, issued
// one tile earlier.
__global__ __launch_bounds__(256, 2) void apb_pair_bias_lds(PairBiasArgs a) {
  constexpr int C = 128, kU = C / 16;
  __shared__ float wsum_s[4][32];
  __shared__ __attribute__((aligned(16))) bf16 zt[4][2][32 * C];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, li = lane & 31, g = lane >> 5;
  const int n = a.n;
  const int njt = a.np / 32;
  const int64_t stride = (int64_t)gridDim.x * 4;
  const uint32_t zt_lds = lds_addr(&zt[wave][0][0]);

  // Rows j0 .. j0 + 31 of tile `tile` (keys past n repeat key n - 1: finite, masked) into
  // buffer buf; a tile index past the end re-reads the last tile. Piece p = rows 4 p .. 4 p + 3:
  // lane L fills slot L & 15 of row 4 p + L / 16 with the row's chunk (L & 15) ^ (row & 15).
  auto tile_dma = [&](int64_t tile, int buf) {
    const int64_t tt = tile < a.tiles ? tile : a.tiles - 1;
    const int64_t bi = tt / njt;
    const int j0 = (int)(tt - bi * njt) * 32;
    const int64_t b = bi / n, i = bi - b * n;
    const bf16* base = a.transposed ? a.z + (b * n * n + i) * C : a.z + bi * n * C;
    const uint32_t rstride = a.transposed ? (uint32_t)n * C * 2 : (uint32_t)C * 2;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int r = 4 * p + (lane >> 4);
      const int key = min(j0 + r, n - 1);
      dma16_stream(base, (uint32_t)key * rstride + 16 * ((lane & 15) ^ (r & 15)),
                   zt_lds + (uint32_t)(buf * 32 * C * 2 + 1024 * p));
    }
  };
  int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t < a.tiles) tile_dma(t, 0);

  bf16x8 wf[kU], wl[kU];
  float rs = 0.f;
  const float* wrow = a.w_bias + min(li, a.heads - 1) * C + 8 * g;
  const float* lrow = a.ln_w + 8 * g;
  const float keep = li < a.heads ? kLog2e : 0.f;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(wrow + 16 * u);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(wrow + 16 * u + 4);
    const f32x4 l0 = *reinterpret_cast<const f32x4*>(lrow + 16 * u);
    const f32x4 l1 = *reinterpret_cast<const f32x4*>(lrow + 16 * u + 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = keep * (e < 4 ? l0[e] * w0[e] : l1[e - 4] * w1[e - 4]);
      wf[u][e] = (bf16)v;
      wl[u][e] = (bf16)(v - (float)wf[u][e]);
      rs += v;
    }
  }
  rs = pair_sum(rs);
  if (g == 0) wsum_s[wave][li] = rs;
  __syncthreads();
  if (t >= a.tiles) return;  // no transfer of this wave is in flight

  for (int k = 0;; ++k) {
    const bool more = t + stride < a.tiles;
    if (more) {
      tile_dma(t + stride, (k + 1) & 1);
      wait_vm_lds<8>();  // tile k's rows (and everything before them) landed
    } else {
      wait_vm_lds<0>();
    }
    bf16x8 zf[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) zf[u] = ld8(&zt[wave][k & 1][off128(li, 2 * u + g)]);

    float s1 = 0.f;
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) s1 += (float)zf[u][e];
    const float mean = pair_sum(s1) * (1.f / C);
    float s2 = 0.f;
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = (float)zf[u][e] - mean;
        s2 += d * d;
      }
    const float rstd = __builtin_amdgcn_rsqf(pair_sum(s2) * (1.f / C) + a.eps);
    f32x16 acc = zero16();
#pragma unroll
    for (int u = 0; u < kU; ++u) acc = mfma32(wl[u], zf[u], acc);
#pragma unroll
    for (int u = 0; u < kU; ++u) acc = mfma32(wf[u], zf[u], acc);

    const int64_t bi = t / njt;
    const int key = (int)(t - bi * njt) * 32 + li;
    const int64_t b = bi / n;
    const int64_t i = bi - b * n;
    const bool valid = key < n && a.mask[b * n + key] != 0;
    float* out = a.bias + (b * a.heads * n + i) * a.np + key;
    if (a.blocked) out = a.bias + bias_index(b * a.heads, a.np / 32, i, key);
    const int64_t hstride = a.blocked ? (int64_t)a.np * a.np : (int64_t)n * a.np;
    const float masked = a.blocked ? -INFINITY : kMaskedLogit;
    const int64_t xe = b * a.extra_sb + i * a.extra_si + key;  // head 0's extra logit
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int h = acc_row(r, g);
      if (h < a.heads) {
        float y = rstd * (acc[r] - mean * wsum_s[wave][h]);
        if (a.extra && valid) {
          const int64_t at = xe + h * a.extra_sh;
          y += kLog2e * (a.extra_bf16 ? (float)static_cast<const bf16*>(a.extra)[at]
                                      : static_cast<const float*>(a.extra)[at]);
        }
        out[h * hstride] = valid ? y : masked;
      }
    }
    t += stride;
    if (t >= a.tiles) break;
  }
}

// ---------------------------------------------------------------------------- attention
// One workgroup per (32 queries, head, batch); its four waves split the key blocks
// (wave w takes blocks w, w + 4, ...), run an online softmax each and are merged through LDS.
// Per 32-key block: S^T = K Q^T + bias^T (A = k rows, B = q rows, the bias as the MFMA
// accumulator input: lane (li, g) holds query li and keys 8 v + 4 g + e), then
// O^T += V^T P^T (A = v^T rows in the permuted key order, B = this lane's 16 weights).
// DT 32-channel tiles of the head (DT = 2: heads of 40 to 64 channels): DT 32 x 32 output
// tiles, 2 DT MFMAs of the logits per key block.
template <int DT>
__global__ __launch_bounds__(256) void apb_attention(ApbAttnArgs a) {
  __shared__ float sm[4][32], sl[4][32];
  __shared__ float so[3][64][16 * DT];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, li = lane & 31, g = lane >> 5;
  const int q0 = blockIdx.x * 32, h = blockIdx.y, b = blockIdx.z;
  const int n = a.n, dh = a.dh, cs = a.cs;

  const int bb = b / a.rows_per_bias;  // the batch element of the bias and the key mask
  int any = 0;
  for (int t = threadIdx.x; t < n; t += 256) any |= a.mask[(int64_t)bb * n + t];
  const bool empty = !__syncthreads_or(any);

  const int qr = min(q0 + li, n - 1);
  const bf16* qp = a.q + ((int64_t)b * n + qr) * cs + h * dh;
  bf16x8 qf[2 * DT];
#pragma unroll
  for (int f = 0; f < 2 * DT; ++f) qf[f] = 16 * f + 8 * g < dh ? ld8(qp + 16 * f + 8 * g) : zero8();
  const float* bp = a.bias + (((int64_t)bb * a.heads + h) * n + qr) * a.np + 4 * g;
  const bf16* vp[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
    vp[t] = a.vt + (((int64_t)b * a.heads + h) * dh + min(32 * t + li, dh - 1)) * a.np + 8 * g;
  const bf16* kbase = a.k + (int64_t)b * n * cs + h * dh;

  float m = -INFINITY, l = 0.f;
  f32x16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = zero16();
  const int nkb = a.np / 32;
  for (int kb = wave; kb < nkb; kb += 4) {
    const bf16* kp = kbase + (int64_t)min(kb * 32 + li, n - 1) * cs;
    bf16x8 kf[2 * DT];
#pragma unroll
    for (int f = 0; f < 2 * DT; ++f) kf[f] = 16 * f + 8 * g < dh ? ld8(kp + 16 * f + 8 * g) : zero8();
    f32x16 s;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(bp + kb * 32 + 8 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) s[4 * v + e] = bv[e];
    }
    bf16x8 vf[DT][2];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      vf[t][0] = ld8(vp[t] + kb * 32);
      vf[t][1] = ld8(vp[t] + kb * 32 + 16);
    }
#pragma unroll
    for (int f = 0; f < 2 * DT; ++f) s = mfma32(kf[f], qf[f], s);

    float bm = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) bm = fmaxf(bm, s[r]);
    bm = pair_max(bm);
    const float mn = fmaxf(m, bm);
    const float alpha = fast_exp2(m - mn);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = fast_exp2(s[r] - mn);
      ps += s[r];
    }
    l = l * alpha + ps;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= alpha;

    if (kb * 32 + 32 > n) {  // keys past n: their v^T entries were never written
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = kb * 32 + 4 * g + 8 * (j >> 2) + (j & 3);
          if (key >= n) vf[t][0][j] = (bf16)0.f;
          if (key + 16 >= n) vf[t][1][j] = (bf16)0.f;
        }
    }
    bf16x8 p0, p1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p0[j] = (bf16)s[j];
      p1[j] = (bf16)s[8 + j];
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      o[t] = mfma32(vf[t][0], p0, o[t]);
      o[t] = mfma32(vf[t][1], p1, o[t]);
    }
  }
  l = pair_sum(l);

  if (g == 0) {
    sm[wave][li] = m;
    sl[wave][li] = l;
  }
  __syncthreads();
  const float mx = fmaxf(fmaxf(sm[0][li], sm[1][li]), fmaxf(sm[2][li], sm[3][li]));
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) total += sl[w][li] * fast_exp2(sm[w][li] - mx);
  const float f = empty ? 0.f : fast_exp2(m - mx) / total;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] *= f;
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) so[wave - 1][lane][16 * t + r] = o[t][r];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] += so[w][lane][16 * t + r];
  const int qq = q0 + li;
  if (qq >= n) return;
  const int64_t row = ((int64_t)b * n + qq) * cs + h * dh;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int d0 = 32 * t + 8 * v + 4 * g;
      if (d0 < dh) {
        const bf16x4 gv = *reinterpret_cast<const bf16x4*>(a.gate + row + d0);
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = o[t][4 * v + e] * (float)gv[e];
        *reinterpret_cast<f32x4*>(a.og + row + d0) = y;
      }
    }
}

}  // namespace

template <int EPI, int XSRC, int NO>
void launch_row_gemm_t(const RowGemmArgs& a, hipStream_t stream) {
  const int otiles = a.O / 32;
  const dim3 grid((unsigned)((a.M + 31) / 32), (unsigned)((otiles + NO - 1) / NO));
  const size_t lds = row_gemm_lds(XSRC, a.K, NO);
  auto kernel = row_gemm<EPI, XSRC, NO>;
  if (lds > 65536)  // beyond the default dynamic LDS size (K > 480 with the LayerNorm tile)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  kernel<<<grid, 64 * kGemmWaves, lds, stream>>>(a);
}

// Tile shapes: the LayerNorm-fed GEMMs give each workgroup several output tiles (the tile is
// normalised once per workgroup); the fp32-fed ones split k 8 ways when k is long, and give the
// waves separate output tiles when k has fewer groups than waves.
// Output parts: halve the weight rows per workgroup until a workgroup's LDS is at most 72 KiB
// (two workgroups of 4 waves per CU), as long as the parts stay whole tiles. Measured on the
// template stacks: splitting at 56 KiB instead (three workgroups per CU, the input read twice
// for 384 outputs) was 2.5% slower per block. Rows of 256 channels or more: at most 160 KiB
// (one workgroup of 8 waves per CU), so that each part re-reads and re-normalises the input
// rows as few times as possible.
size_t row_stream_lds_cap(int K) { return (K >= 256 ? 160 : 72) * 1024; }
int row_stream_parts(int K, int O) {
  int parts = 1;
  while (row_stream_lds(K, O, O / parts) > row_stream_lds_cap(K) && (O / 32) % (2 * parts) == 0) parts *= 2;
  return parts;
}

template <int EPI, int XSRC, int K>
void launch_row_stream_t(const RowGemmArgs& a, hipStream_t stream) {
  constexpr int kStreamWaves = stream_waves(K);
  const int parts = row_stream_parts(K, a.O);
  const size_t lds = row_stream_lds(K, a.O, a.O / parts);
  auto kernel = row_stream<EPI, XSRC, K>;
  if (lds > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  const int64_t tiles = (a.M + 31) / 32;
  const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(4, (160 * 1024) / (int64_t)lds));
  const int64_t blocks = std::min<int64_t>((tiles + kStreamWaves - 1) / kStreamWaves,
                                           std::max<int64_t>(1, cu_count() * per_cu / parts));
  kernel<<<dim3((unsigned)std::max<int64_t>(1, blocks), (unsigned)parts), 64 * kStreamWaves, lds, stream>>>(a);
}

// The streaming kernel's cases: the pair path's short rows, a part of the weights fitting in LDS.
template <int EPI, int XSRC>
bool launch_row_stream(const RowGemmArgs& a, hipStream_t stream) {
  // k 64 or 128; bf16 rows (normalised or plain) also 256; plain bf16 rows also 512
  if (a.K != 64 && a.K != 128 && !(XSRC != kXF32 && a.K == 256) && !(XSRC == kXBf16 && a.K == 512))
    return false;
  const size_t cap = a.K >= 256 ? 160 * 1024 : 80 * 1024;
  if (row_stream_lds(a.K, a.O, a.O / row_stream_parts(a.K, a.O)) > cap) return false;
  if (a.K == 64) {
    launch_row_stream_t<EPI, XSRC, 64>(a, stream);
  } else if (a.K == 128) {
    launch_row_stream_t<EPI, XSRC, 128>(a, stream);
  } else if constexpr (XSRC != kXF32) {
    if (a.K == 256)
      launch_row_stream_t<EPI, XSRC, 256>(a, stream);
    else if constexpr (XSRC == kXBf16)
      launch_row_stream_t<EPI, XSRC, 512>(a, stream);
  }
  return true;
}

void launch_row_gemm(const RowGemmArgs& a, int epi, int xsrc, hipStream_t stream) {
  // short rows of the pair path: the streaming kernel (false: not a case it takes)
  if (xsrc == kXLn) {
    if (epi == kEpiApb && launch_row_stream<kEpiApb, kXLn>(a, stream)) return;
    if (epi == kEpiTrimul && launch_row_stream<kEpiTrimul, kXLn>(a, stream)) return;
    if (epi == kEpiStoreY && launch_row_stream<kEpiStoreY, kXLn>(a, stream)) return;
    if (epi == kEpiGateResid && launch_row_stream<kEpiGateResid, kXLn>(a, stream)) return;
    if (epi == kEpiSwiglu && launch_row_stream<kEpiSwiglu, kXLn>(a, stream)) return;
    if (epi == kEpiResid && a.ln_plain && launch_row_stream<kEpiResid, kXBf16>(a, stream)) return;
    if (epi == kEpiResid && launch_row_stream<kEpiResid, kXLn>(a, stream)) return;
    if (epi == kEpiOpm && launch_row_stream<kEpiOpm, kXLn>(a, stream)) return;
    if (epi == kEpiPwa && launch_row_stream<kEpiPwa, kXLn>(a, stream)) return;
  } else if (epi == kEpiResid && launch_row_stream<kEpiResid, kXF32>(a, stream)) {
    return;
  }
  if (epi == kEpiApb && xsrc == kXLn)
    launch_row_gemm_t<kEpiApb, kXLn, 4>(a, stream);
  else if (epi == kEpiSwiglu && xsrc == kXLn)
    launch_row_gemm_t<kEpiSwiglu, kXLn, 8>(a, stream);
  else if (epi == kEpiResid && xsrc == kXF32) {
    // k split into KS parts of whole 64-wide groups with none left idle (8 from 6 groups up)
    const int groups = a.K / 64;
    if (groups >= 6)
      launch_row_gemm_t<kEpiResid, kXF32, 1>(a, stream);
    else if (groups >= 4)
      launch_row_gemm_t<kEpiResid, kXF32, 2>(a, stream);
    else if (groups >= 2)
      launch_row_gemm_t<kEpiResid, kXF32, 4>(a, stream);
    else
      launch_row_gemm_t<kEpiResid, kXF32, 8>(a, stream);
  }
  else if (epi == kEpiResid && xsrc == kXLn) {
    if (a.O >= 256)
      launch_row_gemm_t<kEpiResid, kXLn, 8>(a, stream);
    else if (a.O >= 128)
      launch_row_gemm_t<kEpiResid, kXLn, 4>(a, stream);
    else
      launch_row_gemm_t<kEpiResid, kXLn, 2>(a, stream);
  } else if (epi == kEpiPwa && xsrc == kXLn)
    launch_row_gemm_t<kEpiPwa, kXLn, 8>(a, stream);
  else if (epi == kEpiOpm && xsrc == kXLn)
    launch_row_gemm_t<kEpiOpm, kXLn, 2>(a, stream);
  else if (epi == kEpiTrimul && xsrc == kXLn)
    launch_row_gemm_t<kEpiTrimul, kXLn, 8>(a, stream);
  else if (epi == kEpiStoreY && xsrc == kXLn) {
    if (a.O >= 256)
      launch_row_gemm_t<kEpiStoreY, kXLn, 8>(a, stream);
    else if (a.O >= 128)
      launch_row_gemm_t<kEpiStoreY, kXLn, 4>(a, stream);
    else
      launch_row_gemm_t<kEpiStoreY, kXLn, 2>(a, stream);
  } else if (epi == kEpiLinear && xsrc == kXLn) {
    if (a.O >= 256)
      launch_row_gemm_t<kEpiLinear, kXLn, 8>(a, stream);
    else if (a.O >= 128)
      launch_row_gemm_t<kEpiLinear, kXLn, 4>(a, stream);
    else
      launch_row_gemm_t<kEpiLinear, kXLn, 2>(a, stream);
  } else if (epi == kEpiGateResid && xsrc == kXLn) {
    // one workgroup column (O <= 256): a workgroup owns its rows, so out may alias the input
    if (a.O > 128)
      launch_row_gemm_t<kEpiGateResid, kXLn, 8>(a, stream);
    else if (a.O > 64)
      launch_row_gemm_t<kEpiGateResid, kXLn, 4>(a, stream);
    else
      launch_row_gemm_t<kEpiGateResid, kXLn, 2>(a, stream);
  }
}

void launch_apb_pair_bias(const PairBiasArgs& a, hipStream_t stream) {
  // pair width 128: the LDS-staged persistent kernel (two workgroups per CU), unless a
  // transposed key offset would not fit its 32-bit DMA offset
  if (a.c == 128 && (!a.transposed || (int64_t)a.n * a.n * 256 <= 0xffffffffLL)) {
    int64_t blocks = (a.tiles + 3) / 4;
    const int64_t cap = (int64_t)cu_count() * 2;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    apb_pair_bias_lds<<<dim3((unsigned)blocks), 256, 0, stream>>>(a);
    return;
  }
  int64_t blocks = (a.tiles + 7) / 8;  // about two tiles per wave
  const int64_t cap = (int64_t)cu_count() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  if (a.c == 64)
    apb_pair_bias<64><<<dim3((unsigned)blocks), 256, 0, stream>>>(a);
  else if (a.c == 256)
    apb_pair_bias<256><<<dim3((unsigned)blocks), 256, 0, stream>>>(a);
  else
    apb_pair_bias<128><<<dim3((unsigned)blocks), 256, 0, stream>>>(a);
}

void launch_apb_attention(const ApbAttnArgs& a, int batch, hipStream_t stream) {
  const dim3 grid((unsigned)((a.n + 31) / 32), (unsigned)a.heads, (unsigned)batch);
  if (a.dh > 32)
    apb_attention<2><<<grid, 256, 0, stream>>>(a);
  else
    apb_attention<1><<<grid, 256, 0, stream>>>(a);
}

}  // namespace ffk
