// Fused pair transition on gfx950: x + squeeze(silu(expand_a(LN(x))) * expand_b(LN(x))).
//
// Equations: src/foldforge/models/checkpoints/legacy/reference/transition.py:40-41 and
// src/foldforge/modules/dense/diffusion_transformer.py:36-44 (SwiGLU). The 4c-wide hidden
// layer never reaches HBM: x is read once and the output written once.
//
// Persistent over tiles of 128 positions; 8 waves per workgroup = 4 position groups of 32
// x 2 halves. The 384 KB of bf16 weights are streamed through LDS in chunks of 64 hidden
// channels (Wa, Wb rows and the matching Ws columns), each chunk shared by the four
// position groups; the next chunk's loads are in flight while the current one is used.
// Per chunk a wave computes a, b for its 32 positions x 32 hidden channels (the LN'd
// operand stays in registers for the whole tile), writes silu(a) * b to LDS, and after a
// barrier accumulates its 32 positions x 64 output channels over the chunk's 64 hidden
// channels (the other half's h comes from the partner wave through LDS).
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kXT = 128;       // positions per tile
constexpr int kXC = 64;        // hidden channels per chunk
constexpr int kWS = 128 + 8;   // LDS row stride of a Wa / Wb chunk (K = 128)
constexpr int kSS = kXC + 8;   // LDS row stride of a Ws chunk and of the h chunk (K = 64)

struct __attribute__((aligned(16))) TransitionLds {
  bf16 xr[kXT * kRow];   // raw x (residual), then the output tile
  bf16 xh[kXT * kRow];   // LN(x)
  bf16 wa[kXC * kWS];    // expand_a rows of the chunk
  bf16 wb[kXC * kWS];    // expand_b rows of the chunk
  bf16 ws[128 * kSS];    // squeeze columns of the chunk, [out channel][hidden]
  bf16 h[kXT * kSS];     // silu(a) * b of the chunk, [position][hidden]
};

// grid: persistent (one workgroup per CU); block 512.
__global__ __launch_bounds__(512) void transition_128x4(
    const bf16* __restrict__ x, const float* __restrict__ ln_w, const float* __restrict__ ln_b,
    const bf16* __restrict__ wa, const bf16* __restrict__ wb, const bf16* __restrict__ ws,
    bf16* __restrict__ out, int64_t rows, int residual, float eps) {
  constexpr int C = 128, HID = 512;
  __shared__ TransitionLds L;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, g = lane >> 5, li = lane & 31;
  const int pg = wave & 3;   // position group: positions 32 pg .. 32 pg + 31
  const int hh = wave >> 2;  // hidden half of the chunk / output channel half
  // chunk staging: 3 x 1024 chunks of 16 bytes (Wa, Wb: 64 rows x 16; Ws: 128 rows x 8)
  bf16x8 pre[6];
  auto gload = [&](int h0) {
#pragma unroll
    for (int u = 0; u < 6; ++u) {
      const int c = tid + 512 * u;  // 0 .. 3071
      const int part = c >> 10, w = c & 1023;
      if (part < 2) {
        const int row = w >> 4, k8 = w & 15;
        pre[u] = ld8((part == 0 ? wa : wb) + (int64_t)(h0 + row) * C + 8 * k8);
      } else {
        const int row = w >> 3, k8 = w & 7;
        pre[u] = ld8(ws + (int64_t)row * HID + h0 + 8 * k8);
      }
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int u = 0; u < 6; ++u) {
      const int c = tid + 512 * u;
      const int part = c >> 10, w = c & 1023;
      if (part < 2) {
        const int row = w >> 4, k8 = w & 15;
        *reinterpret_cast<bf16x8*>(&(part == 0 ? L.wa : L.wb)[row * kWS + 8 * k8]) = pre[u];
      } else {
        const int row = w >> 3, k8 = w & 7;
        *reinterpret_cast<bf16x8*>(&L.ws[row * kSS + 8 * k8]) = pre[u];
      }
    }
  };

  const int64_t ntiles = (rows + kXT - 1) / kXT;
#pragma unroll 1
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row0 = tile * kXT;
    const int valid = (int)min<int64_t>(kXT, rows - row0);
    gload(0);
    __syncthreads();  // the previous tile's LDS readers are done
    ln_tile_128<kXT, 512>(x + row0 * C, C, valid, ln_w, ln_b, eps, L.xh, L.xr);
    sstore();
    __syncthreads();
    bf16x8 xf[8];
    {
      const bf16* xrow = L.xh + (32 * pg + li) * kRow + 8 * g;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) xf[kk] = ld8(xrow + 16 * kk);
    }
    f32x16 acc[2] = {zero16(), zero16()};  // output channels 64 hh + 32 t + li
#pragma unroll 1
    for (int h0 = 0; h0 < HID; h0 += kXC) {
      const bool more = h0 + kXC < HID;
      if (more) gload(h0 + kXC);
      f32x16 aa = zero16(), ab = zero16();
      const bf16* war = L.wa + (32 * hh + li) * kWS + 8 * g;
      const bf16* wbr = L.wb + (32 * hh + li) * kWS + 8 * g;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        aa = mfma32(xf[kk], ld8(war + 16 * kk), aa);
        ab = mfma32(xf[kk], ld8(wbr + 16 * kk), ab);
      }
      // D[position][hidden]: lane li is hidden channel 32 hh + li of the chunk
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int p = 32 * pg + acc_row(q, g);
        L.h[p * kSS + 32 * hh + li] = (bf16)(siluf_(aa[q]) * ab[q]);
      }
      __syncthreads();  // h complete for the chunk
      const bf16* hrow = L.h + (32 * pg + li) * kSS + 8 * g;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16* wsr = L.ws + (64 * hh + 32 * t + li) * kSS + 8 * g;
#pragma unroll
        for (int kk = 0; kk < kXC / 16; ++kk) acc[t] = mfma32(ld8(hrow + 16 * kk), ld8(wsr + 16 * kk), acc[t]);
      }
      __syncthreads();  // chunk weights and h consumed
      if (more) {
        sstore();
        __syncthreads();
      }
    }
    // D[position][out channel]: add the residual, stage the tile in place of raw x
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c = 64 * hh + 32 * t + li;
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int p = 32 * pg + acc_row(q, g);
        float v = acc[t][q];
        if (residual) v += (float)L.xr[p * kRow + c];
        L.xr[p * kRow + c] = (bf16)v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int chunk = tid + 512 * u;
      const int p = chunk >> 4, c8 = chunk & 15;
      if (p < valid)
        *reinterpret_cast<bf16x8*>(out + (row0 + p) * C + 8 * c8) = ld8(&L.xr[p * kRow + 8 * c8]);
    }
  }
}

void launch_transition(const TransitionArgs& a, hipStream_t stream) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipGetDevice(&dev);
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus <= 0) cus = 256;
  }
  const int64_t ntiles = (a.rows + kXT - 1) / kXT;
  const int grid = (int)(ntiles < cus ? ntiles : cus);
  transition_128x4<<<dim3(grid), 512, 0, stream>>>(a.x, a.ln_w, a.ln_b, a.wa, a.wb, a.ws, a.out,
                                                   a.rows, a.residual, a.eps);
}

}  // namespace ffk
