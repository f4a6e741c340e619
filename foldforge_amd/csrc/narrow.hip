// Pair ops at widths other than the fused kernels' (the template stack's 64-channel pair, hidden
// widths of 64 or 256, triangle-attention heads of 16): the shared pieces below, the rest is
// the token-row GEMMs of single.hip, the contraction of trimul.hip and the attention of
// single.hip, composed by api.hip.
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

void launch_pair_add_transposed(const bf16* base, const bf16* t, bf16* out, int64_t batch, int n,
                                int c, hipStream_t stream) {
  const int64_t total = batch * n * n * (c / 8);
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = (int64_t)cu_count() * 16;
  blocks = blocks < 1 ? 1 : blocks > cap ? cap : blocks;
  pair_add_transposed<<<dim3((unsigned)blocks), 256, 0, stream>>>(base, t, out, batch, n, c);
}

}  // namespace ffk
