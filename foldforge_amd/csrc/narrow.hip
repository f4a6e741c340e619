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

void launch_planes_to_rows(const bf16* planes, bf16* rows, int batch, int hid, int n, int np,
                           hipStream_t stream) {
  const size_t lds = (size_t)hid * (kRowTile + 2) * sizeof(bf16);
  if (lds > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(planes_to_rows),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  planes_to_rows<<<dim3((unsigned)((n + kRowTile - 1) / kRowTile), (unsigned)n, (unsigned)batch),
                   256, lds, stream>>>(planes, rows, hid, n, np);
}

}  // namespace ffk
