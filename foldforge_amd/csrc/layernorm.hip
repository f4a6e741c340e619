// LayerNorm over the last axis on gfx950 (fp32 statistics, fp32 affine, input dtype kept).
//
// Reference: the engine LayerNorm (src/foldforge/modules/engine/modules.py:230-238) and the
// torch.nn.LayerNorm of the legacy graph (legacy/attention.py:90). HBM-bound: the 128-wide
// bf16 path streams 16-byte vectors with 16 lanes per row and 2 rows per lane (32 rows per
// 256-thread workgroup, up to 32 workgroups per CU, so a pair tensor of up to 262144 rows is
// one pass of workgroups and larger ones loop), fetches a workgroup's next rows while it
// normalises the current ones (two register buffers used alternately), keeps each row in
// registers between the two statistics passes (exact two-pass variance) and writes the output
// with non-temporal stores (measured at N = 512: 22.5 -> 19.6 us against 8 rows per lane, four
// persistent workgroups per CU and regular stores).
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

constexpr int kLnRowsPerLane = 2;
constexpr int kLnRowsPerBlock = 16 * kLnRowsPerLane;  // 16 rows per pass (16 lanes each)

// Normalise and store the rows row0 + 16 it (it < kLnRowsPerLane) whose 8-channel slices
// `sub` this lane holds in v; rows at or past `rows` are skipped.
__device__ __forceinline__ void ln_rows_compute(const bf16x8 (&v)[kLnRowsPerLane], int64_t row0, int64_t rows,
                                                const float (&wv)[8], const float (&bv)[8],
                                                bf16* __restrict__ y, int sub, float eps) {
#pragma unroll
  for (int it = 0; it < kLnRowsPerLane; ++it) {
    const int64_t row = row0 + 16 * it;
    float xv[8];
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xv[e] = row < rows ? (float)v[it][e] : 0.f;
      s += xv[e];
    }
    const float mean = sum16(s) * (1.f / 128.f);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xv[e] -= mean;
      q += xv[e] * xv[e];
    }
    const float rstd = __builtin_amdgcn_rsqf(sum16(q) * (1.f / 128.f) + eps);
    if (row < rows) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)(xv[e] * rstd * wv[e] + bv[e]);
      __builtin_nontemporal_store(o, reinterpret_cast<bf16x8*>(y + row * 128 + 8 * sub));
    }
  }
}

// bf16 rows of exactly 128 channels. grid min(ceil(rows / 32), 32 per CU); block 256.
__global__ __launch_bounds__(256) void layer_norm_bf16_128(const bf16* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ b,
                                                           bf16* __restrict__ y, int64_t rows,
                                                           float eps) {
  const int tid = threadIdx.x;
  const int sub = tid & 15;
  float wv[8], bv[8];
  auto load = [&](bf16x8 (&v)[kLnRowsPerLane], int64_t row0) {
#pragma unroll
    for (int it = 0; it < kLnRowsPerLane; ++it) {
      const int64_t row = row0 + 16 * it;
      if (row < rows) v[it] = ld8(x + row * 128 + 8 * sub);
    }
  };
  const int64_t step = (int64_t)gridDim.x * kLnRowsPerBlock;
  int64_t row0 = (int64_t)blockIdx.x * kLnRowsPerBlock + (tid >> 4);
  bf16x8 va[kLnRowsPerLane], vb[kLnRowsPerLane];
  load(va, row0);
  // one uniform branch per pointer (a per-element select compiles to a branch per load)
  if (w != nullptr) {
#pragma unroll
    for (int e = 0; e < 8; ++e) wv[e] = w[8 * sub + e];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) wv[e] = 1.f;
  }
  if (b != nullptr) {
#pragma unroll
    for (int e = 0; e < 8; ++e) bv[e] = b[8 * sub + e];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) bv[e] = 0.f;
  }
  // row0 - tid / 16 is the workgroup's first row: the loop condition is uniform
  while (row0 - (tid >> 4) < rows) {
    load(vb, row0 + step);
    ln_rows_compute(va, row0, rows, wv, bv, y, sub, eps);
    row0 += step;
    if (row0 - (tid >> 4) >= rows) break;
    load(va, row0 + step);
    ln_rows_compute(vb, row0, rows, wv, bv, y, sub, eps);
    row0 += step;
  }
}

// Any width, bf16 or fp32: one wave per row. grid min(ceil(rows / 4), 65535 * 4); block 256.
template <typename T>
__global__ __launch_bounds__(256) void layer_norm_rows(const T* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       const float* __restrict__ b,
                                                       T* __restrict__ y, int64_t rows, int cols,
                                                       float eps) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float inv = 1.f / (float)cols;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < rows; row += (int64_t)gridDim.x * 4) {
    const T* xr = x + row * cols;
    float s = 0.f;
    for (int c = lane; c < cols; c += 64) s += (float)xr[c];
    const float mean = wave_sum(s) * inv;
    float q = 0.f;
    for (int c = lane; c < cols; c += 64) {
      const float d = (float)xr[c] - mean;
      q += d * d;
    }
    const float rstd = 1.f / sqrtf(wave_sum(q) * inv + eps);
    T* yr = y + row * cols;
    for (int c = lane; c < cols; c += 64) {
      float v = ((float)xr[c] - mean) * rstd;
      if (w) v *= w[c];
      if (b) v += b[c];
      yr[c] = (T)v;
    }
  }
}

void launch_layer_norm(const void* x, const float* w, const float* b, void* y, int64_t rows,
                       int cols, float eps, int dtype, hipStream_t stream) {
  if (dtype == 0 && cols == 128) {
    int64_t blocks = (rows + kLnRowsPerBlock - 1) / kLnRowsPerBlock;
    if (blocks > (int64_t)cu_count() * 32) blocks = (int64_t)cu_count() * 32;
    layer_norm_bf16_128<<<dim3((unsigned)blocks), 256, 0, stream>>>(
        static_cast<const bf16*>(x), w, b, static_cast<bf16*>(y), rows, eps);
    return;
  }
  int64_t blocks = (rows + 3) / 4;
  if (blocks > 65535 * 4) blocks = 65535 * 4;
  if (dtype == 0) {
    layer_norm_rows<bf16><<<dim3((unsigned)blocks), 256, 0, stream>>>(
        static_cast<const bf16*>(x), w, b, static_cast<bf16*>(y), rows, cols, eps);
  } else {
    layer_norm_rows<float><<<dim3((unsigned)blocks), 256, 0, stream>>>(
        static_cast<const float*>(x), w, b, static_cast<float*>(y), rows, cols, eps);
  }
}

}  // namespace ffk
