// C-ABI of the pair-stack kernels: argument checks, workspace carving, weight packing and
// launches. Declarations and contracts: include/foldforge_amd.h.
//
// Parameters arrive as the engine module's fp32 tensors; each op converts the ones its
// MFMA kernels read into bf16 inside the caller's workspace (one small launch per call),
// folding the softmax scale * log2(e) into the query rows and log2(e) into the pair-bias
// rows. Nothing is cached between calls, so an updated parameter is always seen.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "foldforge_amd.h"
#include "ffk_device.h"
#include "ffk_kernels.h"

namespace ffk {

namespace {

thread_local std::string g_error;

int32_t fail(int32_t code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int32_t ok() {
  g_error.clear();
  return FFK_OK;
}

constexpr int kMaxDevices = 64;
int g_device_state[kMaxDevices];  // 0 unknown, 1 supported, 2 unsupported

int32_t device_state(int device) {
  if (device < 0 || device >= kMaxDevices) return 2;
  if (g_device_state[device] == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
    g_device_state[device] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
  }
  return g_device_state[device];
}

int g_cu_count[kMaxDevices];

int32_t check_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FFK_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  const int32_t s = device_state(dev);
  if (s == 0) return fail(FFK_ERR_HIP, "hipGetDeviceProperties failed for device %d", dev);
  if (s != 1) return fail(FFK_ERR_DEVICE, "device %d is not a gfx950 (MI355X)", dev);
  return FFK_OK;
}

int32_t check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FFK_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  if (g_cu_count[dev] <= 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    g_cu_count[dev] = cus;
  }
  return g_cu_count[dev];
}

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

size_t up256(size_t x) { return (x + 255) & ~size_t(255); }

int64_t pad128(int64_t n) { return (n + 127) / 128 * 128; }

// Sequential sub-allocation of the caller's workspace (256-byte aligned pieces).
struct Carver {
  char* base;
  size_t used = 0;
  template <typename T>
  T* take(size_t count) {
    T* p = reinterpret_cast<T*>(base ? base + used : nullptr);
    used += up256(count * sizeof(T));
    return p;
  }
};

// Workgroup row y converts segment y (the row past the last segment converts the mask), so
// the segments' loads are in flight together rather than one segment after another.
__global__ __launch_bounds__(256) void pack_bf16(PackJob job) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t first = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if ((int)blockIdx.y < job.nseg) {
    const PackSeg sg = job.seg[blockIdx.y];
    for (int64_t i = first; i < sg.n; i += stride) {
      const int64_t j = sg.swap23 ? (i & ~int64_t(12)) | ((i & 4) << 1) | ((i & 8) >> 1) : i;
      sg.dst[i] = (bf16)(sg.src ? sg.src[j] * sg.scale : 0.f);
    }
  } else if (job.mask) {
    // one workgroup per batch element: its mask row, and the number of key stages up to the
    // last real key
    __shared__ int last;
    for (int b = blockIdx.x; b < job.batch; b += gridDim.x) {
      if (threadIdx.x == 0) last = -1;
      __syncthreads();
      int mine = -1;
      for (int s = threadIdx.x; s < job.np; s += blockDim.x) {
        const bool real = s < job.n && job.mask[(int64_t)b * job.n + s] != 0;
        job.maskf[(int64_t)b * job.np + s] = real ? 1.f : 0.f;
        if (real) mine = s;
      }
      if (mine >= 0) atomicMax(&last, mine);
      __syncthreads();
      if (threadIdx.x == 0 && job.kstages) job.kstages[b] = (last + 32) / 32;
      __syncthreads();
    }
  }
}

}  // namespace

// Grid: one row of workgroups per segment (plus one for the mask), each row as wide as the
// largest segment needs (at most 1024 workgroups); the weights of one op are a few hundred
// thousand values, a latency-bound pass either way.
void launch_pack(const PackJob& job, hipStream_t stream) {
  int64_t most = job.mask ? (int64_t)job.batch * 256 : 0;  // the mask row: a workgroup per batch
  for (int s = 0; s < job.nseg; ++s) most = job.seg[s].n > most ? job.seg[s].n : most;
  int64_t blocks = (most + 255) / 256;
  blocks = blocks < 1 ? 1 : blocks > 1024 ? 1024 : blocks;
  const unsigned rows = (unsigned)job.nseg + (job.mask ? 1u : 0u);
  pack_bf16<<<dim3((unsigned)blocks, rows < 1 ? 1u : rows), 256, 0, stream>>>(job);
}

// ---------------------------------------------------------------------------------------
// workspace layouts (shared by the size queries and the entry points)

// The fused kernels serve the AF3 trunk widths; other widths run the generic path
// (token-row GEMMs + the plane contraction).
bool trimul_fused(int c, int h) { return c == 128 && h == 128; }
bool triattn_fused(int c, int heads, int d) { return c == 128 && heads == 4 && d == 32; }

struct TrimulWs {
  bf16 *wp, *wg, *wo, *A, *B, *P, *Pt;
  bf16* y;  // the update before the gate (generic path, bf16)
  float *maskf, *eps_out;
  int* kst;
  size_t bytes;
};
// Pair width 64 with hidden 64 or 128 on the generic path: one output kernel reading the
// contraction's planes (its tile index is a 32-bit int).
bool trimul_planes(int64_t batch, int64_t n, int c, int h) {
  return c == 64 && (h == 64 || h == 128) && batch * n * ((n + 31) / 32) < 0x7fffffffLL;
}

TrimulWs trimul_ws(void* ws, int64_t batch, int64_t n, int c, int h) {
  Carver cv{static_cast<char*>(ws)};
  const int64_t np = pad128(n);
  const size_t plane = (size_t)batch * h * np * np;
  TrimulWs w{};
  w.eps_out = cv.take<float>(1);  // the centre norm's epsilon of a length-divided call
  if (!trimul_fused(c, h)) {
    w.A = cv.take<bf16>(plane);
    w.B = cv.take<bf16>(plane);
    w.P = cv.take<bf16>(plane);
    // the token rows of P and the bf16 output projection between the row GEMMs (pair and
    // hidden width 64: one kernel reading the planes)
    if (!trimul_planes(batch, n, c, h)) {
      w.Pt = cv.take<bf16>((size_t)batch * n * n * h);
      w.y = cv.take<bf16>((size_t)batch * n * n * c);
    }
    w.bytes = cv.used;
    return w;
  }
  w.wp = cv.take<bf16>((size_t)4 * h * c);
  w.wg = cv.take<bf16>((size_t)c * c);
  w.wo = cv.take<bf16>((size_t)c * h);
  w.A = cv.take<bf16>(plane);
  w.B = cv.take<bf16>(plane);
  w.P = cv.take<bf16>(plane);
  w.maskf = cv.take<float>((size_t)batch * np);
  w.kst = cv.take<int>((size_t)batch);
  w.bytes = cv.used;
  return w;
}

int64_t pad32(int64_t n);

struct TriattnWs {
  bf16 *wqkv, *wb, *wg, *wo, *wo_t, *q, *k, *vt, *o, *gate, *tbuf, *ogb;
  float *bias, *og, *maskf;
  int* kst;
  size_t bytes;
};
// Head widths the generic path runs on the flash core (the rest: apb_attention).
bool triattn_flash_width(int d) { return d == 16 || d == 32 || d == 64; }
// Generic widths whose output kernel computes the gate from z (pair 64, gated width 64, 128 or
// 256): the projection then writes q, k, v only and the flash core the plain attention output.
bool triattn_gate_out(int c, int heads, int d) {
  return triattn_flash_width(d) && c == 64 && (heads * d == 64 || heads * d == 128 || heads * d == 256);
}
int64_t pad4(int64_t n) { return (n + 3) / 4 * 4; }

TriattnWs triattn_ws(void* ws, int64_t batch, int64_t n, int c, int heads, int d, int form) {
  Carver cv{static_cast<char*>(ws)};
  const int64_t np = pad128(n);
  const int hd = heads * d;
  TriattnWs w{};
  // the untransposed and dual forms stage one z-frame update before the transposed add
  if (form != kTriattnStandard) w.tbuf = cv.take<bf16>((size_t)batch * n * n * c);
  if (!triattn_fused(c, heads, d)) {
    const int64_t np32 = pad32(n);
    const size_t tok = (size_t)batch * n * n * hd;
    if (triattn_flash_width(d)) {
      // the flash core's layouts: rows padded to whole row groups, keys to np32
      const size_t blk = (size_t)batch * heads * pad4(n) * np32 * d;
      w.q = cv.take<bf16>(blk);
      w.k = cv.take<bf16>(blk);
      w.vt = cv.take<bf16>(blk);
      if (!triattn_gate_out(c, heads, d)) w.gate = cv.take<bf16>(tok);
      w.bias = cv.take<float>((size_t)batch * heads * np32 * np32);
      w.ogb = cv.take<bf16>(tok);  // the attention output (gated unless the output kernel gates it), bf16
      w.bytes = cv.used;
      return w;
    } else {
      w.q = cv.take<bf16>(tok);
      w.k = cv.take<bf16>(tok);
      w.gate = cv.take<bf16>(tok);
      w.vt = cv.take<bf16>((size_t)batch * n * hd * np32);
      w.bias = cv.take<float>((size_t)batch * heads * n * np32);
    }
    w.og = cv.take<float>(tok);
    w.bytes = cv.used;
    return w;
  }
  w.wqkv = cv.take<bf16>((size_t)3 * hd * c);
  w.wb = cv.take<bf16>((size_t)32 * c);
  w.wg = cv.take<bf16>((size_t)hd * c);
  w.wo = cv.take<bf16>((size_t)c * hd);
  if (form == kTriattnDual) w.wo_t = cv.take<bf16>((size_t)c * hd);
  w.q = cv.take<bf16>((size_t)batch * heads * np * np * d);
  w.k = cv.take<bf16>((size_t)batch * heads * np * np * d);
  w.vt = cv.take<bf16>((size_t)batch * heads * np * np * d);
  w.bias = cv.take<float>((size_t)batch * heads * np * np);
  w.o = cv.take<bf16>((size_t)batch * n * n * hd);
  w.maskf = cv.take<float>((size_t)batch * np);
  w.kst = cv.take<int>((size_t)batch);
  w.bytes = cv.used;
  return w;
}

// The fused kernel (d = 128, factor 4) takes the three weights packed chunk by chunk in its
// LDS image order; other widths run expand (LayerNorm prologue, SwiGLU epilogue) -> squeeze
// through the hidden rows h [rows][factor d] (fp32).
bool transition_fused(int d, int factor) { return d == 128 && factor == 4; }

struct TransitionWs {
  bf16* w;
  float* h;   // hidden rows wider than the LayerNorm-fed GEMM's k limit: fp32
  bf16* hb;   // else bf16 (the squeeze reads them as plain bf16 rows)
  size_t bytes;
};
TransitionWs transition_ws(void* ws, int64_t rows, int d, int factor) {
  Carver cv{static_cast<char*>(ws)};
  TransitionWs w{};
  if (transition_fused(d, factor)) {
    w.w = cv.take<bf16>((size_t)3 * factor * d * d);
  } else if ((int64_t)factor * d <= kLnGemmMaxK) {
    w.hb = cv.take<bf16>((size_t)rows * factor * d);
  } else {
    w.h = cv.take<float>((size_t)rows * factor * d);
  }
  w.bytes = cv.used;
  return w;
}

int64_t pad32(int64_t n) { return (n + 31) / 32 * 32; }

int64_t pad64(int64_t n) { return (n + 63) / 64 * 64; }

struct PwaWs {
  bf16 *vt, *gate, *w, *og;
  float* logits;
  size_t bytes;
};
PwaWs pwa_ws(void* ws, int64_t batch, int64_t depth, int64_t n, int heads, int dh) {
  Carver cv{static_cast<char*>(ws)};
  const int64_t np = pad64(n);
  const size_t tok = (size_t)batch * depth * n * heads * dh;
  PwaWs w;
  w.vt = cv.take<bf16>((size_t)batch * heads * depth * dh * np);
  w.gate = cv.take<bf16>(tok);
  w.logits = cv.take<float>((size_t)batch * heads * n * np);
  w.w = cv.take<bf16>((size_t)batch * heads * n * np);
  w.og = cv.take<bf16>(tok);
  w.bytes = cv.used;
  return w;
}

struct OpmWs {
  bf16 *lt, *rt, *mt, *wp;
  float* count;
  size_t bytes;
};
OpmWs opm_ws(void* ws, int64_t batch, int64_t depth, int64_t n, int cz) {
  Carver cv{static_cast<char*>(ws)};
  const int64_t sp = pad64(depth);
  OpmWs w;
  w.lt = cv.take<bf16>((size_t)batch * n * 32 * sp);
  w.rt = cv.take<bf16>((size_t)batch * n * 32 * sp);
  w.mt = cv.take<bf16>((size_t)batch * n * sp);
  w.count = cv.take<float>((size_t)batch * n * n);
  w.wp = cv.take<bf16>((size_t)cz * 1024);
  w.bytes = cv.used;
  return w;
}

struct ApbWs {
  bf16 *q, *k, *vt, *gate;
  float *og, *bias;
  size_t bytes;
};
ApbWs apb_ws(void* ws, int64_t batch, int64_t n, int cs, int heads) {
  Carver cv{static_cast<char*>(ws)};
  const int64_t np = pad32(n);
  const size_t tok = (size_t)batch * n * cs;
  ApbWs w;
  w.q = cv.take<bf16>(tok);
  w.k = cv.take<bf16>(tok);
  w.gate = cv.take<bf16>(tok);
  w.og = cv.take<float>(tok);
  w.vt = cv.take<bf16>((size_t)batch * cs * np);
  w.bias = cv.take<float>((size_t)batch * heads * n * np);
  w.bytes = cv.used;
  return w;
}

// Argument checks shared by the transition entry points (not the workspace).
int32_t transition_check(const void* x, const float* ln_w, const float* ln_b, const float* wa,
                         const float* wb, const float* wsq, const void* out, int64_t rows, int d,
                         int factor) {
  const bool fused = transition_fused(d, factor);
  if (!fused && (d <= 0 || factor <= 0 || d % 64 != 0 || d > kLnGemmMaxK || ((int64_t)factor * d) % 64 != 0))
    return fail(FFK_ERR_INVALID, "transition: d=%d factor=%d (kernels take 128 x 4, or d <= %d and factor * d multiples of 64)", d, factor, kLnGemmMaxK);
  if (rows < 0) return fail(FFK_ERR_INVALID, "transition: negative rows");
  if (!fused && (rows + 31) / 32 > 0x7fffffffLL)
    return fail(FFK_ERR_INVALID, "transition: %lld rows exceed the launch grid", (long long)rows);
  if (!x || !ln_w || !ln_b || !wa || !wb || !wsq || !out)
    return fail(FFK_ERR_INVALID, "transition: null argument");
  if (!aligned16(x) || !aligned16(out))
    return fail(FFK_ERR_INVALID, "transition: x/out must be 16-byte aligned");
  if (!fused && (!aligned16(wa) || !aligned16(wb) || !aligned16(wsq)))
    return fail(FFK_ERR_INVALID, "transition: weights must be 16-byte aligned");
  return FFK_OK;
}

// The launches of one transition call on a carved workspace (caller's or the static scratch).
int32_t transition_run(const TransitionWs& w, const void* x, const float* ln_w, const float* ln_b,
                       const float* wa, const float* wb, const float* wsq, void* out, int64_t rows,
                       int d, int factor, int residual, float eps, hipStream_t st) {
  if (!transition_fused(d, factor)) {
    RowGemmArgs g{};
    g.w_split = 1;  // fp32-accurate weights (see row_gemm)
    g.ln_x = static_cast<const bf16*>(x);
    g.ln_w = ln_w;
    g.ln_b = ln_b;
    g.eps = eps;
    g.w0 = wa;
    g.w1 = wb;
    g.M = rows;
    g.K = d;
    g.O = 2 * factor * d;
    g.h32 = w.h;
    g.h16 = w.hb;
    launch_row_gemm(g, kEpiSwiglu, kXLn, st);
    RowGemmArgs s{};
    s.w_split = 1;  // fp32-accurate weights (see row_gemm)
    s.x32 = w.h;
    s.ln_x = w.hb;
    s.ln_plain = 1;
    s.w0 = wsq;
    s.M = rows;
    s.K = factor * d;
    s.O = d;
    s.res = static_cast<const bf16*>(x);
    s.out = static_cast<bf16*>(out);
    s.residual = residual ? 1 : 0;
    launch_row_gemm(s, kEpiResid, w.hb ? kXLn : kXF32, st);
    return check_launch("transition");
  }
  launch_transition_pack(wa, wb, wsq, w.w, st);
  TransitionArgs a;
  a.x = static_cast<const bf16*>(x);
  a.ln_w = ln_w;
  a.ln_b = ln_b;
  a.w = w.w;
  a.out = static_cast<bf16*>(out);
  a.rows = rows;
  a.residual = residual ? 1 : 0;
  a.eps = eps;
  launch_transition(a, st);
  return check_launch("transition");
}

}  // namespace ffk

// ---------------------------------------------------------------------------------------
// Static scratch of ffk_transition_noalloc, for callers that cannot allocate device memory.
// Each device holds its own copy of this array for the life of the process. In host code its
// name is only a stand-in, not a device address: the address of a device's copy comes from
// hipGetSymbolAddress, looked up once per device with that device current, and only that
// address is handed to kernels. Calls on one device share the array, so calls that overlap
// in time on one device (different streams, other threads) race; nothing in it has to start
// at zero (every launch writes what it later reads).
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace ffk {
namespace {
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices];
}  // namespace

int32_t noalloc_scratch(void** address) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FFK_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(FFK_ERR_DEVICE, "device %d beyond the library's table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_address[dev]) {
    void* p = nullptr;
    const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (r != hipSuccess || !p)
      return fail(FFK_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(r));
    g_scratch_address[dev] = p;
  }
  *address = g_scratch_address[dev];
  return FFK_OK;
}
}  // namespace ffk

using namespace ffk;

extern "C" {

int32_t ffk_version(void) { return 100; }

const char* ffk_last_error(void) { return g_error.c_str(); }

int32_t ffk_device_supported(int32_t device) { return device_state(device) == 1 ? 1 : 0; }

int32_t ffk_layer_norm(const void* x, const float* weight, const float* bias, void* y,
                       int64_t rows, int32_t cols, float eps, int32_t dtype, void* stream) {
  if (int32_t s = check_device()) return s;
  if (!x || !y) return fail(FFK_ERR_INVALID, "layer_norm: null tensor");
  if (rows < 0 || cols <= 0) return fail(FFK_ERR_INVALID, "layer_norm: bad shape rows=%lld cols=%d", (long long)rows, cols);
  if (dtype != FFK_DTYPE_BF16 && dtype != FFK_DTYPE_F32)
    return fail(FFK_ERR_INVALID, "layer_norm: dtype %d is neither bf16 nor fp32", dtype);
  if (dtype == FFK_DTYPE_BF16 && cols == 128 && (!aligned16(x) || !aligned16(y)))
    return fail(FFK_ERR_INVALID, "layer_norm: bf16 rows of 128 need 16-byte aligned tensors");
  if (rows == 0) return ok();
  launch_layer_norm(x, weight, bias, y, rows, cols, eps, dtype, static_cast<hipStream_t>(stream));
  return check_launch("layer_norm");
}

size_t ffk_triangle_multiplication_workspace(int64_t batch, int64_t n, int32_t d_pair,
                                             int32_t d_hidden) {
  if (batch <= 0 || n <= 0 || d_pair <= 0 || d_hidden <= 0) return 0;
  return trimul_ws(nullptr, batch, n, d_pair, d_hidden).bytes;
}

int32_t ffk_triangle_multiplication(
    const void* z, const uint8_t* key_mask, const float* ln_pair_w, const float* ln_pair_b,
    const float* w_left, const float* w_right, const float* w_left_gate,
    const float* w_right_gate, const float* ln_out_w, const float* ln_out_b,
    const float* w_out, const float* w_gate, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t n, int32_t d_pair, int32_t d_hidden,
    int32_t outgoing, int32_t residual, int32_t length_divided, float eps, void* stream) {
  if (int32_t s = check_device()) return s;
  const bool fused = trimul_fused(d_pair, d_hidden);
  if (!fused && (d_pair <= 0 || d_pair % 64 != 0 || d_pair > 256 || d_hidden <= 0 ||
                 d_hidden % 64 != 0 || d_hidden > kLnGemmMaxK))
    return fail(FFK_ERR_INVALID, "triangle_multiplication: d_pair=%d d_hidden=%d (kernels take 128/128, or d_pair a multiple of 64 up to 256 with d_hidden a multiple of 64 up to %d)", d_pair, d_hidden, kLnGemmMaxK);
  if (batch <= 0 || n <= 0) return fail(FFK_ERR_INVALID, "triangle_multiplication: empty shape");
  if (batch * 128 > 65535 || pad128(n) > 65535)
    return fail(FFK_ERR_INVALID, "triangle_multiplication: batch=%lld n=%lld exceed the launch grid", (long long)batch, (long long)n);
  if (!z || !key_mask || !ln_pair_w || !ln_pair_b || !w_left || !w_right || !w_left_gate ||
      !w_right_gate || !ln_out_w || !ln_out_b || !w_out || !w_gate || !out)
    return fail(FFK_ERR_INVALID, "triangle_multiplication: null argument");
  if (!aligned16(z) || !aligned16(out))
    return fail(FFK_ERR_INVALID, "triangle_multiplication: z/out must be 16-byte aligned");
  const TrimulWs need = trimul_ws(nullptr, batch, n, d_pair, d_hidden);
  if (!workspace || workspace_bytes < need.bytes || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "triangle_multiplication: workspace %zu bytes < %zu", workspace_bytes, need.bytes);
  const TrimulWs w = trimul_ws(workspace, batch, n, d_pair, d_hidden);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the output kernel addresses 8 channel planes from one base with 32-bit byte offsets
  if (fused && 7 * 2 * pad128(n) * pad128(n) > 0xffffffffLL)
    return fail(FFK_ERR_INVALID, "triangle_multiplication: n=%lld exceeds the fused kernels' plane offsets", (long long)n);
  if (!fused && batch * d_hidden * (pad128(n) / 128) * (pad128(n) / 128) > 0x7fffffffLL)
    return fail(FFK_ERR_INVALID, "triangle_multiplication: shape exceeds the launch grid");
  // every argument check is behind us: nothing is queued or written before a refusal
  if (length_divided) launch_length_eps(key_mask, (int)batch, (int)n, eps, w.eps_out, st);
  const float* eps_out = length_divided ? w.eps_out : nullptr;
  if (!fused) {
    const int64_t np = pad128(n);
    RowGemmArgs p{};
    p.ln_x = static_cast<const bf16*>(z);
    p.ln_w = ln_pair_w;
    p.ln_b = ln_pair_b;
    p.eps = eps;
    p.w0 = w_left;
    p.w1 = w_right;
    p.w2 = w_left_gate;
    p.w3 = w_right_gate;
    p.M = batch * np * np;
    p.K = d_pair;
    p.O = 4 * d_hidden;
    p.n = (int)n;
    p.npm = (int)np;
    p.tmap = outgoing ? kMapGridOut : kMapGridIn;
    p.mask = key_mask;
    p.pa = w.A;
    p.pb = w.B;
    launch_row_gemm(p, kEpiTrimul, kXLn, st);
    launch_trimul_contract(w.A, w.B, w.P, batch * d_hidden, (int)np, st);
    if (trimul_planes(batch, n, d_pair, d_hidden)) {
      TrimulPlanesArgs r{};
      r.planes = w.P;
      r.z = static_cast<const bf16*>(z);
      r.lno_w = ln_out_w;
      r.lno_b = ln_out_b;
      r.ln_w = ln_pair_w;
      r.ln_b = ln_pair_b;
      r.w_out = w_out;
      r.w_gate = w_gate;
      r.eps_out = eps_out;
      r.out = static_cast<bf16*>(out);
      r.batch = (int)batch;
      r.n = (int)n;
      r.np = (int)np;
      r.hid = d_hidden;
      r.residual = residual ? 1 : 0;
      r.eps = eps;
      launch_trimul_out_planes(r, st);
      return check_launch("triangle_multiplication");
    }
    launch_planes_to_rows(w.P, w.Pt, (int)batch, d_hidden, (int)n, (int)np, st);
    RowGemmArgs o{};
    o.ln_x = w.Pt;
    o.ln_w = ln_out_w;
    o.ln_b = ln_out_b;
    o.eps = eps;
    o.eps_dev = eps_out;
    o.w0 = w_out;
    o.M = batch * n * n;
    o.K = d_hidden;
    o.O = d_pair;
    o.hy = w.y;
    launch_row_gemm(o, kEpiStoreY, kXLn, st);
    RowGemmArgs f{};
    f.ln_x = static_cast<const bf16*>(z);
    f.ln_w = ln_pair_w;
    f.ln_b = ln_pair_b;
    f.eps = eps;
    f.w0 = w_gate;
    f.M = batch * n * n;
    f.K = d_pair;
    f.O = d_pair;
    f.yin = w.y;
    f.res = static_cast<const bf16*>(z);
    f.out = static_cast<bf16*>(out);
    f.residual = residual ? 1 : 0;
    launch_row_gemm(f, kEpiGateResid, kXLn, st);
    return check_launch("triangle_multiplication");
  }
  const int64_t hc = (int64_t)d_hidden * d_pair;
  PackJob job{};
  // gate projections pre-multiplied by -log2(e): the kernels' sigmoid is 1 / (1 + 2^y)
  job.seg[0] = {w_left, w.wp, hc, 1.f};
  job.seg[1] = {w_left_gate, w.wp + hc, hc, -kLog2e};
  job.seg[2] = {w_right, w.wp + 2 * hc, hc, 1.f};
  job.seg[3] = {w_right_gate, w.wp + 3 * hc, hc, -kLog2e};
  job.seg[4] = {w_gate, w.wg, (int64_t)d_pair * d_pair, -kLog2e};
  job.seg[5] = {w_out, w.wo, (int64_t)d_pair * d_hidden, 1.f};
  job.nseg = 6;
  job.mask = key_mask;
  job.maskf = w.maskf;
  job.kstages = w.kst;
  job.batch = (int)batch;
  job.n = (int)n;
  job.np = (int)pad128(n);
  launch_pack(job, st);
  TrimulArgs a;
  a.z = static_cast<const bf16*>(z);
  a.mask = key_mask;
  a.ln_w = ln_pair_w;
  a.ln_b = ln_pair_b;
  a.lno_w = ln_out_w;
  a.lno_b = ln_out_b;
  a.wp = w.wp;
  a.wg = w.wg;
  a.wo = w.wo;
  a.A = w.A;
  a.B = w.B;
  a.P = w.P;
  a.maskf = w.maskf;
  a.kstages = w.kst;
  a.out = static_cast<bf16*>(out);
  a.batch = (int)batch;
  a.n = (int)n;
  a.np = (int)pad128(n);
  a.outgoing = outgoing ? 1 : 0;
  a.residual = residual ? 1 : 0;
  a.eps = eps;
  a.eps_out = eps_out;
  launch_trimul(a, st);
  return check_launch("triangle_multiplication");
}

// The pack and the launches of the fused-width triangle attention (d_pair 128, 4 x 32) on a
// carved workspace; project_only: the projection and the flash core only (w.o holds the
// attention output in z frame, nothing is written to out).
static void triattn_fused_launch(const TriattnWs& w, const void* z, const uint8_t* key_mask,
                          const float* ln_pair_w, const float* ln_pair_b, const float* w_bias,
                          const float* w_query, const float* w_key, const float* w_value,
                          const float* w_gate, const float* w_out, const float* b_gate,
                          const float* b_out, const float* w_out_t, const float* b_out_t,
                          void* out, int64_t batch, int64_t n, int n_head, int d_head,
                          int starting, int transposed_bias, int form, int residual, float eps,
                          bool project_only, hipStream_t st) {
  const int d_pair = 128;
  const int hd = n_head * d_head;
  const int64_t m = (int64_t)hd * d_pair;
  const float qscale = kLog2e / sqrtf((float)d_head);
  PackJob job{};
  job.seg[0] = {w_query, w.wqkv, m, qscale};
  job.seg[1] = {w_key, w.wqkv + m, m, 1.f};
  job.seg[2] = {w_value, w.wqkv + 2 * m, m, 1.f};
  job.seg[3] = {w_bias, w.wb, (int64_t)n_head * d_pair, kLog2e};
  job.seg[4] = {nullptr, w.wb + (int64_t)n_head * d_pair, (int64_t)(32 - n_head) * d_pair, 0.f};
  // (the fused output-transition kernel packs the gate and output weights itself)
  job.seg[5] = {w_gate, w.wg, project_only ? 0 : m, -kLog2e};  // sigmoid(x) = 1 / (1 + 2^(-log2(e) x))
  job.seg[6] = {w_out, w.wo, project_only ? 0 : m, 1.f};
  job.seg[7] = {w_out_t, w.wo_t, form == kTriattnDual ? m : 0, 1.f};
  job.nseg = 8;
  job.mask = key_mask;
  job.maskf = w.maskf;
  job.kstages = w.kst;
  job.batch = (int)batch;
  job.n = (int)n;
  job.np = (int)pad128(n);
  launch_pack(job, st);
  TriattnArgs a{};
  a.z = static_cast<const bf16*>(z);
  a.mask = key_mask;
  a.maskf = w.maskf;
  a.kstages = w.kst;
  a.ln_w = ln_pair_w;
  a.ln_b = ln_pair_b;
  a.wqkv = w.wqkv;
  a.wb = w.wb;
  a.wg = w.wg;
  a.wo = w.wo;
  a.q = w.q;
  a.k = w.k;
  a.vt = w.vt;
  a.bias = w.bias;
  a.o = w.o;
  a.bg = b_gate;
  a.bo = b_out;
  a.form = form;
  a.wo_t = w.wo_t;
  a.bo_t = b_out_t;
  a.tbuf = w.tbuf;
  a.out = static_cast<bf16*>(out);
  a.batch = (int)batch;
  a.n = (int)n;
  a.np = (int)pad128(n);
  a.heads = n_head;
  a.starting = starting ? 1 : 0;
  a.transposed_bias = transposed_bias ? 1 : 0;
  a.residual = residual ? 1 : 0;
  a.eps = eps;
  a.project_only = project_only ? 1 : 0;
  launch_triattn(a, st);
}

size_t ffk_triangle_attention_workspace(int64_t batch, int64_t n, int32_t d_pair,
                                        int32_t n_head, int32_t d_head, int32_t output_form) {
  if (batch <= 0 || n <= 0 || d_pair <= 0 || n_head <= 0 || d_head <= 0) return 0;
  if (output_form < kTriattnStandard || output_form > kTriattnDual) return 0;
  return triattn_ws(nullptr, batch, n, d_pair, n_head, d_head, output_form).bytes;
}

int32_t ffk_triangle_attention(
    const void* z, const uint8_t* key_mask, const float* ln_pair_w, const float* ln_pair_b,
    const float* w_bias, const float* w_query, const float* w_key, const float* w_value,
    const float* w_gate, const float* w_out, const float* b_gate, const float* b_out,
    const float* w_out_t, const float* b_out_t, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t n, int32_t d_pair, int32_t n_head,
    int32_t d_head, int32_t starting, int32_t transposed_bias, int32_t output_form,
    int32_t residual, float eps, void* stream) {
  if (int32_t s = check_device()) return s;
  if (output_form < kTriattnStandard || output_form > kTriattnDual)
    return fail(FFK_ERR_INVALID, "triangle_attention: output_form %d (0 standard, 1 untransposed, 2 dual)", output_form);
  if ((output_form == kTriattnDual) != (w_out_t != nullptr))
    return fail(FFK_ERR_INVALID, "triangle_attention: w_out_t is required by, and only by, the dual output form");
  if (b_out_t && !w_out_t) return fail(FFK_ERR_INVALID, "triangle_attention: b_out_t without w_out_t");
  const bool fused = triattn_fused(d_pair, n_head, d_head);
  if (!fused && (!(d_pair == 64 || d_pair == 128 || d_pair == 256) || n_head <= 0 || n_head > 32 ||
                 d_head <= 0 || d_head % 8 != 0 || d_head > 64 || (n_head * d_head) % 64 != 0))
    return fail(FFK_ERR_INVALID, "triangle_attention: d_pair=%d heads=%d x %d (kernels take 128 with 4 x 32, or d_pair 64 / 128 / 256 with at most 32 heads of 8 to 64 channels, heads x d_head a multiple of 64)", d_pair, n_head, d_head);
  if (batch <= 0 || n <= 0) return fail(FFK_ERR_INVALID, "triangle_attention: empty shape");
  if (batch * n_head > 65535 || pad128(n) > 65535)
    return fail(FFK_ERR_INVALID, "triangle_attention: batch=%lld n=%lld exceed the launch grid", (long long)batch, (long long)n);
  if (!z || !key_mask || !ln_pair_w || !ln_pair_b || !w_bias || !w_query || !w_key ||
      !w_value || !w_gate || !w_out || !out)
    return fail(FFK_ERR_INVALID, "triangle_attention: null argument");
  if (!aligned16(z) || !aligned16(out))
    return fail(FFK_ERR_INVALID, "triangle_attention: z/out must be 16-byte aligned");
  const TriattnWs need = triattn_ws(nullptr, batch, n, d_pair, n_head, d_head, output_form);
  if (!workspace || workspace_bytes < need.bytes || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "triangle_attention: workspace %zu bytes < %zu", workspace_bytes, need.bytes);
  const TriattnWs w = triattn_ws(workspace, batch, n, d_pair, n_head, d_head, output_form);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int hd = n_head * d_head;
  // the ending node's untransposed update is the starting orientation's: nothing to turn
  const int form = output_form == kTriattnUntransposed && starting ? kTriattnStandard : output_form;
  if (!fused) {
    if (batch * n > 65535 || batch * n * n * hd / 32 > 0x7fffffffLL * 8)
      return fail(FFK_ERR_INVALID, "triangle_attention: batch * n = %lld exceeds the launch grid", (long long)(batch * n));
    const int64_t np32 = pad32(n);
    const bool flash = triattn_flash_width(d_head);
    const bool gate_out = triattn_gate_out(d_pair, n_head, d_head);
    // q, k, v^T, gate of every pair row (the transposed pair for the ending node); for the flash
    // core on keys padded to np32 (the padding repeats key n - 1, so its k and v are finite)
    RowGemmArgs p{};
    p.ln_x = static_cast<const bf16*>(z);
    p.ln_w = ln_pair_w;
    p.ln_b = ln_pair_b;
    p.eps = eps;
    p.w0 = w_query;
    p.w1 = w_key;
    p.w2 = w_value;
    p.w3 = w_gate;
    p.M = flash ? batch * n * np32 : batch * n * n;
    p.K = d_pair;
    p.O = (gate_out ? 3 : 4) * hd;
    p.apb_no_gate = gate_out ? 1 : 0;
    p.q_bias = nullptr;
    p.q_scale = kLog2e / sqrtf((float)d_head);
    p.gate_bias = 0.f;
    p.gate_b = b_gate;
    p.q = w.q;
    p.k = w.k;
    p.vt = w.vt;
    p.gate = w.gate;
    p.n = (int)n;
    p.np = (int)np32;
    p.heads = n_head;
    p.dh = d_head;
    if (flash) {
      p.tmap = starting ? kMapPadKeys : kMapPadKeysT;
      p.flash_rows = (int)pad4(n);
    } else {
      p.tmap = starting ? kMapIdentity : kMapPairT;
    }
    launch_row_gemm(p, kEpiApb, kXLn, st);
    // the pair bias from the un-transposed pair (the OpenFold lineage's ending node: the
    // transposed one); the norm's offset adds one constant per head, which the softmax cancels
    PairBiasArgs pb{};
    pb.z = static_cast<const bf16*>(z);
    pb.mask = key_mask;
    pb.ln_w = ln_pair_w;
    pb.w_bias = w_bias;
    pb.bias = w.bias;
    pb.tiles = batch * n * (np32 / 32);
    pb.n = (int)n;
    pb.np = (int)np32;
    pb.heads = n_head;
    pb.eps = eps;
    pb.c = d_pair;
    pb.transposed = !starting && transposed_bias ? 1 : 0;
    pb.blocked = flash ? 1 : 0;
    launch_apb_pair_bias(pb, st);
    if (flash) {
      // og = gate * o in the attention frame (row r, query j), as apb_attention writes it
      FlashArgs f{};
      f.q = w.q;
      f.k = w.k;
      f.vt = w.vt;
      f.bias = w.bias;
      f.batch = batch;
      f.rows = pad4(n);
      f.np = np32;
      f.rows_valid = n;
      f.n_valid = n;
      f.heads = n_head;
      f.kstages = nullptr;
      f.dh = d_head;
      if (gate_out) {
        f.o = w.ogb;
      } else {
        f.gate = w.gate;
        f.og = w.ogb;
      }
      f.o_sb = n * n * hd;
      f.o_sr = n * hd;
      f.o_sj = hd;
      launch_flash(f, st);
    } else {
      ApbAttnArgs at;
      at.q = w.q;
      at.k = w.k;
      at.vt = w.vt;
      at.gate = w.gate;
      at.bias = w.bias;
      at.mask = key_mask;
      at.og = w.og;
      at.n = (int)n;
      at.np = (int)np32;
      at.heads = n_head;
      at.dh = d_head;
      at.cs = hd;
      at.rows_per_bias = (int)n;
      launch_apb_attention(at, (int)(batch * n), st);
    }
    // the output projection of the gated values into dst (z frame), with the residual or not
    auto project = [&](const float* wo, const float* bo, bf16* dst, int res) {
      if (gate_out) {
        TriattnRowsArgs r{};
        r.z = static_cast<const bf16*>(z);
        r.o = w.ogb;
        r.ln_w = ln_pair_w;
        r.ln_b = ln_pair_b;
        r.w_gate = w_gate;
        r.b_gate = b_gate;
        r.w_out = wo;
        r.b_out = bo;
        r.out = dst;
        r.batch = (int)batch;
        r.n = (int)n;
        r.hd = hd;
        r.transposed = starting ? 0 : 1;
        r.residual = res;
        r.eps = eps;
        launch_triattn_out_rows(r, st);
        return;
      }
      RowGemmArgs o{};
      o.x32 = w.og;
      o.ln_x = w.ogb;
      o.ln_plain = 1;
      o.w0 = wo;
      o.bias_out = bo;
      o.M = batch * n * n;
      o.K = hd;
      o.O = d_pair;
      o.n = (int)n;
      o.tmap = starting ? kMapIdentity : kMapPairT;
      o.res = static_cast<const bf16*>(z);
      o.out = dst;
      o.residual = res;
      launch_row_gemm(o, kEpiResid, flash ? kXLn : kXF32, st);
    };
    bf16* dst = static_cast<bf16*>(out);
    if (form == kTriattnUntransposed) {
      project(w_out, b_out, w.tbuf, 0);
      launch_pair_add_transposed(residual ? static_cast<const bf16*>(z) : nullptr, w.tbuf, dst,
                                 batch, (int)n, d_pair, st);
    } else if (form == kTriattnDual) {
      project(w_out_t, b_out_t, w.tbuf, 0);
      project(w_out, b_out, dst, residual ? 1 : 0);
      launch_pair_add_transposed(dst, w.tbuf, dst, batch, (int)n, d_pair, st);
    } else {
      project(w_out, b_out, dst, residual ? 1 : 0);
    }
    return check_launch("triangle_attention");
  }
  triattn_fused_launch(w, z, key_mask, ln_pair_w, ln_pair_b, w_bias, w_query, w_key, w_value,
                       w_gate, w_out, b_gate, b_out, w_out_t, b_out_t, out, batch, n, n_head,
                       d_head, starting, transposed_bias, form, residual, eps, false, st);
  return check_launch("triangle_attention");
}

// The ending node's triangle attention and the pair transition behind it, with the
// attention's gate / output projection fused into the transition kernel.
static TriattnWs attn_transition_ws(void* ws, int64_t batch, int64_t n, bf16** wt) {
  TriattnWs w = triattn_ws(ws, batch, n, 128, 4, 32, kTriattnStandard);
  Carver cv{static_cast<char*>(ws), w.bytes};  // after the attention's pieces
  *wt = cv.take<bf16>((size_t)(16 + 3) * 3 * 32 * 128);
  w.bytes = cv.used;
  return w;
}

size_t ffk_triangle_attention_transition_workspace(int64_t batch, int64_t n) {
  if (batch <= 0 || n <= 0) return 0;
  bf16* wt;
  return attn_transition_ws(nullptr, batch, n, &wt).bytes;
}

int32_t ffk_triangle_attention_transition(
    const void* z, const uint8_t* key_mask, const float* ln_pair_w, const float* ln_pair_b,
    const float* w_bias, const float* w_query, const float* w_key, const float* w_value,
    const float* w_gate, const float* w_out, const float* ln_in_w, const float* ln_in_b,
    const float* w_expand_a, const float* w_expand_b, const float* w_squeeze, void* out,
    void* workspace, size_t workspace_bytes, int64_t batch, int64_t n, int32_t starting,
    int32_t transposed_bias, float eps_pair, float eps_in, void* stream) {
  if (int32_t s = check_device()) return s;
  if (batch <= 0 || n <= 0) return fail(FFK_ERR_INVALID, "triangle_attention_transition: empty shape");
  if (batch * 4 > 65535 || pad128(n) > 65535)
    return fail(FFK_ERR_INVALID, "triangle_attention_transition: batch=%lld n=%lld exceed the launch grid", (long long)batch, (long long)n);
  if (!z || !key_mask || !ln_pair_w || !ln_pair_b || !w_bias || !w_query || !w_key || !w_value ||
      !w_gate || !w_out || !ln_in_w || !ln_in_b || !w_expand_a || !w_expand_b || !w_squeeze || !out)
    return fail(FFK_ERR_INVALID, "triangle_attention_transition: null argument");
  if (!aligned16(z) || !aligned16(out))
    return fail(FFK_ERR_INVALID, "triangle_attention_transition: z/out must be 16-byte aligned");
  bf16* wt = nullptr;
  const size_t need = attn_transition_ws(nullptr, batch, n, &wt).bytes;
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "triangle_attention_transition: workspace %zu bytes < %zu", workspace_bytes, need);
  const TriattnWs w = attn_transition_ws(workspace, batch, n, &wt);
  hipStream_t st = static_cast<hipStream_t>(stream);
  launch_attention_transition_pack(w_gate, w_out, w_expand_a, w_expand_b, w_squeeze, wt, st);
  triattn_fused_launch(w, z, key_mask, ln_pair_w, ln_pair_b, w_bias, w_query, w_key, w_value,
                       w_gate, w_out, nullptr, nullptr, nullptr, nullptr, out, batch, n, 4, 32,
                       starting ? 1 : 0, transposed_bias ? 1 : 0, kTriattnStandard, 1, eps_pair,
                       true, st);
  AttnTransitionArgs a{};
  a.z = static_cast<const bf16*>(z);
  a.o = w.o;
  a.lnp_w = ln_pair_w;
  a.lnp_b = ln_pair_b;
  a.ln_w = ln_in_w;
  a.ln_b = ln_in_b;
  a.w = wt;
  a.out = static_cast<bf16*>(out);
  a.rows = batch * n * n;
  a.eps_pair = eps_pair;
  a.eps = eps_in;
  launch_attention_output_transition(a, st);
  return check_launch("triangle_attention_transition");
}

int32_t ffk_flash_attention_bias(const void* q, const void* k, const void* v_t,
                                 const void* bias, void* o, int64_t batch, int32_t heads,
                                 int64_t rows, int64_t n_pad, int64_t rows_valid,
                                 int64_t n_valid, int64_t o_sb, int64_t o_sr, int64_t o_sj,
                                 void* stream) {
  if (int32_t s = check_device()) return s;
  if (!q || !k || !v_t || !bias || !o) return fail(FFK_ERR_INVALID, "flash_attention_bias: null tensor");
  if (batch <= 0 || heads <= 0 || rows <= 0 || n_pad <= 0 || n_pad % 128 != 0 || rows % 4 != 0)
    return fail(FFK_ERR_INVALID, "flash_attention_bias: bad shape (n_pad %lld must be a positive multiple of 128, rows %lld of 4)", (long long)n_pad, (long long)rows);
  if (rows_valid < 0 || rows_valid > rows || n_valid < 0 || n_valid > n_pad)
    return fail(FFK_ERR_INVALID, "flash_attention_bias: valid extents exceed the padded shape");
  if ((n_pad + 127) / 128 * (rows / 4) * batch * heads > 0x7fffffffLL)
    return fail(FFK_ERR_INVALID, "flash_attention_bias: grid too large");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v_t) || !aligned16(bias))
    return fail(FFK_ERR_INVALID, "flash_attention_bias: q/k/v_t/bias must be 16-byte aligned");
  if (((uintptr_t)o & 15u) != 0 || (o_sb | o_sr | o_sj) % 8 != 0)
    return fail(FFK_ERR_INVALID, "flash_attention_bias: o and its strides must be 16-byte aligned");
  FlashArgs f{};
  f.q = static_cast<const bf16*>(q);
  f.k = static_cast<const bf16*>(k);
  f.vt = static_cast<const bf16*>(v_t);
  f.bias = static_cast<const float*>(bias);
  f.o = static_cast<bf16*>(o);
  f.batch = batch;
  f.rows = rows;
  f.np = n_pad;
  f.rows_valid = rows_valid;
  f.n_valid = n_valid;
  f.o_sb = o_sb;
  f.o_sr = o_sr;
  f.o_sj = o_sj;
  f.heads = heads;
  f.kstages = nullptr;
  if (rows_valid == 0 || n_valid == 0) return ok();
  launch_flash(f, static_cast<hipStream_t>(stream));
  return check_launch("flash_attention_bias");
}

size_t ffk_transition_workspace(int64_t rows, int32_t d, int32_t factor) {
  if (rows < 0 || d <= 0 || factor <= 0) return 0;
  return transition_ws(nullptr, rows, d, factor).bytes;
}

int32_t ffk_transition(const void* x, const float* ln_w, const float* ln_b,
                       const float* w_expand_a, const float* w_expand_b,
                       const float* w_squeeze, void* out, void* workspace,
                       size_t workspace_bytes, int64_t rows, int32_t d, int32_t factor,
                       int32_t residual, float eps, void* stream) {
  if (int32_t s = check_device()) return s;
  if (int32_t s = transition_check(x, ln_w, ln_b, w_expand_a, w_expand_b, w_squeeze, out, rows, d, factor))
    return s;
  const TransitionWs need = transition_ws(nullptr, rows, d, factor);
  if (!workspace || workspace_bytes < need.bytes || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "transition: workspace %zu bytes < %zu", workspace_bytes, need.bytes);
  if (rows == 0) return ok();
  return transition_run(transition_ws(workspace, rows, d, factor), x, ln_w, ln_b, w_expand_a, w_expand_b,
                        w_squeeze, out, rows, d, factor, residual, eps, static_cast<hipStream_t>(stream));
}

int32_t ffk_transition_noalloc(const void* x, const float* ln_w, const float* ln_b,
                               const float* w_expand_a, const float* w_expand_b,
                               const float* w_squeeze, void* out, int64_t rows, int32_t d,
                               int32_t factor, int32_t residual, float eps, void* stream) {
  if (int32_t s = check_device()) return s;
  if (int32_t s = transition_check(x, ln_w, ln_b, w_expand_a, w_expand_b, w_squeeze, out, rows, d, factor))
    return s;
  const size_t need = transition_ws(nullptr, rows, d, factor).bytes;
  if (need > kNoAllocScratchBytes)
    return fail(FFK_ERR_WORKSPACE, "transition_noalloc: d=%d factor=%d rows=%lld needs %zu bytes of scratch; the static scratch holds %zu (use ffk_transition with a workspace)",
                d, factor, (long long)rows, need, kNoAllocScratchBytes);
  if (rows == 0) return ok();
  void* base = nullptr;
  if (int32_t s = noalloc_scratch(&base)) return s;
  return transition_run(transition_ws(base, rows, d, factor), x, ln_w, ln_b, w_expand_a, w_expand_b,
                        w_squeeze, out, rows, d, factor, residual, eps, static_cast<hipStream_t>(stream));
}

int32_t ffk_layer_norm_linear(const void* x, const float* ln_w, const float* ln_b,
                              const float* weight, const float* bias, void* y, int64_t rows,
                              int32_t d_in, int32_t d_out, int32_t activation, int32_t out_dtype,
                              float eps, void* stream) {
  if (int32_t s = check_device()) return s;
  if (!x || !weight || !y) return fail(FFK_ERR_INVALID, "layer_norm_linear: null tensor");
  if (rows < 0 || d_in <= 0 || d_in % 64 != 0 || d_in > kLnGemmMaxK || d_out <= 0 || d_out % 32 != 0)
    return fail(FFK_ERR_INVALID, "layer_norm_linear: rows=%lld d_in=%d d_out=%d (d_in a multiple of 64 up to %d, d_out a multiple of 32)",
                (long long)rows, d_in, d_out, kLnGemmMaxK);
  if (activation < FFK_ACT_NONE || activation > FFK_ACT_RELU)
    return fail(FFK_ERR_INVALID, "layer_norm_linear: unknown activation %d", activation);
  if (out_dtype != FFK_DTYPE_BF16 && out_dtype != FFK_DTYPE_F32)
    return fail(FFK_ERR_INVALID, "layer_norm_linear: unknown output dtype %d", out_dtype);
  if ((rows + 31) / 32 > 0x7fffffffLL) return fail(FFK_ERR_INVALID, "layer_norm_linear: too many rows");
  if (!aligned16(x) || !aligned16(y) || !aligned16(weight) || (ln_w && !aligned16(ln_w)) ||
      (ln_b && !aligned16(ln_b)))
    return fail(FFK_ERR_INVALID, "layer_norm_linear: x, y, weight and the norm affine must be 16-byte aligned");
  if (rows == 0) return ok();
  RowGemmArgs g{};
  g.ln_x = static_cast<const bf16*>(x);
  g.ln_w = ln_w;
  g.ln_b = ln_b;
  g.eps = eps;
  g.w0 = weight;
  g.M = rows;
  g.K = d_in;
  g.O = d_out;
  g.bias_out = bias;
  g.act = activation;
  g.y_f32 = out_dtype == FFK_DTYPE_F32 ? 1 : 0;
  g.y = y;
  launch_row_gemm(g, kEpiLinear, kXLn, static_cast<hipStream_t>(stream));
  return check_launch("layer_norm_linear");
}

size_t ffk_swiglu_ffn_workspace(int64_t rows, int32_t hidden) {
  if (rows < 0 || hidden <= 0) return 0;
  return up256((size_t)rows * hidden * sizeof(float));
}

int32_t ffk_swiglu_ffn(const void* x, const float* w_a, const float* w_b, const float* w_out,
                       const void* residual, void* out, void* workspace, size_t workspace_bytes,
                       int64_t rows, int32_t d, int32_t hidden, void* stream) {
  if (int32_t s = check_device()) return s;
  if (!x || !w_a || !w_b || !w_out || !out) return fail(FFK_ERR_INVALID, "swiglu_ffn: null argument");
  if (rows < 0 || d <= 0 || d % 64 != 0 || d > kLnGemmMaxK || hidden <= 0 || hidden % 64 != 0)
    return fail(FFK_ERR_INVALID, "swiglu_ffn: rows=%lld d=%d hidden=%d (d a multiple of 64 up to %d, hidden a multiple of 64)",
                (long long)rows, d, hidden, kLnGemmMaxK);
  if ((rows + 31) / 32 > 0x7fffffffLL) return fail(FFK_ERR_INVALID, "swiglu_ffn: too many rows");
  if (!aligned16(x) || !aligned16(out) || !aligned16(w_a) || !aligned16(w_b) || !aligned16(w_out) ||
      (residual && !aligned16(residual)))
    return fail(FFK_ERR_INVALID, "swiglu_ffn: tensors must be 16-byte aligned");
  const size_t need = ffk_swiglu_ffn_workspace(rows, hidden);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "swiglu_ffn: workspace %zu bytes < %zu", workspace_bytes, need);
  if (rows == 0) return ok();
  hipStream_t st = static_cast<hipStream_t>(stream);
  RowGemmArgs g{};
  g.w_split = 1;  // fp32-accurate weights (see row_gemm)
  g.ln_x = static_cast<const bf16*>(x);
  g.ln_plain = 1;
  g.w0 = w_a;
  g.w1 = w_b;
  g.M = rows;
  g.K = d;
  g.O = 2 * hidden;
  g.h32 = static_cast<float*>(workspace);
  launch_row_gemm(g, kEpiSwiglu, kXLn, st);
  RowGemmArgs s{};
  s.w_split = 1;  // fp32-accurate weights (see row_gemm)
  s.x32 = static_cast<const float*>(workspace);
  s.w0 = w_out;
  s.M = rows;
  s.K = hidden;
  s.O = d;
  s.res = static_cast<const bf16*>(residual);
  s.out = static_cast<bf16*>(out);
  s.residual = residual ? 1 : 0;
  launch_row_gemm(s, kEpiResid, kXF32, st);
  return check_launch("swiglu_ffn");
}

size_t ffk_attention_pair_bias_workspace(int64_t batch, int64_t n, int32_t d_single,
                                         int32_t d_pair, int32_t n_head) {
  if (batch <= 0 || n <= 0 || d_single <= 0 || d_pair <= 0 || n_head <= 0) return 0;
  return apb_ws(nullptr, batch, n, d_single, n_head).bytes;
}

int32_t ffk_attention_pair_bias(
    const void* s, const void* z, const uint8_t* key_mask, const float* ln_single_w,
    const float* ln_single_b, const float* w_query, const float* b_query, const float* w_key,
    const float* w_value, const float* ln_pair_w, const float* w_bias, const float* w_gate,
    const float* w_out, const void* extra_bias, int32_t extra_bf16, int64_t extra_stride_b,
    int64_t extra_stride_h, int64_t extra_stride_i, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t n, int32_t d_single, int32_t d_pair,
    int32_t n_head, float gate_bias, int32_t residual, float eps_single, float eps_pair,
    void* stream) {
  if (int32_t st = check_device()) return st;
  if (extra_bias && (extra_stride_b < 0 || extra_stride_h < 0 || extra_stride_i < 0))
    return fail(FFK_ERR_INVALID, "attention_pair_bias: negative extra_bias stride");
  if (d_pair != 128)
    return fail(FFK_ERR_INVALID, "attention_pair_bias: d_pair=%d (kernels take 128)", d_pair);
  if (n_head <= 0 || n_head > 32 || d_single <= 0 || d_single % 64 != 0 || d_single > kLnGemmMaxK ||
      d_single % n_head != 0 || (d_single / n_head) % 8 != 0 || d_single / n_head > 32)
    return fail(FFK_ERR_INVALID, "attention_pair_bias: d_single=%d heads=%d (kernels take a multiple of 64 up to %d split into at most 32 heads of 8, 16, 24 or 32)", d_single, n_head, kLnGemmMaxK);
  if (batch <= 0 || n <= 0) return fail(FFK_ERR_INVALID, "attention_pair_bias: empty shape");
  if (batch > 65535 || n > (1 << 24))
    return fail(FFK_ERR_INVALID, "attention_pair_bias: batch=%lld n=%lld exceed the launch grid", (long long)batch, (long long)n);
  if (!s || !z || !key_mask || !ln_single_w || !ln_single_b || !w_query || !b_query || !w_key ||
      !w_value || !ln_pair_w || !w_bias || !w_gate || !w_out || !out)
    return fail(FFK_ERR_INVALID, "attention_pair_bias: null argument");
  if (!aligned16(s) || !aligned16(z) || !aligned16(out))
    return fail(FFK_ERR_INVALID, "attention_pair_bias: s/z/out must be 16-byte aligned");
  if (!aligned16(w_query) || !aligned16(w_key) || !aligned16(w_value) || !aligned16(w_gate) ||
      !aligned16(w_out))
    return fail(FFK_ERR_INVALID, "attention_pair_bias: projection weights must be 16-byte aligned");
  const ApbWs need = apb_ws(nullptr, batch, n, d_single, n_head);
  if (!workspace || workspace_bytes < need.bytes || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "attention_pair_bias: workspace %zu bytes < %zu", workspace_bytes, need.bytes);
  const ApbWs w = apb_ws(workspace, batch, n, d_single, n_head);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rows = batch * n;
  const int64_t np = pad32(n);
  const int dh = d_single / n_head;
  RowGemmArgs p{};
  p.w_split = 1;  // fp32-accurate weights (see row_gemm)
  p.ln_x = static_cast<const bf16*>(s);
  p.ln_w = ln_single_w;
  p.ln_b = ln_single_b;
  p.eps = eps_single;
  p.w0 = w_query;
  p.w1 = w_key;
  p.w2 = w_value;
  p.w3 = w_gate;
  p.M = rows;
  p.K = d_single;
  p.O = 4 * d_single;
  p.q_bias = b_query;
  p.q_scale = kLog2e / sqrtf((float)dh);
  p.gate_bias = gate_bias;
  p.q = w.q;
  p.k = w.k;
  p.vt = w.vt;
  p.gate = w.gate;
  p.n = (int)n;
  p.np = (int)np;
  p.heads = n_head;
  p.dh = dh;
  launch_row_gemm(p, kEpiApb, kXLn, st);

  PairBiasArgs pb{};
  pb.z = static_cast<const bf16*>(z);
  pb.mask = key_mask;
  pb.ln_w = ln_pair_w;
  pb.w_bias = w_bias;
  pb.bias = w.bias;
  pb.tiles = batch * n * (np / 32);
  pb.n = (int)n;
  pb.np = (int)np;
  pb.heads = n_head;
  pb.eps = eps_pair;
  pb.c = 128;
  pb.transposed = 0;
  pb.extra = extra_bias;
  pb.extra_bf16 = extra_bf16 ? 1 : 0;
  pb.extra_sb = extra_stride_b;
  pb.extra_sh = extra_stride_h;
  pb.extra_si = extra_stride_i;
  launch_apb_pair_bias(pb, st);

  ApbAttnArgs at;
  at.q = w.q;
  at.k = w.k;
  at.vt = w.vt;
  at.gate = w.gate;
  at.bias = w.bias;
  at.mask = key_mask;
  at.og = w.og;
  at.n = (int)n;
  at.np = (int)np;
  at.heads = n_head;
  at.dh = dh;
  at.cs = d_single;
  at.rows_per_bias = 1;
  launch_apb_attention(at, (int)batch, st);

  RowGemmArgs o{};
  o.w_split = 1;  // fp32-accurate weights (see row_gemm)
  o.x32 = w.og;
  o.w0 = w_out;
  o.M = rows;
  o.K = d_single;
  o.O = d_single;
  o.res = static_cast<const bf16*>(s);
  o.out = static_cast<bf16*>(out);
  o.residual = residual ? 1 : 0;
  launch_row_gemm(o, kEpiResid, kXF32, st);
  return check_launch("attention_pair_bias");
}

size_t ffk_msa_pair_weighted_averaging_workspace(int64_t batch, int64_t depth, int64_t n,
                                                  int32_t d_msa, int32_t d_pair, int32_t n_head,
                                                  int32_t d_head) {
  if (batch <= 0 || depth <= 0 || n <= 0 || d_msa <= 0 || d_pair <= 0 || n_head <= 0 || d_head <= 0)
    return 0;
  return pwa_ws(nullptr, batch, depth, n, n_head, d_head).bytes;
}

int32_t ffk_msa_pair_weighted_averaging(
    const void* m, const void* z, const uint8_t* key_mask, const float* ln_msa_w,
    const float* ln_msa_b, const float* ln_pair_w, const float* w_bias, const float* w_value,
    const float* w_gate, const float* w_out, void* out, void* workspace, size_t workspace_bytes,
    int64_t batch, int64_t depth, int64_t n, int32_t d_msa, int32_t d_pair, int32_t n_head,
    int32_t d_head, int32_t residual, float eps_msa, float eps_pair, void* stream) {
  if (int32_t st = check_device()) return st;
  const int64_t hd = (int64_t)n_head * d_head;
  if (d_pair != 128)
    return fail(FFK_ERR_INVALID, "msa_pair_weighted_averaging: d_pair=%d (kernels take 128)", d_pair);
  if (d_msa <= 0 || d_msa % 64 != 0 || d_msa > kLnGemmMaxK || n_head <= 0 || n_head > 32 ||
      d_head <= 0 || d_head % 4 != 0 || hd % 64 != 0 || hd > kLnGemmMaxK)
    return fail(FFK_ERR_INVALID, "msa_pair_weighted_averaging: d_msa=%d heads=%d x %d (kernels take d_msa a multiple of 64 up to %d, at most 32 heads, d_head a multiple of 4, heads * d_head a multiple of 64 up to %d)", d_msa, n_head, d_head, kLnGemmMaxK, kLnGemmMaxK);
  if (batch <= 0 || depth <= 0 || n <= 0) return fail(FFK_ERR_INVALID, "msa_pair_weighted_averaging: empty shape");
  if ((depth * d_head + 127) / 128 * ((n + 127) / 128) * batch * n_head > 0x7fffffffLL ||
      batch * n_head * n > 0x7fffffffLL * 4)
    return fail(FFK_ERR_INVALID, "msa_pair_weighted_averaging: shape exceeds the launch grid");
  if (!m || !z || !key_mask || !ln_msa_w || !ln_msa_b || !ln_pair_w || !w_bias || !w_value ||
      !w_gate || !w_out || !out)
    return fail(FFK_ERR_INVALID, "msa_pair_weighted_averaging: null argument");
  if (!aligned16(m) || !aligned16(z) || !aligned16(out) || !aligned16(w_value) ||
      !aligned16(w_gate) || !aligned16(w_out))
    return fail(FFK_ERR_INVALID, "msa_pair_weighted_averaging: m/z/out and the projection weights must be 16-byte aligned");
  const PwaWs need = pwa_ws(nullptr, batch, depth, n, n_head, d_head);
  if (!workspace || workspace_bytes < need.bytes || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "msa_pair_weighted_averaging: workspace %zu bytes < %zu", workspace_bytes, need.bytes);
  const PwaWs w = pwa_ws(workspace, batch, depth, n, n_head, d_head);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rows = batch * depth * n;
  const int64_t np = pad64(n);

  RowGemmArgs p{};
  p.ln_x = static_cast<const bf16*>(m);
  p.ln_w = ln_msa_w;
  p.ln_b = ln_msa_b;
  p.eps = eps_msa;
  p.w0 = w_value;
  p.w1 = w_gate;
  p.M = rows;
  p.K = d_msa;
  p.O = (int)(2 * hd);
  p.vt = w.vt;
  p.gate = w.gate;
  p.n = (int)n;
  p.np = (int)np;
  p.heads = n_head;
  p.dh = d_head;
  p.depth = (int)depth;
  launch_row_gemm(p, kEpiPwa, kXLn, st);

  PairBiasArgs pb{};
  pb.z = static_cast<const bf16*>(z);
  pb.mask = key_mask;
  pb.ln_w = ln_pair_w;
  pb.w_bias = w_bias;
  pb.bias = w.logits;
  pb.tiles = batch * n * (np / 32);
  pb.n = (int)n;
  pb.np = (int)np;
  pb.heads = n_head;
  pb.eps = eps_pair;
  pb.c = 128;
  pb.transposed = 0;
  launch_apb_pair_bias(pb, st);

  PwaSoftmaxArgs sm;
  sm.logits = w.logits;
  sm.w = w.w;
  sm.rows = batch * n_head * n;
  sm.np = (int)np;
  launch_pwa_softmax(sm, st);

  PwaAverageArgs av;
  av.vt = w.vt;
  av.w = w.w;
  av.gate = w.gate;
  av.og = w.og;
  av.batch = (int)batch;
  av.heads = n_head;
  av.depth = (int)depth;
  av.n = (int)n;
  av.np = (int)np;
  av.dh = d_head;
  launch_pwa_average(av, st);

  RowGemmArgs o{};
  o.ln_x = w.og;
  o.ln_plain = 1;
  o.w0 = w_out;
  o.M = rows;
  o.K = (int)hd;
  o.O = d_msa;
  o.res = static_cast<const bf16*>(m);
  o.out = static_cast<bf16*>(out);
  o.residual = residual ? 1 : 0;
  launch_row_gemm(o, kEpiResid, kXLn, st);
  return check_launch("msa_pair_weighted_averaging");
}

// Chai-1's grouped form: both sides' projections (64 channels each) and the bf16 output weight.
struct OpmGroupedWs {
  bf16 *lt, *rt, *mt, *wp;
  size_t bytes;
};
OpmGroupedWs opm_grouped_ws(void* ws, int64_t batch, int64_t depth, int64_t n, int cz) {
  Carver cv{static_cast<char*>(ws)};
  const int64_t sp = pad64(depth);
  OpmGroupedWs w;
  w.lt = cv.take<bf16>((size_t)batch * n * 64 * sp);
  w.rt = cv.take<bf16>((size_t)batch * n * 64 * sp);
  w.mt = cv.take<bf16>((size_t)batch * n * sp);
  w.wp = cv.take<bf16>((size_t)cz * 512);
  w.bytes = cv.used;
  return w;
}

size_t ffk_outer_product_mean_workspace(int64_t batch, int64_t depth, int64_t n, int32_t d_msa,
                                        int32_t d_hidden, int32_t d_pair) {
  if (batch <= 0 || depth <= 0 || n <= 0 || d_msa <= 0 || d_hidden <= 0 || d_pair <= 0) return 0;
  return opm_ws(nullptr, batch, depth, n, d_pair).bytes;
}

int32_t ffk_outer_product_mean(
    const void* m, const uint8_t* rows_mask, const float* ln_w, const float* ln_b,
    const float* w_left, const float* b_left, const float* w_right, const float* b_right,
    const float* w_out, const float* b_out, const void* residual, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t depth, int64_t n, int32_t d_msa,
    int32_t d_hidden, int32_t d_pair, float eps, float count_offset,
    int32_t normalize_before_proj, void* stream) {
  if (int32_t st = check_device()) return st;
  if (d_hidden != 32 || d_pair != 128)
    return fail(FFK_ERR_INVALID, "outer_product_mean: d_hidden=%d d_pair=%d (kernels take 32 and 128)", d_hidden, d_pair);
  if (d_msa <= 0 || d_msa % 64 != 0 || d_msa > kLnGemmMaxK)
    return fail(FFK_ERR_INVALID, "outer_product_mean: d_msa=%d (kernels take a multiple of 64 up to %d)", d_msa, kLnGemmMaxK);
  if (batch <= 0 || depth <= 0 || n <= 0) return fail(FFK_ERR_INVALID, "outer_product_mean: empty shape");
  const int64_t sp = pad64(depth);
  const int64_t nt = (n + 7) / 8;
  if (batch > 65535 || (n + 31) / 32 > 65535 || nt * nt * batch > 0x7fffffffLL ||
      batch * n * sp / 32 > 0x7fffffffLL || n * n > 0x7fffffffLL)
    return fail(FFK_ERR_INVALID, "outer_product_mean: shape exceeds the launch grid");
  if (!m || !rows_mask || !ln_w || !ln_b || !w_left || !w_right || !w_out || !b_out || !out)
    return fail(FFK_ERR_INVALID, "outer_product_mean: null argument");
  if (!aligned16(m) || !aligned16(out) || !aligned16(w_left) || !aligned16(w_right) ||
      !aligned16(b_out) || (residual && !aligned16(residual)))
    return fail(FFK_ERR_INVALID, "outer_product_mean: m/out/residual, the projection weights and the output bias must be 16-byte aligned");
  const OpmWs need = opm_ws(nullptr, batch, depth, n, d_pair);
  if (!workspace || workspace_bytes < need.bytes || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "outer_product_mean: workspace %zu bytes < %zu", workspace_bytes, need.bytes);
  const OpmWs w = opm_ws(workspace, batch, depth, n, d_pair);
  hipStream_t st = static_cast<hipStream_t>(stream);

  RowGemmArgs p{};
  p.ln_x = static_cast<const bf16*>(m);
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.eps = eps;
  p.w0 = w_left;
  p.w1 = w_right;
  p.bias0 = b_left;
  p.bias1 = b_right;
  p.M = batch * n * sp;
  p.K = d_msa;
  p.O = 64;
  p.n = (int)n;
  p.depth = (int)depth;
  p.sp = (int)sp;
  p.rows_mask = rows_mask;
  p.lt = w.lt;
  p.rt = w.rt;
  p.mt = w.mt;
  launch_row_gemm(p, kEpiOpm, kXLn, st);

  OpmCountArgs c;
  c.mt = w.mt;
  c.count = w.count;
  c.batch = (int)batch;
  c.n = (int)n;
  c.sp = (int)sp;
  launch_opm_count(c, st);

  launch_opm_pack(w_out, w.wp, d_pair, st);

  OpmContractArgs o;
  o.lt = w.lt;
  o.rt = w.rt;
  o.wp = w.wp;
  o.bias = b_out;
  o.count = w.count;
  o.res = static_cast<const bf16*>(residual);
  o.out = static_cast<bf16*>(out);
  o.batch = (int)batch;
  o.n = (int)n;
  o.sp = (int)sp;
  o.cz = d_pair;
  o.count_offset = count_offset;
  o.normalize_before_proj = normalize_before_proj ? 1 : 0;
  launch_opm_contract(o, st);
  return check_launch("outer_product_mean");
}

size_t ffk_outer_product_mean_grouped_workspace(int64_t batch, int64_t depth, int64_t n,
                                                int32_t d_msa, int32_t groups, int32_t d_group,
                                                int32_t d_pair) {
  if (batch <= 0 || depth <= 0 || n <= 0 || d_msa <= 0 || groups <= 0 || d_group <= 0 || d_pair <= 0)
    return 0;
  return opm_grouped_ws(nullptr, batch, depth, n, d_pair).bytes;
}

int32_t ffk_outer_product_mean_grouped(
    const void* m, const uint8_t* rows_mask, const float* ln_w, const float* ln_b,
    const float* w_left, const float* b_left, const float* w_right, const float* b_right,
    const float* norm_w, const float* norm_b, const float* w_out, const float* b_out,
    const void* residual, void* out, void* workspace, size_t workspace_bytes, int64_t batch,
    int64_t depth, int64_t n, int32_t d_msa, int32_t groups, int32_t d_group, int32_t d_pair,
    float eps, float norm_eps, void* stream) {
  if (int32_t st = check_device()) return st;
  if (groups != 8 || d_group != 8 || (d_pair != 128 && d_pair != 256))
    return fail(FFK_ERR_INVALID, "outer_product_mean_grouped: %d groups of %d, d_pair=%d (kernels take 8 groups of 8 and d_pair 128 or 256)", groups, d_group, d_pair);
  if (d_msa <= 0 || d_msa % 64 != 0 || d_msa > kLnGemmMaxK)
    return fail(FFK_ERR_INVALID, "outer_product_mean_grouped: d_msa=%d (kernels take a multiple of 64 up to %d)", d_msa, kLnGemmMaxK);
  if (batch <= 0 || depth <= 0 || n <= 0) return fail(FFK_ERR_INVALID, "outer_product_mean_grouped: empty shape");
  const int64_t sp = pad64(depth);
  const int64_t tiles = ((n + 3) / 4) * ((n + 7) / 8) * batch;
  if (batch > 65535 || tiles > 0x7fffffffLL || batch * n * sp / 32 > 0x7fffffffLL || n * n > 0x7fffffffLL)
    return fail(FFK_ERR_INVALID, "outer_product_mean_grouped: shape exceeds the launch grid");
  if (!m || !rows_mask || !ln_w || !ln_b || !w_left || !w_right || !norm_w || !norm_b || !w_out ||
      !b_out || !out)
    return fail(FFK_ERR_INVALID, "outer_product_mean_grouped: null argument");
  if (!aligned16(m) || !aligned16(out) || !aligned16(w_left) || !aligned16(w_right) ||
      !aligned16(b_out) || (residual && !aligned16(residual)))
    return fail(FFK_ERR_INVALID, "outer_product_mean_grouped: m/out/residual, the projection weights and the output bias must be 16-byte aligned");
  const OpmGroupedWs need = opm_grouped_ws(nullptr, batch, depth, n, d_pair);
  if (!workspace || workspace_bytes < need.bytes || !aligned16(workspace))
    return fail(FFK_ERR_WORKSPACE, "outer_product_mean_grouped: workspace %zu bytes < %zu", workspace_bytes, need.bytes);
  const OpmGroupedWs w = opm_grouped_ws(workspace, batch, depth, n, d_pair);
  hipStream_t st = static_cast<hipStream_t>(stream);

  // LayerNorm + both 64-channel projections, masked, MSA rows contiguous (l^T, r^T)
  RowGemmArgs p{};
  p.ln_x = static_cast<const bf16*>(m);
  p.ln_w = ln_w;
  p.ln_b = ln_b;
  p.eps = eps;
  p.w0 = w_left;
  p.w1 = w_right;
  p.bias0 = b_left;
  p.bias1 = b_right;
  p.M = batch * n * sp;
  p.K = d_msa;
  p.O = 128;
  p.n = (int)n;
  p.depth = (int)depth;
  p.sp = (int)sp;
  p.rows_mask = rows_mask;
  p.lt = w.lt;
  p.rt = w.rt;
  p.mt = w.mt;
  launch_row_gemm(p, kEpiOpm, kXLn, st);

  PackJob job{};
  job.seg[0] = {w_out, w.wp, (int64_t)d_pair * 512, 1.f};
  job.nseg = 1;
  launch_pack(job, st);

  OpmGroupedArgs o;
  o.lt = w.lt;
  o.rt = w.rt;
  o.wp = w.wp;
  o.bias = b_out;
  o.norm_w = norm_w;
  o.norm_b = norm_b;
  o.res = static_cast<const bf16*>(residual);
  o.out = static_cast<bf16*>(out);
  o.batch = (int)batch;
  o.n = (int)n;
  o.sp = (int)sp;
  o.cz = d_pair;
  o.norm_eps = norm_eps;
  launch_opm_contract_grouped(o, st);
  return check_launch("outer_product_mean_grouped");
}

}  // extern "C"
