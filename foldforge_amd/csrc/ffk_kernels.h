// Host-side launch interfaces of the pair-stack kernels (one struct per op, filled by
// the C-ABI layer in api.hip after it has validated shapes and carved the workspace).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ffk_device.h"

namespace ffk {

struct TrimulArgs {
  const bf16* z;
  const uint8_t* mask;
  const float *ln_w, *ln_b, *lno_w, *lno_b;
  const bf16* wp;  // [4h][c]: left, left_gate, right, right_gate
  const bf16* wg;  // [c][c]
  const bf16* wo;  // [c][h]
  bf16 *A, *B, *P;  // [batch][h][np][np]
  float* maskf;     // [batch][np] scratch: the key mask as 1 / 0, zero past n
  const int* kstages;  // [batch] 32-wide k stages up to the last real key (NULL: all)
  bf16* out;
  int batch, n, np, outgoing, residual;
  float eps;
  const float* eps_out;  // device epsilon of the centre norm (NULL: eps)
};
void launch_trimul(const TrimulArgs& a, hipStream_t stream);
// eps_out[0] = eps * L^2 for the length-divided contraction, L the number of positions real in
// any batch element (at least 1), from the key mask [batch][n].
void launch_length_eps(const uint8_t* mask, int batch, int n, float eps, float* eps_out,
                       hipStream_t stream);
// P[p] = X[p] Y[p]^T for `planes` planes of [np][np] bf16 (np % 128 == 0). With kstages, plane
// p runs only the first kstages[p / planes_per_batch] k stages of 32 (the operands are zero past
// them, so the product is unchanged).
void launch_trimul_contract(const bf16* A, const bf16* B, bf16* P, int64_t planes, int np,
                            hipStream_t stream, const int* kstages = nullptr,
                            int planes_per_batch = 1);

struct TriattnArgs {
  const bf16* z;
  const uint8_t* mask;
  const float* maskf;  // [batch][np] key mask as 1 / 0, zero past n
  const float *ln_w, *ln_b;
  const bf16* wqkv;  // [3 * 128][128], query rows carry d^-1/2 * log2(e)
  const bf16* wb;    // [32][128], rows < heads carry log2(e) * to_bias, others zero
  const bf16* wg;    // [128][128] to_gate
  const bf16* wo;    // [128][128] to_out
  bf16 *q, *k, *vt;  // [batch * heads][np][np][32], vt: [batch * heads][np][np / 32][32][32]
  float* bias;       // [batch * heads][np / 32][np / 32][2][32][16] blocked, see triattn.hip
  const int* kstages;  // [batch] key stages holding a real key (written by the weight packing)
  bf16* o;           // [batch][n][n][128] z-frame attention output
  const float *bg, *bo;  // gate / output projection biases [128] (NULL: none)
  int form;          // kTriattn*: how the update reaches out
  const bf16* wo_t;  // kTriattnDual: the second output projection [128][128] and its bias
  const float* bo_t;
  bf16* tbuf;        // kTriattnUntransposed / kTriattnDual: [batch][n][n][128] update scratch
  bf16* out;
  int batch, n, np, heads, starting, transposed_bias, residual;
  float eps;
  int project_only;  // 1: the projection and the flash core only (o in z frame, no output)
};
// Output forms: the z-frame update (AF3 and its descendants); the update transposed (Chai-1's
// trunk, ending node); the update plus the transpose of a second projection's (Chai-1's
// confidence head).
enum { kTriattnStandard = 0, kTriattnUntransposed = 1, kTriattnDual = 2 };
void launch_triattn(const TriattnArgs& a, hipStream_t stream);
// out[b][i][j][:] = (base ? base[b][i][j][:] : 0) + t[b][j][i][:] for c channels (c % 8 == 0);
// base may be out, t may not.
void launch_pair_add_transposed(const bf16* base, const bf16* t, bf16* out, int64_t batch, int n,
                                int c, hipStream_t stream);

struct FlashArgs {
  const bf16 *q, *k, *vt;
  const float* bias;  // blocked pair bias (log2 units, -inf at masked keys)
  bf16* o;
  int64_t batch, rows, np, rows_valid, n_valid, o_sb, o_sr, o_sj;
  int heads;
  // optional [batch] key-stage counts: the stages past them hold only masked keys (bias
  // -inf), which add exact zeros, and are skipped (NULL: every stage runs)
  const int* kstages;
  // Head width 16 or 32: q, k [batch heads][rows][np][dh], v^T [batch heads][rows][dh][np]
  // (keys permuted as the 32-wide layout). With og set, the kernel writes the gated output
  // og = gate * o (bf16) instead of o, at the same strides (in elements) plus h dh + d, and
  // reads the gate (bf16) at that offset too.
  int dh = 32;
  const bf16* gate = nullptr;
  bf16* og = nullptr;
};
void launch_flash(const FlashArgs& a, hipStream_t stream);

struct TransitionArgs {
  const bf16* x;
  const float *ln_w, *ln_b;
  const bf16* w;  // expand_a, expand_b, squeeze as written by launch_transition_pack
  bf16* out;
  int64_t rows;
  int residual;
  float eps;
};
// expand_a [4c][c], expand_b [4c][c], squeeze [c][4c] (fp32) -> the transition kernel's packed
// bf16 weight stream (3 * 4c * c elements).
void launch_transition_pack(const float* wa, const float* wb, const float* ws, bf16* dst,
                            hipStream_t stream);
void launch_transition(const TransitionArgs& a, hipStream_t stream);
// Triangle attention's gate / output projection (no biases) fused in front of the pair
// transition: out = y + transition(y), y = z + (sigmoid(LN_pair(z) w_gate^T) * o) w_out^T with
// y rounded to bf16 (the two ops' result). z, o, out [rows][128] bf16 (out may alias z); w as
// written by launch_attention_transition_pack (gate [128][128], out [128][128] and the
// transition's weights: (16 + 3) * 12288 elements).
struct AttnTransitionArgs {
  const bf16 *z, *o;
  const float *lnp_w, *lnp_b;  // the attention's pair LayerNorm
  const float *ln_w, *ln_b;    // the transition's LayerNorm
  const bf16* w;
  bf16* out;
  int64_t rows;
  float eps_pair, eps;
};
void launch_attention_transition_pack(const float* wg, const float* wo, const float* wa,
                                      const float* wb, const float* ws, bf16* dst,
                                      hipStream_t stream);
void launch_attention_output_transition(const AttnTransitionArgs& a, hipStream_t stream);

// Token-row GEMM out[m][o] = sum_k W[o][k] x[m][k] (single track, single.hip) with one of
// three epilogues, x either LayerNorm(ln_x) (kXLn, K <= kLnGemmMaxK) or fp32 rows x32 (kXF32).
// K % 64 == 0, O % 32 == 0; weights are the fp32 parameters. Pairs served: (kEpiApb, kXLn),
// (kEpiSwiglu, kXLn), (kEpiResid, kXF32), (kEpiResid, kXLn), (kEpiPwa, kXLn), (kEpiOpm, kXLn), (kEpiTrimul, kXLn),
// (kEpiStoreY, kXLn), (kEpiGateResid, kXLn), (kEpiLinear, kXLn).
enum {
  kEpiApb = 0,
  kEpiSwiglu = 1,
  kEpiResid = 2,
  kEpiPwa = 3,
  kEpiOpm = 4,
  kEpiTrimul = 5,     // gated, masked left / right projections into channel planes
  kEpiStoreY = 6,     // hy = y (bf16)
  kEpiGateResid = 7,  // out = res + yin * sigmoid(y) (or yin * sigmoid(y))
  kEpiLinear = 8,     // y = act(W x + bias_out), bf16 or fp32 rows [M][O]
};
// kEpiLinear activations (the C-ABI's FFK_ACT_* values)
enum { kActNone = 0, kActSigmoid = 1, kActSilu = 2, kActRelu = 3 };
// Row maps (RowGemmArgs.tmap): the input row read for logical row m, and the rows the epilogue
// of kEpiResid writes. kMapPairT: m = (b n + r) n + j reads row (b n + j) n + r (the
// transposed pair); kMapGridOut / kMapGridIn: m = (b npm + i) npm + k over the padded grid
// reads pair row (b n + i) n + k / (b n + k) n + i (clamped past n); kMapPadKeys /
// kMapPadKeysT: m = (b n + r) np + j over keys padded to np reads pair row (b n + r) n + j' /
// (b n + j') n + r with j' = min(j, n - 1).
enum { kMapIdentity = 0, kMapPairT = 1, kMapGridOut = 2, kMapGridIn = 3, kMapPadKeys = 4, kMapPadKeysT = 5 };
// kXBf16: bf16 rows entered as they are (the streaming kernel's form of kXLn with ln_plain)
enum { kXLn = 0, kXF32 = 1, kXBf16 = 2 };
constexpr int kLnGemmMaxK = 768;
struct RowGemmArgs {
  const bf16* ln_x;             // kXLn: [M][K] rows to normalise with ln_w, ln_b, eps
  const float *ln_w, *ln_b;     // NULL: weight 1 / offset 0
  float eps;
  const float* eps_dev;         // kXLn: device epsilon, read in place of eps (NULL: eps)
  int ln_plain;                 // kXLn with 1: the rows enter as they are (no normalisation)
  const float* x32;             // kXF32: [M][K]
  // kEpiApb: w0..w3 = to_query, to_key, to_value, to_gate ([cs][cs] each, O = 4 cs);
  // kEpiSwiglu: w0 = expand_a, w1 = expand_b ([hid][K] each, O = 2 hid);
  // kEpiResid: w0 = [O][K]
  const float *w0, *w1, *w2, *w3;
  // token-row GEMM (row_gemm): 1 = the weights enter as bf16 hi + lo as well, three MFMAs per
  // k step (W x to about fp32 accuracy, as fp32 parameters multiply in the reference); 0 = the
  // weights are rounded to bf16. The streaming GEMM (row_stream) always holds bf16 weights.
  int w_split;
  int64_t M;
  int K, O;
  // kEpiApb: q = (x W_q^T + q_bias) * q_scale, k, v^T [batch][heads][dh][np] (keys permuted
  // as in the attention kernel), gate = sigmoid(x W_g^T + gate_bias); q, k, gate [M][cs]
  const float* q_bias;
  float q_scale, gate_bias;
  const float* gate_b;          // kEpiApb: per-channel gate bias [cs] (NULL: none)
  bf16 *q, *k, *vt, *gate;
  int n, np, heads, dh;
  // kEpiApb with flash_rows > 0 (logical rows m = (b n + r) np + j, a kMapPadKeys* map): the
  // flash core's layouts, q, k [batch heads][flash_rows][np][dh] and v^T
  // [batch heads][flash_rows][dh][np] (keys permuted), written for every j < np; the gate
  // [batch n n][cs] for j < n
  int flash_rows;
  int apb_no_gate;  // kEpiApb: 1 = q, k, v only (O = 3 cs; the gate is computed downstream)
  // kEpiPwa: w0 = to_value, w1 = to_gate ([hd][K] each, O = 2 hd); tokens m = (b S + s) n + j;
  // v^T [batch][heads][S][dh][np] (bf16, keys contiguous), gate = sigmoid(x W_g^T) [M][hd]
  int depth;
  // kEpiOpm: w0 = to_left, w1 = to_right ([32][K] each, O = 64), bias0 / bias1 their biases
  // (NULL: none). Logical rows m = (b n + j) sp + s (s < sp, sp % 32 == 0) read MSA row
  // (b depth + s) n + j; rows with s >= depth, or masked in rows_mask [batch][depth][n],
  // project to 0. Outputs: lt / rt [batch][n][32][sp] (bf16, MSA rows contiguous) and mt
  // [batch][n][sp] (bf16 0 / 1, the row mask transposed).
  const uint8_t* rows_mask;
  const float *bias0, *bias1;
  bf16 *lt, *rt, *mt;
  int sp;
  // kEpiTrimul: w0..w3 = to_left, to_right, to_left_gate, to_right_gate ([hid][K], O = 4 hid),
  // tiles packed as 16 projection rows + their 16 gate rows; rows on the padded grid (kMapGrid*);
  // pa / pb [batch][hid][npm][npm] = proj * mask_i mask_k * sigmoid(gate), 0 past n.
  const uint8_t* mask;
  bf16 *pa, *pb;
  int tmap, npm;
  const bf16* yin;   // kEpiGateResid: [M][O]
  float* h32;  // kEpiSwiglu: [M][hid] = silu(a) * b
  bf16* hy;    // kEpiStoreY: [M][O] = y
  bf16* h16;   // kEpiSwiglu: the hidden rows in bf16 instead (h32 unused)
  const bf16* res;  // kEpiResid: out = res + y (residual) or y, y with bias_out when set
  bf16* out;
  int residual;
  const float* bias_out;  // kEpiLinear, kEpiResid: [O] or NULL
  int act, y_f32;         // kEpiLinear: kAct*, 1 = fp32 rows
  void* y;                // kEpiLinear: [M][O]
};
void launch_row_gemm(const RowGemmArgs& a, int epi, int xsrc, hipStream_t stream);

struct PairBiasArgs {
  const bf16* z;         // [batch][n][n][128]
  const uint8_t* mask;   // [batch][n]
  const float* ln_w;     // [128] pair-norm weight (the norm has no offset)
  const float* w_bias;   // [heads][128]
  float* bias;           // [batch][heads][n][np], log2 units, kMaskedLogit at masked keys
  int64_t tiles;         // batch * n * np / 32
  int n, np, heads;
  float eps;
  int c;                 // pair width: 64, 128 or 256
  int transposed;        // 1: the logit of (query i, key j) comes from z[b, j, i]
  // 1: bias in the flash core's blocked layout [batch heads][np / 32][np / 32][1024], -inf at
  // masked keys (rows of queries past n are left unwritten)
  int blocked;
  // optional extra logits (natural units) at extra[b sb + h sh + i si + j], fp32 or bf16
  // (extra_bf16); strides in elements, 0 broadcasts
  const void* extra;
  int extra_bf16;
  int64_t extra_sb, extra_sh, extra_si;
};
void launch_apb_pair_bias(const PairBiasArgs& a, hipStream_t stream);

struct ApbAttnArgs {
  const bf16 *q, *k, *vt, *gate;
  const float* bias;
  const uint8_t* mask;
  float* og;  // [M][cs] gate * attention output
  int n, np, heads, dh, cs;
  int rows_per_bias;  // attention batches sharing one bias and key mask (pair rows: n; else 1)
};
void launch_apb_attention(const ApbAttnArgs& a, int batch, hipStream_t stream);

// Generic-width triangle multiplication output at pair width 64, hidden width 64 or 128:
// out = (residual ? z : 0) + (LN_out(p) W_out^T) * sigmoid(LN_pair(z) W_g^T), p the contraction's
// channel planes.
struct TrimulPlanesArgs {
  const bf16* planes;             // [batch][hid][np][np]
  const bf16* z;                  // [batch][n][n][64]
  const float *lno_w, *lno_b;     // centre norm affine [hid]
  const float *ln_w, *ln_b;       // pair norm affine [64]
  const float *w_out, *w_gate;    // [64][hid], [64][64] fp32 parameters
  const float* eps_out;           // device epsilon of the centre norm (NULL: eps)
  bf16* out;                      // [batch][n][n][64]; may alias z
  int batch, n, np, hid;          // batch * n * ceil(n / 32) < 2^31
  int residual;
  float eps;
};
void launch_trimul_out_planes(const TrimulPlanesArgs& a, hipStream_t stream);

// Generic-width triangle attention output at pair width 64, gated width hd 64 or 128:
// out = (residual ? z : 0) + (sigmoid(LN_pair(z) W_g^T + b_g) * o) W_out^T + b_out.
struct TriattnRowsArgs {
  const bf16* z;                  // [batch][n][n][64]
  const bf16* o;                  // [batch][n][n][hd] attention output in the attention's frame
  const float *ln_w, *ln_b;       // pair norm affine [64]
  const float *w_gate, *b_gate;   // [hd][64], [hd] (NULL: none)
  const float *w_out, *b_out;     // [64][hd], [64] (NULL: none)
  bf16* out;                      // [batch][n][n][64]; may alias z
  int batch, n, hd;
  int transposed;                 // 1: position (b, i, j) takes o row (b, j, i)
  int residual;
  float eps;
};
void launch_triattn_out_rows(const TriattnRowsArgs& a, hipStream_t stream);

// Channel planes P [batch][hid][np][np] -> token rows Pt [batch][n][n][hid] (bf16).
void launch_planes_to_rows(const bf16* planes, bf16* rows, int batch, int hid, int n, int np,
                           hipStream_t stream);

// MSA pair-weighted averaging (msa.hip): the softmax over keys of the pair logits and the
// weighted average of every MSA row's values.
struct PwaSoftmaxArgs {
  const float* logits;  // [batch][heads][n][np] (log2 units, masked keys very negative)
  bf16* w;              // [batch][heads][n][np] softmax weights, 0 at masked / padding keys
  int64_t rows;         // batch * heads * n
  int np;
};
void launch_pwa_softmax(const PwaSoftmaxArgs& a, hipStream_t stream);

struct PwaAverageArgs {
  const bf16* vt;    // [batch][heads][S][dh][np]
  const bf16* w;     // [batch][heads][n][np]
  const bf16* gate;  // [batch][S][n][heads dh]
  bf16* og;          // [batch][S][n][heads dh] = gate * sum_j w[h][i][j] v[s][j][h], bf16
  int batch, heads, depth, n, np, dh;
};
void launch_pwa_average(const PwaAverageArgs& a, hipStream_t stream);

// Outer product mean (opm.hip). For every pair (i, j): o[(c, e)] = sum_s l[s][i][c] r[s][j][e]
// over the MSA rows, out = (o W^T scale1 + bias) scale2 with the count n_ij = sum_s
// m[s][i] m[s][j]: divisor d = n_ij + count_offset (count_offset >= 0) or max(n_ij, 1)
// (count_offset < 0); normalize_before_proj: scale1 = 1 / d, scale2 = 1, else scale1 = 1,
// scale2 = 1 / d. Optional residual: out = res + value.
struct OpmCountArgs {
  const bf16* mt;  // [batch][n][sp]
  float* count;    // [batch][n][n]
  int batch, n, sp;
};
void launch_opm_count(const OpmCountArgs& a, hipStream_t stream);
// to_out.weight [c_z][32 * 32] fp32 (column c * 32 + e) -> the contraction's bf16 order.
void launch_opm_pack(const float* w, bf16* wp, int cz, hipStream_t stream);
struct OpmContractArgs {
  const bf16 *lt, *rt;   // [batch][n][32][sp]
  const bf16* wp;        // [c_z][1024] from launch_opm_pack
  const float* bias;     // [c_z]
  const float* count;    // [batch][n][n]
  const bf16* res;       // [batch][n][n][c_z] or NULL
  bf16* out;             // [batch][n][n][c_z]
  int batch, n, sp, cz;
  float count_offset;
  int normalize_before_proj;
};
void launch_opm_contract(const OpmContractArgs& a, hipStream_t stream);
// Chai-1's grouped form: 8 groups of 8 channels a side, product norm, no count division.
struct OpmGroupedArgs {
  const bf16 *lt, *rt;               // [batch][n][64][sp]
  const bf16* wp;                    // [c_z][512] bf16 (to_out.weight rounded, same order)
  const float *bias, *norm_w, *norm_b;  // [c_z], [512], [512]
  const bf16* res;                   // [batch][n][n][c_z] or NULL
  bf16* out;                         // [batch][n][n][c_z]
  int batch, n, sp, cz;              // cz 128 or 256
  float norm_eps;
};
void launch_opm_contract_grouped(const OpmGroupedArgs& a, hipStream_t stream);

struct PackSeg {
  const float* src;  // NULL: write zeros
  bf16* dst;
  int64_t n;
  float scale;
  int swap23;        // 1: dst[i] = src[i with index bits 2 and 3 exchanged]
};
struct PackJob {
  PackSeg seg[8];
  int nseg;
  // optional: the key mask as fp32 rows maskf[b][s] = mask[b][s] ? 1 : 0 (s < n), 0 for
  // n <= s < np (mask NULL: none)
  const uint8_t* mask;
  float* maskf;
  // optional with the mask: kstages[b] = the number of 32-key stages up to the last real key
  // of batch element b (0 when it has none)
  int* kstages;
  int batch, n, np;
};
void launch_pack(const PackJob& job, hipStream_t stream);

// Compute units of the current device (cached per device).
int cu_count();

void launch_layer_norm(const void* x, const float* w, const float* b, void* y, int64_t rows,
                       int cols, float eps, int dtype, hipStream_t stream);

}  // namespace ffk
