/*
 * foldforge_amd: C-ABI of the MI355X (gfx950) Pairformer pair-stack kernels.
 *
 * Plain pointers and sizes only. Every tensor argument is a device pointer on the
 * current HIP device; `stream` is a hipStream_t (NULL = the default stream). All
 * entry points are asynchronous on `stream`, allocate nothing, keep no state between
 * calls (no weight caches), never throw, and return an FFK_* status; the text of the
 * last failure on the calling thread is ffk_last_error().
 *
 * Layouts (engine layout of the reference, src/foldforge/modules/engine/graph.py:191-235):
 *   pair z      [batch, n, n, d_pair] bf16, channel-last, contiguous
 *   key mask    [batch, n] uint8 (torch.bool), 1 = real token
 *   parameters  fp32, the engine module's own tensors (state_dict layout), contiguous
 * Outputs are caller-allocated; `out` may alias the pair input (each output tile reads
 * its own input before writing it). Entry points with a workspace take a caller-
 * allocated device buffer of at least the matching *_workspace() bytes, 256-byte
 * aligned. "residual" = 1 returns x + f(x) (the engine's residual-owning forward),
 * 0 returns the bare update f(x) (the engine's `.delta`).
 */
#ifndef FOLDFORGE_AMD_H
#define FOLDFORGE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FFK_OK 0
#define FFK_ERR_INVALID 1   /* an argument is outside the kernels' range */
#define FFK_ERR_WORKSPACE 2 /* workspace missing or too small */
#define FFK_ERR_HIP 3       /* HIP runtime error (device query, launch) */
#define FFK_ERR_DEVICE 4    /* the current device is not a gfx950 (MI355X) */

#define FFK_DTYPE_BF16 0
#define FFK_DTYPE_F32 1

#define FFK_ACT_NONE 0    /* y = t */
#define FFK_ACT_SIGMOID 1 /* y = 1 / (1 + exp(-t)) */
#define FFK_ACT_SILU 2    /* y = t / (1 + exp(-t)) */
#define FFK_ACT_RELU 3    /* y = max(t, 0) */

/* Library version (major * 10000 + minor * 100 + patch). */
int32_t ffk_version(void);

/* Text of the last non-zero status returned on this thread ("" if none). */
const char* ffk_last_error(void);

/* 1 when HIP device `device` is a gfx950 the kernels were built for, else 0. */
int32_t ffk_device_supported(int32_t device);

/*
 * LayerNorm over the last axis: y = (x - mean) / sqrt(var + eps) * weight + bias,
 * fp32 statistics and fp32 affine, input dtype kept (bf16 or fp32).
 * Replaces: the engine LayerNorm module and `miniworld_engine.kernels.layer_norm`
 * (src/foldforge/modules/engine/modules.py:230-238; kernel name in
 * docs/guides/ENGINE-2.4.2.md:18-21). weight/bias may be NULL (no affine / no offset).
 */
int32_t ffk_layer_norm(const void* x, const float* weight, const float* bias, void* y,
                       int64_t rows, int32_t cols, float eps, int32_t dtype, void* stream);

/*
 * LayerNorm fused into a linear projection, with a bias and an activation epilogue:
 *   y[r, :] = act(LN(x[r, :]) W^T + bias)
 * x [rows, d_in] bf16; LN with fp32 statistics, ln_w / ln_b fp32 [d_in] (either may be NULL:
 * weight 1, offset 0); weight fp32 [d_out, d_in] (the engine Linear's own tensor, rounded to
 * bf16 for the matrix cores; the normalised rows keep fp32 precision as a bf16 hi + lo pair);
 * bias fp32 [d_out] or NULL; y [rows, d_out] in out_dtype (FFK_DTYPE_BF16 or FFK_DTYPE_F32);
 * activation one of FFK_ACT_*. d_in a multiple of 64 up to 768, d_out a multiple of 32.
 * Replaces: `miniworld_engine.kernels.layernorm_linear.interface.layer_norm_linear`
 * (docs/guides/ENGINE-2.4.2.md:21; the reference holds no signature for it). The pair ops
 * below fuse this prologue into their own projection kernels.
 */
int32_t ffk_layer_norm_linear(const void* x, const float* ln_w, const float* ln_b,
                              const float* weight, const float* bias, void* y, int64_t rows,
                              int32_t d_in, int32_t d_out, int32_t activation, int32_t out_dtype,
                              float eps, void* stream);

/*
 * SwiGLU feed-forward on token rows, no normalisation:
 *   out[r, :] = residual[r, :] + (silu(x[r, :] w_a^T) * (x[r, :] w_b^T)) w_out^T
 * (residual NULL: the bare update). x, residual, out [rows, d] bf16 (out may alias x or the
 * residual); w_a, w_b fp32 [hidden, d], w_out fp32 [d, hidden]; the hidden rows stay fp32 in
 * the workspace (ffk_swiglu_ffn_workspace bytes). d a multiple of 64 up to 768, hidden a
 * multiple of 64. The transition is x + swiglu_ffn(LN(x)).
 * Replaces: `miniworld_engine.kernels.swiglu_ffn` (docs/guides/ENGINE-2.4.2.md:18; no
 * signature in the reference).
 */
size_t ffk_swiglu_ffn_workspace(int64_t rows, int32_t hidden);
int32_t ffk_swiglu_ffn(const void* x, const float* w_a, const float* w_b, const float* w_out,
                       const void* residual, void* out, void* workspace, size_t workspace_bytes,
                       int64_t rows, int32_t d, int32_t hidden, void* stream);

/*
 * Triangle multiplicative update, outgoing (outgoing = 1) or incoming (0), including
 * the LayerNorm + gated projections prologue and the centre norm + output projection +
 * output gate epilogue. d_pair = d_hidden = 128 runs the fused kernels; other widths (d_pair
 * a multiple of 64 up to 256, d_hidden a multiple of 64 up to 768: the template stack's)
 * run the generic path with a larger workspace. length_divided = 1 is RoseTTAFold3's exact
 * form: the contraction divided by the real length L (positions real in any batch element,
 * counted on the device from key_mask) before the centre norm.
 * Replaces: engine TriangleMultiplication.forward / `triangle_multiplicative_update`
 * (equations src/foldforge/models/checkpoints/legacy/reference/triangle.py:19-49,
 * engine parameters legacy/released.py:135-173; op name "trimul",
 * src/foldforge/modules/engine/backends.py:36-40) and, with length_divided,
 * TriangleMultiplicationRF3 (legacy/routing.py:33-55).
 */
size_t ffk_triangle_multiplication_workspace(int64_t batch, int64_t n, int32_t d_pair,
                                             int32_t d_hidden);
int32_t ffk_triangle_multiplication(
    const void* z, const uint8_t* key_mask, const float* ln_pair_w, const float* ln_pair_b,
    const float* w_left, const float* w_right, const float* w_left_gate,
    const float* w_right_gate, const float* ln_out_w, const float* ln_out_b,
    const float* w_out, const float* w_gate, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t n, int32_t d_pair, int32_t d_hidden,
    int32_t outgoing, int32_t residual, int32_t length_divided, float eps, void* stream);

/*
 * Triangle attention around the starting (starting = 1) or ending (0) node: LayerNorm,
 * pair bias, q/k/v/gate projections, flash attention with key mask, gate, output
 * projection. d_pair = 128 with 4 heads x 32 runs the fused kernels; d_pair 64 / 128 / 256
 * with at most 32 heads of 8 to 64 channels (n_head * d_head a multiple of 64, batch * n at
 * most 65535) runs the generic path. transposed_bias = 1 takes the ending node's bias from
 * the transposed pair (OpenFold lineage). b_gate [n_head * d_head] and b_out [d_pair] are the
 * gate / output projection biases (RoseTTAFold3; NULL: none). output_form: 0 the z-frame
 * update (AF3 and its descendants); 1 the ending node's update left in the attention's
 * orientation (Chai-1's trunk; the starting node is unchanged); 2 the update plus the
 * transpose over the pair axes of a second projection w_out_t [d_pair, n_head * d_head]
 * (+ b_out_t) of the same gated values (Chai-1's confidence head; w_out_t is required by, and
 * only by, this form). The workspace depends on the form: forms 1 and 2 add a staging buffer
 * of batch * n * n * d_pair bf16; a starting-node call of form 1 is the standard form and
 * never touches that buffer, so a caller may pass output_form 0 for it (and size the
 * workspace for form 0).
 * Replaces: engine TriangleAttention(AF3 / OpenFold / RF3 / Chai1 / Chai1Confidence).forward
 * / `triangle_attention` (src/foldforge/models/checkpoints/legacy/attention.py:60-171,
 * legacy/reference/attention.py:77-100; forms src/foldforge/modules/dense/spec.py:116-125,
 * 437, 463-478; engine parameters legacy/released.py:176-208; op name "triangle_attention",
 * src/foldforge/modules/engine/backends.py:41-47).
 */
size_t ffk_triangle_attention_workspace(int64_t batch, int64_t n, int32_t d_pair,
                                        int32_t n_head, int32_t d_head, int32_t output_form);
int32_t ffk_triangle_attention(
    const void* z, const uint8_t* key_mask, const float* ln_pair_w, const float* ln_pair_b,
    const float* w_bias, const float* w_query, const float* w_key, const float* w_value,
    const float* w_gate, const float* w_out, const float* b_gate, const float* b_out,
    const float* w_out_t, const float* b_out_t, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t n, int32_t d_pair, int32_t n_head,
    int32_t d_head, int32_t starting, int32_t transposed_bias, int32_t output_form,
    int32_t residual, float eps, void* stream);

/*
 * The ending (or starting) node's triangle attention followed by the pair transition, the
 * two last pair updates of a Pairformer block in the sequential order:
 *   y   = z + (sigmoid(LN_pair(z) w_gate^T) * attention(z)) w_out^T     (y rounded to bf16)
 *   out = y + w_squeeze (silu(w_expand_a LN_in(y)) * w_expand_b LN_in(y))
 * with the attention's output projection computed inside the transition kernel, so y never
 * reaches HBM; the result equals ffk_triangle_attention (output_form 0, residual 1) followed
 * by ffk_transition (residual 1). Widths fixed at the AF3 trunk's: d_pair 128, 4 heads x 32,
 * transition 128 x 4; no gate / output biases (the RoseTTAFold3 lineage runs the two entry
 * points). out may alias z. Arguments as the two entry points'; eps_pair / eps_in are the
 * two LayerNorms' epsilons.
 * Replaces: the block's last two pair updates, the ending node's attention residual then the
 * transition residual (src/foldforge/models/checkpoints/legacy/pairformer.py:200-202; the
 * engine block, src/foldforge/modules/engine/graph.py:191-235, runs them as the ops
 * tri_atten_ending and transition_pair), each op as ffk_triangle_attention and ffk_transition
 * replace it.
 */
size_t ffk_triangle_attention_transition_workspace(int64_t batch, int64_t n);
int32_t ffk_triangle_attention_transition(
    const void* z, const uint8_t* key_mask, const float* ln_pair_w, const float* ln_pair_b,
    const float* w_bias, const float* w_query, const float* w_key, const float* w_value,
    const float* w_gate, const float* w_out, const float* ln_in_w, const float* ln_in_b,
    const float* w_expand_a, const float* w_expand_b, const float* w_squeeze, void* out,
    void* workspace, size_t workspace_bytes, int64_t batch, int64_t n, int32_t starting,
    int32_t transposed_bias, float eps_pair, float eps_in, void* stream);

/*
 * Flash attention core with an additive pair bias, the building block of triangle
 * attention:
 *   o[b, r, j, h*32 + :] = sum_k softmax_k(q[b,h,r,j,:] . k[b,h,r,k,:] + bias[b,h,j,k]) v[b,h,r,k,:]
 * in the base-2 domain: q must already carry the softmax scale times log2(e); bias is
 * fp32 in log2 units with -inf at masked keys, in the blocked layout
 *   bias_blk[b*heads + h][j / 32][k / 32][v][32 g + j % 32][e],  k % 32 = 8 v + 4 g + e
 * (v in 0..3, g in 0..1, e in 0..3): the register order of the kernel's 32 x 32 logit tiles.
 * Shapes: q, k [batch * heads, rows, n_pad, 32] bf16; v_t [batch * heads, rows, n_pad / 32,
 * 32, 32] bf16 (v transposed and blocked by 32 keys: block kb holds [d][32 keys], the keys of
 * every group of 16 stored in the order 0-3, 8-11, 4-7, 12-15); output bf16 written at
 * o + b*o_sb + r*o_sr + j*o_sj + h*32 + d for
 * r < rows_valid, j < n_valid (o and its strides 16-byte aligned). n_pad must be a multiple
 * of 128 and rows of 4. A query
 * whose keys are all masked gets a zero output. Replaces the engine's triangle-attention
 * kernel (docs/engine-kernel-gaps.md:10-23 names its sm90 source); no reference C signature.
 */
int32_t ffk_flash_attention_bias(const void* q, const void* k, const void* v_t,
                                 const void* bias, void* o, int64_t batch, int32_t heads,
                                 int64_t rows, int64_t n_pad, int64_t rows_valid,
                                 int64_t n_valid, int64_t o_sb, int64_t o_sr, int64_t o_sj,
                                 void* stream);

/*
 * Pair (or single) transition: x + squeeze(silu(expand_a(LN(x))) * expand_b(LN(x))) over
 * `rows` token rows of width d. d = 128, factor = 4 runs one fused kernel (the 4x hidden
 * never reaches HBM); other widths (d and factor * d multiples of 64, e.g. the single
 * track's 384 x 4) run LayerNorm -> expand with SwiGLU epilogue -> squeeze + residual,
 * keeping the hidden rows in the workspace.
 * Replaces: engine Transition.forward / `transition`
 * (src/foldforge/models/checkpoints/legacy/reference/transition.py:28-59,
 * engine parameters legacy/released.py:211-224; op name "transition",
 * src/foldforge/modules/engine/backends.py:51).
 */
size_t ffk_transition_workspace(int64_t rows, int32_t d, int32_t factor);
int32_t ffk_transition(const void* x, const float* ln_w, const float* ln_b,
                       const float* w_expand_a, const float* w_expand_b,
                       const float* w_squeeze, void* out, void* workspace,
                       size_t workspace_bytes, int64_t rows, int32_t d, int32_t factor,
                       int32_t residual, float eps, void* stream);

/*
 * ffk_transition without a workspace argument and without any device allocation: the
 * scratch (packed weights, or the hidden rows of the other widths) lives in a static
 * 4 MiB device array of the library, one per device, held until the process ends. Same
 * arguments, kernels and results as ffk_transition. Calls whose scratch would exceed 4 MiB
 * return FFK_ERR_WORKSPACE: d = 128 x 4 always fits (384 KiB of packed weights); other widths
 * fit while rows * factor * d * 4 bytes <= 4 MiB (e.g. the single track's 384 x 4 up to 682
 * rows). Calls on one device share the array: calls that overlap in time on one device race.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * graph capture, fixed serving loops, harnesses that forbid hipMalloc).
 */
int32_t ffk_transition_noalloc(const void* x, const float* ln_w, const float* ln_b,
                               const float* w_expand_a, const float* w_expand_b,
                               const float* w_squeeze, void* out, int64_t rows, int32_t d,
                               int32_t factor, int32_t residual, float eps, void* stream);

/*
 * Single-track attention with pair bias, residual included:
 *   x = LN_single(s); bias[h, i, j] = LN_pair(z[i, j]) . w_bias[h]  (pair norm without offset)
 *   o_h = softmax_j((x w_query^T + b_query)_h . (x w_key^T)_h / sqrt(dh) + bias[h]) (x w_value^T)_h
 *   out = s + (sigmoid(x w_gate^T + gate_bias) * o) w_out^T
 * with the [batch, n] key mask (masked keys weigh exactly 0; a batch entry without a valid
 * key gets o = 0). s, out [batch, n, d_single] bf16; z [batch, n, n, d_pair] bf16;
 * d_pair = 128; d_single a multiple of 64 split into n_head <= 32 heads of dh = 8, 16, 24
 * or 32 (the trunk: 384 = 16 x 24). `out` may alias `s`. extra_bias (NULL: none) adds
 * extra_bias[b * stride_b + h * stride_h + i * stride_i + j] (fp32, or bf16 with extra_bf16;
 * strides in elements, 0 broadcasts) to the logit of (head h, query i, key j): the block's
 * extra_pair_bias (OpenDDE's structural bias, legacy/pairformer.py:216-218; the engine
 * expands [n, n] over samples and heads, src/foldforge/modules/engine/graph.py:223-225).
 * Replaces: engine AttentionPairBias.forward, op name "single_attention"
 * (src/foldforge/modules/engine/backends.py:50; equations
 * src/foldforge/models/checkpoints/legacy/transformer.py:28-137 as called from
 * legacy/pairformer.py:211-226; engine parameters legacy/released.py:281-315).
 */
size_t ffk_attention_pair_bias_workspace(int64_t batch, int64_t n, int32_t d_single,
                                         int32_t d_pair, int32_t n_head);
int32_t ffk_attention_pair_bias(
    const void* s, const void* z, const uint8_t* key_mask, const float* ln_single_w,
    const float* ln_single_b, const float* w_query, const float* b_query, const float* w_key,
    const float* w_value, const float* ln_pair_w, const float* w_bias, const float* w_gate,
    const float* w_out, const void* extra_bias, int32_t extra_bf16, int64_t extra_stride_b,
    int64_t extra_stride_h, int64_t extra_stride_i, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t n, int32_t d_single, int32_t d_pair,
    int32_t n_head, float gate_bias, int32_t residual, float eps_single, float eps_pair,
    void* stream);

/*
 * MSA pair-weighted averaging, residual included:
 *   x = LN_msa(m); w[h, i, :] = softmax_j(LN_pair(z)[i, j] . w_bias[h]) over valid keys j
 *   (pair norm without offset; the same weights for every MSA row);
 *   o[s, i, h] = sum_j w[h, i, j] (x w_value^T)[s, j, h];
 *   out = m + (sigmoid(x w_gate^T) * o) w_out^T.
 * m, out [batch, depth, n, d_msa] bf16 (depth = MSA rows); z [batch, n, n, d_pair] bf16;
 * key_mask [batch, n] (a column is a key when any MSA row has it); a batch element without a
 * valid key gets a zero update. d_pair = 128; d_msa a multiple of 64 up to 768; at most 32
 * heads of d_head (a multiple of 4), n_head * d_head a multiple of 64 up to 768 (AF3: 8 x 8).
 * `out` may alias `m`.
 * Replaces: engine MSAPairWeightedAveraging.forward, op name "msa_pwa"
 * (src/foldforge/modules/engine/backends.py:49; equations
 * src/foldforge/models/checkpoints/legacy/attention.py:174-229; engine parameters
 * legacy/released.py:253-278; called as graph.py:302).
 */
size_t ffk_msa_pair_weighted_averaging_workspace(int64_t batch, int64_t depth, int64_t n,
                                                  int32_t d_msa, int32_t d_pair, int32_t n_head,
                                                  int32_t d_head);
int32_t ffk_msa_pair_weighted_averaging(
    const void* m, const void* z, const uint8_t* key_mask, const float* ln_msa_w,
    const float* ln_msa_b, const float* ln_pair_w, const float* w_bias, const float* w_value,
    const float* w_gate, const float* w_out, void* out, void* workspace, size_t workspace_bytes,
    int64_t batch, int64_t depth, int64_t n, int32_t d_msa, int32_t d_pair, int32_t n_head,
    int32_t d_head, int32_t residual, float eps_msa, float eps_pair, void* stream);

/* Outer product mean (the MSA-to-pair update), raw or added to a residual.
 * m [batch][depth][n][d_msa] bf16, rows_mask [batch][depth][n] (0 / 1 bytes: which MSA
 * entries are real), residual (NULL, or [batch][n][n][d_pair] bf16; may alias out),
 * out [batch][n][n][d_pair] bf16:
 *   l = mask (LN(m) W_left^T + b_left), r = mask (LN(m) W_right^T + b_right)  (d_hidden each)
 *   o[i][j] = sum_s l[s][i] (x) r[s][j]  (flattened left-channel-major: c * d_hidden + e)
 *   count[i][j] = sum_s mask[s][i] mask[s][j]
 *   d = count + count_offset (count_offset >= 0: AF3's n + 1e-3) or max(count, 1) (< 0)
 *   out = residual + ((o W_out^T + b_out) / d)        normalize_before_proj = 0
 *   out = residual + ((o / d) W_out^T + b_out)        normalize_before_proj = 1
 * Weights fp32: w_left / w_right [d_hidden][d_msa], b_left / b_right [d_hidden] or NULL,
 * w_out [d_pair][d_hidden^2], b_out [d_pair]. Served: d_hidden 32, d_pair 128, d_msa a
 * multiple of 64 up to 768, depth >= 1; anything else returns FFK_ERR_INVALID.
 * Replaces: engine OuterProductMean.forward, op name "opm"
 * (src/foldforge/modules/engine/backends.py:48; factory modules.py:184-210; equations
 * src/foldforge/models/checkpoints/legacy/primitives.py:40-136 and
 * legacy/reference/attention.py:57-74; engine parameters legacy/released.py:227-251; called as
 * graph.py:303).
 */
size_t ffk_outer_product_mean_workspace(int64_t batch, int64_t depth, int64_t n, int32_t d_msa,
                                        int32_t d_hidden, int32_t d_pair);
int32_t ffk_outer_product_mean(
    const void* m, const uint8_t* rows_mask, const float* ln_w, const float* ln_b,
    const float* w_left, const float* b_left, const float* w_right, const float* b_right,
    const float* w_out, const float* b_out, const void* residual, void* out, void* workspace,
    size_t workspace_bytes, int64_t batch, int64_t depth, int64_t n, int32_t d_msa,
    int32_t d_hidden, int32_t d_pair, float eps, float count_offset,
    int32_t normalize_before_proj, void* stream);

/* Chai-1's grouped outer product mean: d_hidden = groups * d_group channels a side, products
 * only within each group and summed over the MSA rows (no count division),
 *   p[b, i, j, (g, k, l)] = sum_s l[b, s, i, g d_group + k] r[b, s, j, g d_group + l],
 *   out = LN_{norm_eps}(p) W_out^T + b_out (+ residual),
 * with l, r as in ffk_outer_product_mean. Weights fp32: w_left / w_right [d_hidden][d_msa],
 * b_left / b_right [d_hidden] or NULL, norm_w / norm_b [groups d_group^2] (the product norm),
 * w_out [d_pair][groups d_group^2] in the (g, k, l) order, b_out [d_pair]. Served: 8 groups of
 * 8, d_pair 128 or 256, d_msa a multiple of 64 up to 768; anything else returns
 * FFK_ERR_INVALID. out may not alias m; residual may be out.
 * Replaces: engine OuterProductMean.forward with groups > 1, op name "opm"
 * (src/foldforge/modules/engine/backends.py:48; factory modules.py:184-210 with graph.py:252-264;
 * equations src/foldforge/models/checkpoints/legacy/primitives.py:62-79,122-136; Chai-1's
 * widths src/foldforge/modules/dense/spec.py:687-688).
 */
size_t ffk_outer_product_mean_grouped_workspace(int64_t batch, int64_t depth, int64_t n,
                                                int32_t d_msa, int32_t groups, int32_t d_group,
                                                int32_t d_pair);
int32_t ffk_outer_product_mean_grouped(
    const void* m, const uint8_t* rows_mask, const float* ln_w, const float* ln_b,
    const float* w_left, const float* b_left, const float* w_right, const float* b_right,
    const float* norm_w, const float* norm_b, const float* w_out, const float* b_out,
    const void* residual, void* out, void* workspace, size_t workspace_bytes, int64_t batch,
    int64_t depth, int64_t n, int32_t d_msa, int32_t groups, int32_t d_group, int32_t d_pair,
    float eps, float norm_eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FOLDFORGE_AMD_H */
