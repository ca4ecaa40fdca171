/*
 * bmx.h -- C ABI of libbmx, the gfx950 (MI355X) kernels for Boltz-2's
 * pair-representation hot path.
 *
 * Every entry point:
 *   - takes device pointers owned by the caller (no allocation, no host sync);
 *   - launches asynchronously on `stream` (a hipStream_t; 0 = null stream);
 *   - returns 0 on success, BMX_EINVAL (1) for a rejected argument,
 *     BMX_EUNSUPPORTED (2) for an unsupported shape, BMX_ELAUNCH (3) when a
 *     launch failed; bmx_last_error() then describes the failure (per thread).
 * dtype codes: 0 = fp32, 1 = bf16.  Pair tensors are [n, n, 128] row-major
 * (one batch element), masks [n, n] fp32.  Weights passed as "bf16" are the
 * module's fp32 parameters rounded to bf16 by the caller.
 *
 * Citations name the reference (lauritsf/boltz-lumi) interface each entry
 * point replaces, relative to the reference repository root.
 */
#ifndef BMX_H
#define BMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* bmx_stream_t; /* hipStream_t */

/* Last error message of the calling thread ("" after a successful call), and the ABI version (2:
 * row_scale added to bmx_trimul_fwd / bmx_triattn_fwd).  No reference counterpart: the reference's
 * torch extensions report errors as Python exceptions (kernels/_build.py:9-34 builds them). */
const char* bmx_last_error(void);
int bmx_abi_version(void);

/* ---- Layer norm -------------------------------------------------------- */

/* LN over exactly 128 channels.  channel_first=0: x[rows][128];
 * channel_first=1: x[128][rows].  out is always [rows][128].
 * Replaces multiplication_norm (src/boltz_lumi/kernels/multiplication_hip.cu:149-156,
 * bound as `norm` in multiplication_hip.cpp) used by normalized_forward
 * (multiplication.py:81-90,117-126) and normalization_forward (triangle.py:107-146). */
int bmx_layernorm128(const void* x, int x_dtype, int channel_first, const float* weight, const float* bias, float eps,
                     void* out, int out_dtype, int64_t rows, bmx_stream_t stream);

/* General LN over dim <= 1024 (dim % 4 == 0) with optional weight/bias (NULL = none).
 * Serves AdaLN.a_norm / s_norm, which the reference leaves to torch (diffusion.py:55-56). */
int bmx_layernorm(const void* x, const float* weight, const float* bias, float eps, void* out, int dtype, int64_t rows,
                  int dim, bmx_stream_t stream);

/* out = sigmoid(scale) * LN_noaffine(a) + shift, one pass.
 * Replaces a_norm + the MODULATION epilogue of adaln_forward
 * (src/boltz_lumi/diffusion.py:52-57; kernels/diffusion_hip.cu:14-18,80-126). */
int bmx_adaln(const void* a, const void* scale, const void* shift, void* out, int dtype, int64_t rows, int dim,
              float eps, bmx_stream_t stream);

/* bmx_adaln with the scale / shift rows at stride ld_mod (ld_mod >= dim, multiple of 4): column
 * slices of one conditioning projection shared by the layers of a diffusion transformer
 * (adaln_forward, src/boltz_lumi/diffusion.py:52-57). */
int bmx_adaln_strided(const void* a, const void* scale, const void* shift, int64_t ld_mod, void* out, int dtype,
                      int64_t rows, int dim, float eps, bmx_stream_t stream);

/* ---- Elementwise operators (reference's unfused operator set) ---------- */

/* out = bf16(x * bf16(sigmoid(g))), bf16.
 * Replaces multiplication_gate (kernels/multiplication_gate_hip.cu:81-94, `gate`). */
int bmx_gate(const void* x, const void* g, void* out, int64_t n, bmx_stream_t stream);

/* a,b[pairs][128] = bf16(gate(p, g)) * mask from p,g rows of 256 channels at row_stride (256 or 512).
 * Replaces multiplication_gate_split (kernels/multiplication_gate_hip.cu:140-172, `split`). */
int bmx_trimul_split(const void* p, const void* g, const float* mask, void* a, void* b, int64_t pairs, int row_stride,
                     bmx_stream_t stream);

/* Channel-major bmm operands a,b[128][n][n] (outgoing: b transposed; incoming: a transposed).
 * p and g must be 16-byte aligned; a and b need bf16 alignment only (16-byte aligned operands
 * take 16-byte stores when n % 8 == 0).
 * Replaces multiplication_gate_pack (kernels/multiplication_gate_hip.cu:96-123, `pack`). */
int bmx_trimul_pack(const void* p, const void* g, const float* mask, void* a, void* b, int64_t n, int row_stride,
                    int outgoing, bmx_stream_t stream);

/* out = bf16(bf16(silu(a)) * b), bf16.
 * Replaces pair_silu_mul (kernels/pair_hip.cu:42-64, `silu_mul`). */
int bmx_silu_mul(const void* a, const void* b, void* out, int64_t n, bmx_stream_t stream);

/* kind 0 MODULATION: sigmoid(b)*a + c;  1 GATE: sigmoid(a)*b;
 * 3 GATED_SWIGLU: silu(a[:, cols:]) * a[:, :cols] * b  (a has 2*cols columns).
 * Replaces diffusion_epilogue (kernels/diffusion_hip.cu:80-126, `epilogue`; op codes diffusion.py:27). */
int bmx_diffusion_epilogue(int kind, const void* a, const void* b, const void* c, void* out, int dtype, int64_t rows,
                           int64_t cols, bmx_stream_t stream);

/* out = c + sigmoid(gate) * a (the MODULATION epilogue, fp32) with the gate rows at stride
 * ld_gate; out may alias c.  The output gate and residual add of a diffusion transformer
 * layer, a + sigmoid(output_projection_linear(s)) * b (transformersv2; diffusion.py:60-68). */
int bmx_gated_residual(const float* a, const float* gate, int64_t ld_gate, const float* c, float* out, int64_t rows,
                       int64_t cols, bmx_stream_t stream);

/* ---- Split-bf16 operands of the near-fp32 linears ---------------------
 * The diffusion blocks' fp32 linears (the reference leaves them to hipBLASLt in fp32:
 * diffusion.py:52-68, pair_bias.py:15-36; no reference counterpart) run as one bf16 GEMM
 * with fp32 accumulation of an operand row of kp = 3k + 64 bf16,
 *     [bf16(x) | bf16(x) | bf16(x - bf16(x)) | 1 1 0 ... 0],
 * against the weight row [Wh | Wl | Wh | bh bl 0 ... 0] (Wh = bf16(W), Wl = bf16(W - Wh),
 * likewise for the bias): x W + b up to about 2^-16 relative per product.  Operands are
 * written dense at row stride kp; inputs are fp32, 16-byte aligned; out 8-byte aligned. */

/* Operand rows of x (rows of k values at row stride ldx; k, ldx multiples of 4): the operand of
 * the linears above that take x itself (diffusion.py:52-68, pair_bias.py:15-36). */
int bmx_split3_bf16(const float* x, int64_t rows, int64_t k, int64_t ldx, void* out, bmx_stream_t stream);

/* Operand rows of LayerNorm-without-affine(x) (dim <= 1024, dim % 4 == 0): the s_norm input of
 * every AdaLN of a diffusion transformer, whose LayerNorm weight the caller folds into the
 * s_scale / s_bias weights (AdaLN.forward, transformersv2; diffusion.py:52-57). */
int bmx_layernorm_split3_bf16(const float* x, int64_t rows, int dim, int64_t ldx, float eps, void* out,
                              bmx_stream_t stream);

/* bmx_layernorm_split3_bf16 over the pairs of an n x n frame read transposed: operand row i n + j
 * is x row j n + i.  The ending-node triangle attention's fp32-mode projection operand
 * (reference triangle.py:38-52 runs TriangleAttentionEndingNode on x.transpose(-2, -3)), without a
 * transposed copy of x. */
int bmx_layernorm_split3_t_bf16(const float* x, int64_t n, int dim, int64_t ldx, float eps, void* out,
                                bmx_stream_t stream);

/* Operand rows of sigmoid(scale) * LN_noaffine(a) + shift (rounded as bmx_adaln), a dense
 * [rows][dim], scale / shift rows at stride ld_mod: the AdaLN output that feeds the
 * attention's q|k|v|g and the transition's swish_gate|a_to_b projections (diffusion.py:52-68). */
int bmx_adaln_split3_bf16(const float* a, const float* scale, const float* shift, int64_t ld_mod, int64_t rows,
                          int dim, float eps, void* out, bmx_stream_t stream);

/* Operand rows of silu(g) * x * b (rounded as the GATED_SWIGLU epilogue) where row r of u
 * holds [x | g | b] of cols values each at stride ldu: the conditioned transition's b from
 * one swish_gate|a_to_b projection, the input of b_to_a (diffusion.py:60-68). */
int bmx_swiglu_split3_bf16(const float* u, int64_t ldu, int64_t rows, int64_t cols, void* out, bmx_stream_t stream);

/* out = c + sigmoid(gate) * a (the MODULATION epilogue: a diffusion layer's gated residual
 * update; gate rows at stride ld_gate; out may alias c), then the operand rows of
 * sigmoid(scale) * LN_noaffine(out) + shift (scale / shift rows at stride ld_mod), as
 * bmx_gated_residual followed by bmx_adaln_split3_bf16 in one pass: the attention's residual
 * update and the conditioned transition's AdaLN (transformersv2 DiffusionTransformerLayer;
 * diffusion.py:52-68). */
int bmx_gated_residual_adaln_split3_bf16(const float* a, const float* gate, int64_t ld_gate, const float* c,
                                         float* out, const float* scale, const float* shift, int64_t ld_mod,
                                         int64_t rows, int dim, float eps, void* op, bmx_stream_t stream);

/* P = softmax(round(round(S + mask) + bias)) over the last axis, rounding to dtype.
 * shape = {B, I, H, Q, K}; element strides of scores [B,I,H,Q,K], bias [B,1,H,Q,K], mask [B,I,1,1,K].
 * out is contiguous.  Replaces ordered_softmax (kernels/triangle_softmax.py:117-161) and
 * triangle_block_softmax (kernels/triangle_block_softmax_hip.cu:120-143). */
int bmx_bias_softmax(const void* scores, const void* bias, const float* mask, void* out, int dtype,
                     const int64_t* shape, const int64_t* s_strides, const int64_t* b_strides,
                     const int64_t* m_strides, bmx_stream_t stream);

/* ---- Fused hot-path modules -------------------------------------------- */

/* out_mode for the fused modules: 0 = write bf16 [n,n,128], 1 = write fp32,
 * 2 = add into fp32 `out` (residual stream; out may alias x),
 * 3 = write fp32 out = x + y (out-of-place residual; out must not alias x).
 * row_scale (trimul / triattn): NULL, or fp32 [n]: the module output of frame row r is
 * multiplied by row_scale[r] before it is written or added.  The frame row is z's row for the
 * multiplications and the starting node, z's column for the ending node: PairformerLayer's
 * eval-mode dropout masks (upstream get_dropout_mask draws them even in eval, row-wise for
 * tri_mul_out / tri_mul_in / tri_att_start and column-wise for tri_att_end; the reference keeps
 * that composition, src/boltz_lumi/adapters.py:24-46 patches only the modules inside it).
 * stages (trimul / triattn): bitmask of the kernels to launch, 1 = projection,
 * 2 = contraction / attention core, 4 = output; 7 runs the whole module.  The
 * workspace carries the intermediates between separately launched stages. */

/* Workspace needed by bmx_trimul_fwd (bytes; 3 * 128 * np^2 bf16, np = round_up(n,256)).  Sizing
 * query: the reference's intermediates are torch allocations inside normalized_forward
 * (multiplication.py:48-137), which this caller-owned workspace replaces. */
size_t bmx_trimul_workspace_bytes(int64_t n);

/* TriangleMultiplication{Outgoing,Incoming}.forward for one batch element.
 * w_in: bf16 [512][128] = [p_in.weight; g_in.weight]; w_pout, w_gout: bf16 [128][128].
 * Replaces normalized_forward (src/boltz_lumi/multiplication.py:48-137) end to end. */
int bmx_trimul_fwd(const float* x, const float* mask, int64_t n, int outgoing, const float* norm_in_w,
                   const float* norm_in_b, float eps_in, const void* w_in, const float* norm_out_w,
                   const float* norm_out_b, float eps_out, const void* w_pout, const void* w_gout, void* out,
                   int out_mode, const float* row_scale, void* workspace, size_t workspace_bytes, int stages,
                   bmx_stream_t stream);

/* bmx_trimul_fwd (all three stages) with no workspace argument and no allocation: the operand
 * planes live in a static device array of the library (48 MiB = 3 planes of 128 x 256 x 256 bf16,
 * held on every GPU the library runs on until the process ends), so n must be <= 256; larger n is
 * rejected with BMX_EINVAL before any launch.  The first call on a device looks the array's device
 * address up (hipGetSymbolAddress), so make one call per device before capturing it into a HIP graph.
 * Calls that overlap on one GPU (other streams, other threads) share the array and race; serialise
 * them.  Nothing left in the array by an earlier call is read.
 * No counterpart in the reference: it serves callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int bmx_trimul_fwd_noalloc(const float* x, const float* mask, int64_t n, int outgoing, const float* norm_in_w,
                           const float* norm_in_b, float eps_in, const void* w_in, const float* norm_out_w,
                           const float* norm_out_b, float eps_out, const void* w_pout, const void* w_gout, void* out,
                           int out_mode, bmx_stream_t stream);

/* Workspace needed by bmx_triattn_fwd (bytes).  Sizing query: the reference's intermediates are
 * torch allocations inside triangle.py:32-104, which this caller-owned workspace replaces. */
size_t bmx_triattn_workspace_bytes(int64_t n);

/* Rows of the packed projection weight of bmx_triattn_fwd (416): upstream's q / k / v linears,
 * which the reference runs through _prep_qkv (triangle.py:80), with the triangle-bias linear's rows
 * appended and zero rows up to 416. */
int bmx_triattn_proj_rows(void);

/* TriangleAttention{,EndingNode}.forward (c_in 128, 4 heads x 32) for one batch element.
 * w_proj: bf16 [416][128] = [linear_q; linear_k; linear_v; linear (4 rows); zeros];
 * w_g, w_o: bf16 [128][128] with fp32 biases b_g, b_o.  mask may be NULL (all ones).
 * Replaces TriangleAttention.forward with the reference's patched layer_norm, _chunk and
 * mha.forward (src/boltz_lumi/triangle.py:18-22,32-104,107-146). */
int bmx_triattn_fwd(const void* x, int x_dtype, const float* mask, int64_t n, int starting, float inf,
                    const float* ln_w, const float* ln_b, float eps, const void* w_proj, const void* w_g,
                    const float* b_g, const void* w_o, const float* b_o, void* out, int out_mode,
                    const float* row_scale, void* workspace, size_t workspace_bytes, int stages, bmx_stream_t stream);

/* Pack a row-major bf16 matrix W[rows][cols] (rows % 32 == 0, cols % 16 == 0) into MFMA
 * A-operand order: element (r, c) goes to ((r/32 * cols/16 + c/16) * 64 + lane) * 8 + c%8
 * with lane = 32 * ((c%16)/8) + r%32, so each 32x16 operand tile is one contiguous 1 KB run.
 * dst holds rows * cols bf16 and must not overlap src.  Weight preparation for the
 * kernels that stream weights per tile (bmx_pair_transition_fwd); it replaces the reference's
 * cached bf16 weight concatenation (src/boltz_lumi/multiplication.py:29-45) for those. */
int bmx_pack_mfma_weights(const void* src, int64_t rows, int64_t cols, void* dst, bmx_stream_t stream);

/* Transition(128, 512).forward on `rows` rows of 128 channels.
 * w12: [fc1.weight; fc2.weight] (bf16 [1024][128]) and w3: fc3.weight (bf16 [128][512]),
 * each packed by bmx_pack_mfma_weights.
 * Replaces transition_forward (src/boltz_lumi/pair_transition.py:8-28). */
int bmx_pair_transition_fwd(const void* x, int x_dtype, int64_t rows, const float* ln_w, const float* ln_b, float eps,
                            const void* w12, const void* w3, void* out, int out_mode, bmx_stream_t stream);

/* Bytes of the folded pair-bias weights written by bmx_pair_bias_fold (8256); sizing query for
 * the fold of AttentionPairBias.proj_z (pair_bias.py:21-36). */
size_t bmx_pair_bias_fold_bytes(void);

/* Fold the sequence stack's pair-bias LayerNorm affine (ln_w, ln_b: [128]) and projection
 * w ([16][128]) into the operand order of bmx_pair_transition_bias_fwd: bf16 high and low parts
 * of W'[h][c] = ln_w[c] * w[h][c] and b[h] = sum_c ln_b[c] * w[h][c].  Weight preparation, once
 * per weight version, like bmx_pack_mfma_weights (AttentionPairBias.proj_z of pair_bias.py:21-36). */
int bmx_pair_bias_fold(const float* ln_w, const float* ln_b, const float* w, int heads, void* folded,
                       bmx_stream_t stream);

/* bmx_pair_transition_fwd (fp32 out_mode 1-3) followed, in the same pass, by the Pairformer
 * sequence stack's pair bias of the updated rows: pb_out[h][row] = sum_c LN(out[row])[c] * w[h][c]
 * (fp32 result, eps pb_eps, 16 heads, pb_out [16][rows]), i.e. bmx_pair_bias_fwd on `out`
 * without reading it back; pb_folded is bmx_pair_bias_fold's output.  The composition upstream
 * PairformerLayer runs (transition_z, then AttentionPairBias.proj_z on the new z;
 * pair_transition.py:8-28 and pair_bias.py:21-36). */
int bmx_pair_transition_bias_fwd(const void* x, int x_dtype, int64_t rows, const float* ln_w, const float* ln_b,
                                 float eps, const void* w12, const void* w3, void* out, int out_mode,
                                 const void* pb_folded, float pb_eps, float* pb_out, bmx_stream_t stream);

/* ---- Sequence-stack pair bias (next to the hot path) ------------------- */

/* bias[h][row] = sum_c LN(z[row])[c] * w[h][c] for heads = 16, fp32 math; out is
 * [16][rows] fp32 (the [B,H,N,N] attention bias for one batch element).
 * Replaces AttentionPairBias.proj_z = LayerNorm + Linear(128, 16) + Rearrange of the
 * Pairformer sequence stack, which the reference leaves to torch (adapters.py:39-45;
 * math restated at src/boltz_lumi/pair_bias.py:21-36). */
int bmx_pair_bias_fwd(const void* z, int z_dtype, int64_t rows, const float* ln_w, const float* ln_b, float eps,
                      const float* w, int heads, float* out, bmx_stream_t stream);

/* out[i][h*D+d] = sigmoid(g[i][h*D+d]) * sum_j softmax_j(q_i.k_j / sqrt(D) + bias[h][i][j]
 *                                                      + (1 - mask[j]) * -inf) v_j[d],  fp32,
 * for head_dim D = 24 (Pairformer sequence stack, 16 x 24) or 48 (diffusion token transformer,
 * 16 x 48) and 1 <= heads <= 64.  q, k, v and the gate logits g are [n] rows of heads * D values
 * at row stride ld (>= heads * D; e.g. column slices of one fused [n, 4 * heads * D] projection),
 * bias is [heads][n][n], mask [n], out [n][heads * D] contiguous.
 * Replaces the logits / softmax / PV / gate part of AttentionPairBias.forward (math as
 * src/boltz_lumi/pair_bias.py:21-36): the trunk's sequence stack, which the reference leaves to
 * torch (adapters.py:39-45), and the token transformer's prepared_forward (pair_bias.py:15-36,
 * installed at adapters.py:39-42); the [heads, n, n] logits never reach HBM. */
int bmx_seq_attention_fwd(const float* q, const float* k, const float* v, const float* bias, const float* mask,
                          const float* g, int64_t n, int64_t ld, int heads, int head_dim, float inf, float* out,
                          bmx_stream_t stream);

/* bmx_seq_attention_fwd over a batch of elements in one launch, with separate query and key
 * counts (attention to other keys, as the atom transformer's windows: AttentionPairBias.forward
 * with k_in != s) and head_dim D = 24, 32 or 48.  Element b: q, g [nq][heads * D] at row stride
 * ldq, element stride sq; k, v [nk][heads * D] at ldk, sk; bias element b / bias_div ([heads][nq][nk]
 * dense, element stride sbias; upstream repeat_interleave(multiplicity)); mask element b ([nk],
 * stride smask, 0 to share one); out [batch][nq][heads * D] contiguous.  Replaces the same part of
 * AttentionPairBias.forward (math as src/boltz_lumi/pair_bias.py:21-36). */
int bmx_seq_attention_batched_fwd(const float* q, const float* k, const float* v, const float* bias, const float* mask,
                                  const float* g, int64_t batch, int64_t nq, int64_t nk, int64_t ldq, int64_t ldk,
                                  int64_t sq, int64_t sk, int64_t sbias, int64_t smask, int64_t bias_div, int heads,
                                  int head_dim, float inf, float* out, bmx_stream_t stream);

/* bmx_seq_attention_batched_fwd for the atom transformer's windows, with upstream's to_keys gather
 * (single_to_keys through its indexing matrix, then AttentionPairBias with k_in = to_keys(s)) done by
 * addressing: element b (window b % windows of sample b / windows) has its nq query rows at rows
 * b * nq .. of q, g (row stride ldq) and reads key j from row b * nq + key_offset + j of k, v (row
 * stride ldk; k, v projected on the atom rows, batch * nq rows) and mask ([batch * nq], the atom
 * mask), present only while 0 <= (b % windows) * nq + key_offset + j < windows * nq; an absent key
 * is a zero key / value row with mask 0, as the zero rows single_to_keys writes.  Element b reads
 * the bias of window b % windows of structure b / bias_group (upstream repeat_interleave of the
 * per-structure window bias over the samples: bias_group = samples * windows) at structure /
 * window / head / query / key strides sbias_group, sbias, sbias_h, sbias_q (>= 1), sbias_k (any
 * layout, e.g. one layer's heads of the [B, windows, nq, nk, layers * heads] atom bias in place or
 * stored channel-major).  out [batch][nq][heads * D]
 * contiguous.  Replaces AttentionPairBias.forward's attention with upstream's to_keys
 * (pair_bias.py:21-36; the keys that transformersv2.AtomTransformer gathers). */
int bmx_seq_attention_windowed_fwd(const float* q, const float* k, const float* v, const float* bias,
                                   const float* mask, const float* g, int64_t batch, int64_t nq, int64_t nk,
                                   int64_t ldq, int64_t ldk, int64_t windows, int64_t key_offset,
                                   int64_t bias_group, int64_t sbias_group, int64_t sbias, int64_t sbias_h,
                                   int64_t sbias_q, int64_t sbias_k, int heads, int head_dim, float inf, float* out,
                                   bmx_stream_t stream);

/* bmx_seq_attention_batched_fwd with both products on bf16 MFMA, each operand split into bf16 high
 * and low parts (x y ~ xh yh + xh yl + xl yh: about 2^-16 relative per product, the same form as the
 * split-bf16 fp32 linears of the diffusion blocks) instead of fp32 MFMA; same arguments and result,
 * within 1e-4 of the fp32 reference.  A pre-pass writes the split K and the split, transposed V into
 * `workspace` (256-byte aligned, bmx_seq_attention_x3_workspace_bytes bytes).  Replaces the same
 * part of AttentionPairBias.forward (math as src/boltz_lumi/pair_bias.py:21-36); the reference runs
 * these products as fp32 matmuls. */
size_t bmx_seq_attention_x3_workspace_bytes(int64_t batch, int64_t nk, int heads, int head_dim);
int bmx_seq_attention_x3_batched_fwd(const float* q, const float* k, const float* v, const float* bias,
                                     const float* mask, const float* g, int64_t batch, int64_t nq, int64_t nk,
                                     int64_t ldq, int64_t ldk, int64_t sq, int64_t sk, int64_t sbias, int64_t smask,
                                     int64_t bias_div, int heads, int head_dim, float inf, float* out,
                                     void* workspace, size_t workspace_bytes, bmx_stream_t stream);

/* bmx_seq_attention_x3_batched_fwd writing each output row as the split-bf16 operand of the next
 * linear (proj_o): out_op [batch * nq][3 * heads * D + 64] bf16, rows [hi | hi | lo | 1 1 0 ...]
 * as bmx_split3_bf16 writes them (16-byte aligned).  Saves the fp32 output and its split pass.
 * Replaces the same part of AttentionPairBias.forward as bmx_seq_attention_x3_batched_fwd
 * (pair_bias.py:21-36) together with proj_o's input. */
int bmx_seq_attention_x3_batched_split_fwd(const float* q, const float* k, const float* v, const float* bias,
                                           const float* mask, const float* g, int64_t batch, int64_t nq, int64_t nk,
                                           int64_t ldq, int64_t ldk, int64_t sq, int64_t sk, int64_t sbias,
                                           int64_t smask, int64_t bias_div, int heads, int head_dim, float inf,
                                           void* out_op, void* workspace, size_t workspace_bytes,
                                           bmx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BMX_H */
