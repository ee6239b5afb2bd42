/*
 * xfold_hip.h -- C ABI of libxfold_hip.so, the MI355X (gfx950) backend for xfold's
 * Pairformer and diffusion-transformer hot operators.
 *
 * Conventions (every entry point):
 *   - Pointers are device pointers unless stated; the caller owns every buffer, including
 *     outputs and workspaces (query sizes with the *_workspace_size functions). The
 *     library never allocates device memory.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t passed as void*; NULL is
 *     the default stream). No entry point synchronises the host.
 *   - Return value: XFH_OK or an error code; xfh_last_error() then holds a message for the
 *     calling host thread. Nothing throws across this boundary.
 *   - Weights follow torch.nn.Linear's layout [out_features, in_features], row-major, in
 *     the compute dtype. LayerNorm parameters are fp32 (NULL = absent).
 *   - dtype codes: XFH_F32, XFH_BF16; masks may also be XFH_BOOL (1 byte, nonzero = keep).
 *
 * Each declaration names the reference interface it replaces (paths in the reference
 * repository Zhengye-AIsys/xfold_cpu).
 */
#ifndef XFOLD_HIP_H
#define XFOLD_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XFH_ABI_VERSION 9

enum { XFH_F32 = 0, XFH_BF16 = 1, XFH_BOOL = 2 };
enum { XFH_OK = 0, XFH_EINVAL = 1, XFH_EUNSUPPORTED = 2, XFH_EWORKSPACE = 3, XFH_EHIP = 4 };

/* Bias "dtype" of xfh_dot_product_attention for a packed bias block [H][Q][align64(K)]:
 * fp32 times log2(e) (xfh_attention_bias_pack, xfh_pair_attention_bias with out_dtype
 * XFH_F32), or bf16 in natural units (xfh_pair_attention_bias with out_dtype XFH_BF16). */
#define XFH_BIAS_PACKED 3
#define XFH_BIAS_PACKED_BF16 4

/* GEMM epilogues of xfh_linear: acc = x @ w^T + bias, a = aux[row % aux_rows, col]. */
enum {
  XFH_EPI_STORE = 0,                 /* y  = acc                     */
  XFH_EPI_MUL_SIGMOID_AUX = 1,       /* y  = acc * sigmoid(a)        */
  XFH_EPI_SIGMOID_MUL_AUX = 2,       /* y  = sigmoid(acc) * a        */
  XFH_EPI_ACCUMULATE = 3,            /* y += acc                     */
  XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE = 4 /* y += acc * sigmoid(a)    */
};

/* ABI marker; replaces the `packed_weight_api` attribute
 * (af3_kernels/src/csrc/bindings.cpp:12). */
int xfh_abi_version(void);

/* Static description of the build (target, HIP version, kernels); replaces
 * `runtime_info()` (af3_kernels/src/csrc/bindings.cpp:13-20). */
const char *xfh_runtime_info(void);

/* Message of the last failed call on this host thread ("" if none). Replaces the
 * TORCH_CHECK -> RuntimeError path of the pybind11 module (af3_kernels/src/csrc/tools.cpp:20-28). */
const char *xfh_last_error(void);

/* Opt-in timing of the library's dominant kernels (no reference counterpart; used by the
 * benchmark): while enabled, launches of the named kernels ("grid_attention", ...) are
 * bracketed by HIP events on their stream. xfh_kernel_timing_read waits for, sums and
 * releases the recorded intervals of one kernel name. */
void xfh_set_kernel_timing(int enable);
int xfh_kernel_timing_read(const char *name, double *total_ms, int64_t *launches);
/* The same, also summing the algorithmic work (FLOPs) the launches declared: 2 M N K per
 * GEMM for "gemm_ring", 4 B H Nq N Dv for "grid_attention" and "mha_attention", 0 for
 * kernels that declare none. */
int xfh_kernel_timing_read_work(const char *name, double *total_ms, int64_t *launches, double *work);

/* LayerNorm over the last dim of a contiguous [rows, cols] tensor; fp32 statistics.
 * Replaces the LayerNorm backends of xfold/fastnn/layer_norm.py:55-81 (torch/triton/ipex). */
int xfh_layer_norm(const void *x, int x_dtype, int64_t rows, int64_t cols,
                   const float *weight, const float *bias, float eps,
                   void *y, int y_dtype, void *stream);

/* Conditioned LayerNorm: y = sigmoid(scale[r % cond_rows]) * LN_noaffine(x[r]) + shift[r % cond_rows].
 * `scale`/`shift` are [cond_rows, cols] in `aux_dtype` (the two Linear outputs of the
 * conditioning branch). Replaces AdaptiveLayerNorm.forward's conditioned branch
 * (xfold/nn/diffusion_transformer.py:57-62) after its two Linears. */
int xfh_adaptive_layer_norm(const void *x, int x_dtype, int64_t rows, int64_t cols,
                            const void *scale, const void *shift, int aux_dtype, int64_t cond_rows,
                            float eps, void *y, int y_dtype, void *stream);

/* y[m, n] = epilogue(sum_k x[m, k] * w[n, k] + bias[n]); x row stride ldx, y row stride ldy,
 * aux row stride ldaux (aux in y_dtype). Replaces `linear` (af3_kernels/src/csrc/matrix.cpp,
 * bound at bindings.cpp:34-36; Python bridge xfold/fastnn/native.py:55-70). */
int xfh_linear(const void *x, int64_t ldx, const void *w, const float *bias,
               int64_t m, int64_t k, int64_t n, int dtype,
               void *y, int64_t ldy, int y_dtype,
               int epilogue, const void *aux, int64_t ldaux, int64_t aux_rows,
               void *stream);

/* Batched plain linear: for b < batch, y[b] = x[b] @ w[b]^T (+ bias[b]) with
 * x[b] = x + b*sx ([m, k] rows of ldx; sx = 0 shares one input), w[b] = w + b*sw ([n, k]),
 * bias[b] = bias + b*sbias (fp32, may be null), y[b] = y + b*sy ([m, n] rows of ldy).
 * No counterpart in the reference, which runs each block's conditioning linears
 * (AdaptiveLayerNorm and AdaLNZero, xfold/nn/diffusion_transformer.py:59-62, 93) as
 * separate nn.Linear calls; the hip DiffusionTransformer runs all of its blocks' ones as
 * one launch per input. */
int xfh_linear_batched(const void *x, int64_t ldx, int64_t sx, const void *w, int64_t sw,
                       const float *bias, int64_t sbias, int64_t m, int64_t k, int64_t n, int64_t batch,
                       int dtype, void *y, int64_t ldy, int64_t sy, int y_dtype, void *stream);

/* Rows of the packed GLU weight for f output features (gate and value interleaved in
 * groups of 16 features, zero rows pad f up to a multiple of 16). */
int64_t xfh_glu_packed_rows(int64_t f);

/* Packs transition1.weight ([2f, k], first f rows = SiLU gate) into the GLU layout. */
int xfh_glu_pack_weight(const void *w, int64_t f, int64_t k, int dtype, void *packed, void *stream);

/* y[m, :f] = silu(x @ Wg^T) * (x @ Wv^T) with a packed weight. Replaces `gated_linear_unit`
 * (af3_kernels/src/csrc/gated_linear_unit.cpp, bindings.cpp:29-32; torch body
 * xfold/fastnn/gated_linear_unit.py:103-107). */
int xfh_gated_linear_unit(const void *x, const void *w_packed, int64_t m, int64_t k, int64_t f,
                          int dtype, void *y, int y_dtype, void *stream);

/* Scaled dot-product attention with additive bias and key mask, flash-style (no [Q, K]
 * logits in memory). shape = {B, H, Q, K, D, Dv}. strides (elements) =
 *   {q_b, q_h, q_n,  k_b, k_h, k_n,  v_b, v_h, v_n,  o_b, o_h, o_n,
 *    mask_b, mask_h, mask_q, mask_k,  bias_b, bias_h, bias_q, bias_k}
 * (the last dim of q/k/v/out is contiguous; 0 strides broadcast). out_dtype may be f32
 * with bf16 inputs (fp32 accumulation is kept to the store). Semantics of
 * xfold/fastnn/attention.py:45-66: logits = (q*scale) k^T + bias; masked logits := -1e9;
 * softmax over keys; @ v. Replaces `dot_product_attention`
 * (af3_kernels/src/csrc/dot_product_attention.cpp:110-174, bindings.cpp:44-48).
 * With bf16 inputs and output, head dims <= 64, a bias shared by the batch entries and a
 * mask that depends on the batch entry and key only (the single-track and diffusion
 * shapes), a workspace of xfh_dot_product_attention_workspace_size(shape, dtype) bytes
 * selects the pipelined kernel; other calls, or workspace = NULL, use the general one.
 * bias_dtype = XFH_BIAS_PACKED or XFH_BIAS_PACKED_BF16: bias points at one [H][Q][align64(K)]
 * packed block (bias strides ignored); such calls must take the pipelined kernel and fail
 * with XFH_EUNSUPPORTED otherwise. */
int64_t xfh_dot_product_attention_workspace_size(const int64_t *shape, int dtype);
int xfh_dot_product_attention(const void *q, const void *k, const void *v, int dtype,
                              const void *mask, int mask_dtype, const void *bias, int bias_dtype,
                              void *out, int out_dtype, const int64_t *shape, const int64_t *strides,
                              float scale, void *workspace, int64_t workspace_bytes, void *stream);

/* Largest key count (and token count N) the pipelined attention kernel takes: the limit of
 * a packed bias (xfh_attention_bias_pack, xfh_pair_attention_bias). Longer key sequences
 * take xfh_dot_product_attention's general kernel with an unpacked bias. Capability query
 * with no counterpart in the reference, which has no such limit. */
int64_t xfh_attention_max_keys(void);

/* Converts G attention biases, bias[g][h][q][k] (shape = {G, H, Q, K}, strides in
 * elements, f32 or bf16), into the pipelined attention kernel's layout once:
 * packed[g][h][q][k'] fp32 = bias * log2(e) for k' < K, 0 for K <= k' < align64(K)
 * (packed holds G*H*Q*align64(K) floats). Block g is then passed to
 * xfh_dot_product_attention with bias_dtype XFH_BIAS_PACKED. No counterpart in the
 * reference: the DiffusionTransformer's pair logits (xfold/nn/diffusion_transformer.py:
 * 258-271) feed the attention biases of a whole super-block, which it converts once
 * instead of once per block. */
int xfh_attention_bias_pack(const void *bias, int dtype, const int64_t *shape, const int64_t *strides,
                            void *packed, void *stream);

/* Self-attention on operands in the pipelined attention kernel's own layouts, for B
 * samples of T tokens and H heads of Dh (Dh a multiple of 4, at most 64; T at most
 * xfh_attention_max_keys()): Dp = 32 (Dh <= 32) or 64, Tpad = align64(T), and bf16
 *   q [B][H][T][Dp], k [B][H][Tpad][Dp], vt [B][H][Dp][Tpad] (keys permuted inside runs of 32).
 * The three calls below split SelfAttention.forward (xfold/nn/diffusion_transformer.py:
 * 184-217: q/k/v projections, dot_product_attention, gating) so that the projection GEMM
 * writes these layouts directly and the gate is applied at the attention's store, with no
 * layout conversion in between; xfh_dot_product_attention keeps the general contract.
 * sizes[0..4] = {Dp, Tpad, q elements, k elements, vt elements}; XFH_EUNSUPPORTED for other
 * head dims or token counts. */
int xfh_attention_operands_size(int64_t B, int64_t T, int64_t H, int64_t Dh, int64_t *sizes);

/* [q | k | v (| gate)] = x w^T + bias in one bf16 GEMM, straight into those layouts:
 * x [B*T][K] bf16 (row stride ldx), w [N][K] bf16 = the stacked projection weights
 * [Wq; Wk; Wv] (N = 3c, c = H*Dh) or [Wq; Wk; Wv; Wg] (N = 4c, gate != NULL), bias fp32
 * [N] or NULL. q is multiplied by qscale; gate [B][T][c] bf16 holds the gating Linear's
 * output (before its sigmoid). The padding of q, k and vt (head dims >= Dh, keys >= T) is
 * never written: allocate them zeroed once and reuse them. Needs K % 32 == 0, ldx % 8 == 0
 * and 16-byte aligned x and w (XFH_EUNSUPPORTED otherwise). */
int xfh_attention_project(const void *x, int64_t ldx, const void *w, const float *bias, int64_t B, int64_t T,
                          int64_t K, int64_t H, int64_t Dh, float qscale, void *q, void *k, void *vt, void *gate,
                          void *stream);

/* Kept-key words of a key mask for xfh_attention_operands: words[b][w] bit j is set iff key
 * 64w + j < T is kept, i.e. mask[b*mask_stride + key] != 0 (NaN kept, as the reference's
 * .to(bool)); mask NULL keeps every key. words holds rows * align64(T)/64 uint64. */
int xfh_attention_mask_words(const void *mask, int mask_dtype, int64_t mask_stride, int64_t rows, int64_t T,
                             uint64_t *words, void *stream);

/* out [B][T][H*Dh] bf16 = softmax(q k^T + bias, masked keys removed) v over operands written
 * by xfh_attention_project (q already scaled), times sigmoid(gate) elementwise when gate is
 * given (gate [B][T][H*Dh] bf16: SelfAttention's gating, diffusion_transformer.py:209-211).
 * bias = one packed [H][T][Tpad] block of bias_dtype XFH_BIAS_PACKED or XFH_BIAS_PACKED_BF16
 * (xfh_attention_bias_pack, xfh_pair_attention_bias), required; words from xfh_attention_mask_words with rows = B, or rows = 1 and
 * words_shared = 1 for a mask shared by the samples. A row whose keys are all masked
 * averages v uniformly, as the reference's -1e9 fill does. */
int xfh_attention_operands(const void *q, const void *k, const void *vt, const uint64_t *words, int words_shared,
                           const void *bias, int bias_dtype, const void *gate, void *out, int64_t B, int64_t T,
                           int64_t H, int64_t Dh, void *stream);

/* Linear(LayerNorm(pair)) rearranged 'i j h -> h i j' straight into a packed bias layout:
 * with out_dtype XFH_F32, packed[h][i][j] fp32 = log2(e) * (LN(pair[i][j]) . w[h]) (the
 * layout of xfh_attention_bias_pack, an XFH_BIAS_PACKED bias per block of heads); with
 * XFH_BF16, packed[h][i][j] bf16 = LN(pair[i][j]) . w[h] (an XFH_BIAS_PACKED_BF16 bias,
 * rounded where the reference's autocast Linear rounds its output); 0 for n <= j <
 * align64(n). pair contiguous [n, n, c] (f32/bf16, c = 128), LayerNorm affine ln_w/ln_b
 * (fp32, may be null), w bf16 [heads][c] (heads <= 384), computed in bf16 with fp32
 * accumulation. Replaces the pair-logits path of PairformerBlock's single-track attention
 * (xfold/nn/pairformer.py:103-106) and of DiffusionTransformer
 * (xfold/nn/diffusion_transformer.py:258-271, all super-blocks' projections stacked). */
int xfh_pair_attention_bias(const void *pair, int pair_dtype, int64_t n, int64_t c, const float *ln_w,
                            const float *ln_b, float eps, const void *w, int w_dtype, int64_t heads,
                            void *packed, int out_dtype, void *stream);

/* Triangle multiplication update of a contiguous [n, n, c] pair tensor (mask [n, n]).
 * out (contiguous [n, n, c]) receives the update, or the update is added to it when
 * `accumulate` is nonzero (out may alias pair then). Replaces `triangle_multiplication`
 * (af3_kernels/src/csrc/triangle_multiplication.cpp:6-73, bindings.cpp:37-43; torch
 * module xfold/nn/triangle_multiplication.py:71-105). */
int64_t xfh_triangle_multiplication_workspace_size(int64_t n, int64_t c, int dtype);
int xfh_triangle_multiplication(const void *pair, int pair_dtype, const void *mask, int mask_dtype,
                                int64_t n, int64_t c, int outgoing,
                                const float *left_w, const float *left_b, float left_eps,
                                const void *proj_w, const void *gate_w,
                                const float *center_w, const float *center_b, float center_eps,
                                const void *out_w, const void *gating_w, int dtype,
                                void *out, int out_dtype, int accumulate,
                                void *workspace, int64_t workspace_bytes, void *stream);

/* Scratch bytes of xfh_triangle_multiplication_noalloc on each device (128 MiB: the bf16
 * c = 128 path up to n = 415, the fp32 path up to n = 161). */
#define XFH_NOALLOC_SCRATCH_BYTES ((int64_t)128 << 20)

/* xfh_triangle_multiplication without a workspace argument: the same arguments, result and
 * kernels, with the scratch in a device array the library holds on each device (of
 * XFH_NOALLOC_SCRATCH_BYTES; larger problems fail with XFH_EUNSUPPORTED). Allocates
 * nothing, so callers that cannot allocate device memory can use it: code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc. Calls on one device share
 * the scratch, so calls that overlap on one device (other streams, other host threads)
 * race; calls ordered on one stream do not. No counterpart in the reference. */
int xfh_triangle_multiplication_noalloc(const void *pair, int pair_dtype, const void *mask, int mask_dtype,
                                        int64_t n, int64_t c, int outgoing,
                                        const float *left_w, const float *left_b, float left_eps,
                                        const void *proj_w, const void *gate_w,
                                        const float *center_w, const float *center_b, float center_eps,
                                        const void *out_w, const void *gating_w, int dtype,
                                        void *out, int out_dtype, int accumulate, void *stream);

/* Grid (triangle) self-attention over a contiguous [n, n, c] pair tensor: starting node
 * (transpose = 0) or ending node (transpose = 1). Same output/accumulate contract as
 * xfh_triangle_multiplication. Replaces GridSelfAttention.forward
 * (xfold/nn/attention.py:80-105), whose cpp path chains `linear` and
 * `dot_product_attention` (xfold/nn/attention.py:49-59). */
int64_t xfh_grid_self_attention_workspace_size(int64_t n, int64_t c, int64_t heads, int dtype);
int xfh_grid_self_attention(const void *pair, int pair_dtype, const void *mask, int mask_dtype,
                            int64_t n, int64_t c, int64_t heads, int transpose,
                            const float *norm_w, const float *norm_b, float eps,
                            const void *bias_w, const void *q_w, const void *k_w, const void *v_w,
                            const void *gating_w, const void *out_w, int dtype,
                            void *out, int out_dtype, int accumulate,
                            void *workspace, int64_t workspace_bytes, void *stream);

/* Transition: LN -> GLU (packed transition1) -> transition2 over contiguous [rows, c].
 * Same output/accumulate contract. Replaces Transition.forward (xfold/nn/primitives.py:33-37),
 * whose GLU goes through `gated_linear_unit` (xfold/fastnn/gated_linear_unit.py:110-122). */
int64_t xfh_transition_workspace_size(int64_t rows, int64_t c, int64_t f, int dtype);
int xfh_transition(const void *x, int x_dtype, int64_t rows, int64_t c, int64_t f,
                   const float *norm_w, const float *norm_b, float eps,
                   const void *w1_packed, const void *w2, int dtype,
                   void *out, int out_dtype, int accumulate,
                   void *workspace, int64_t workspace_bytes, void *stream);

/* The pair transition of a Pairformer block with a single track, in place (pair += the
 * transition of pair, bf16 [n, n, 128], hidden 512), followed by that block's attention
 * bias of the updated pair, Linear(LN(pair)) -> packed [heads, n, align64(n)] fp32 times
 * log2(e) with zero pad columns (the xfh_pair_attention_bias layout), written from the
 * values the transition stores instead of a second pass over the pair. The results equal
 * xfh_transition (accumulate = 1) followed by xfh_pair_attention_bias (fp32 out) bit for
 * bit. 1..16 heads. Replaces pairformer.py:100 and :103-106 (xfold/nn/pairformer.py),
 * the block's last pair update and its pair-logit projection. */
int xfh_transition_pair_bias(void *pair, int64_t n, int64_t c, int64_t f, const float *norm_w,
                             const float *norm_b, float eps, const void *w1_packed, const void *w2,
                             const float *bias_ln_w, const float *bias_ln_b, float bias_eps,
                             const void *bias_w, int64_t heads, float *packed, void *stream);

/* OuterProductMean of the Evoformer's MSA stack over a contiguous msa [rows, n, c_msa] with
 * mask [rows, n] (NULL = all ones):
 *   out[i, j, f] = (sum_{c,e} O[i, j, c, e] * w[f, c * c_outer + e] + b[f]) / (norm_eps + M[i, j])
 *   O[i, j, c, e] = sum_s mask[s, i] L[s, i, c] * mask[s, j] R[s, j, e],
 *   M[i, j] = sum_s mask[s, i] mask[s, j],  [L | R] = LN(msa) @ proj_w^T,
 * proj_w [2 c_outer, c_msa] = [left_projection.weight; right_projection.weight], out_w
 * [c_out, c_outer^2] = output_w permuted 'c e f -> f (c e)', out_b fp32 [c_out]. out is
 * contiguous [n, n, c_out], stored or accumulated into (accumulate nonzero). c_outer a
 * multiple of 4, at most 64; rows >= 1. Replaces OuterProductMean.forward
 * (xfold/nn/primitives.py:40-72). */
int64_t xfh_outer_product_mean_workspace_size(int64_t rows, int64_t n, int64_t c_msa, int64_t c_outer, int dtype);
int xfh_outer_product_mean(const void *msa, int msa_dtype, const void *mask, int mask_dtype, int64_t rows,
                           int64_t n, int64_t c_msa, int64_t c_outer, int64_t c_out, const float *ln_w,
                           const float *ln_b, float ln_eps, const void *proj_w, const void *out_w,
                           const float *out_b, float norm_eps, int dtype, void *out, int out_dtype,
                           int accumulate, void *workspace, int64_t workspace_bytes, void *stream);

/* MSA row attention with pair logits over msa [rows, n, c_msa], msa_mask [rows, n] (NULL =
 * all ones) and pair [n, n, c_pair], all contiguous:
 *   logits[h, q, k] = LN(pair)[q, k] . logits_w[h] + 1e9 * (max_s mask[s, k] - 1),
 *   w = softmax over k (shared by every MSA row), v = LN(msa) @ v_w^T split into heads,
 *   avg[s, q, h, :] = sum_k w[h, q, k] v[s, k, h, :],
 *   out = (avg * sigmoid(LN(msa) @ gating_w^T)) @ out_w^T, stored or accumulated.
 * logits_w [heads, c_pair], v_w/gating_w/out_w [c_msa, c_msa]; head dim c_msa / heads <= 16.
 * With bf16 compute and c_pair = 128 the logits come from the pair-bias kernel of
 * xfh_pair_attention_bias. Replaces MSAAttention.forward (xfold/nn/attention.py:108-144). */
int64_t xfh_msa_attention_workspace_size(int64_t rows, int64_t n, int64_t c_msa, int64_t c_pair, int64_t heads,
                                         int dtype);
int xfh_msa_attention(const void *msa, int msa_dtype, const void *mask, int mask_dtype, const void *pair,
                      int pair_dtype, int64_t rows, int64_t n, int64_t c_msa, int64_t c_pair, int64_t heads,
                      const float *ln_w, const float *ln_b, float ln_eps, const float *pair_ln_w,
                      const float *pair_ln_b, float pair_ln_eps, const void *logits_w, const void *v_w,
                      const void *gating_w, const void *out_w, int dtype, void *out, int out_dtype, int accumulate,
                      void *workspace, int64_t workspace_bytes, void *stream);

/* Logit bias of the atom CrossAttention, fp32 out [batch, heads, nq, nk] contiguous:
 *   out[b, h, q, k] = pair_logits[b, h, q, k] + 1e9 * (mask_q[b, q] == 0 && mask_k[b, k] == 0)
 * pair_logits strided (4 strides in elements, f32/bf16) or NULL (0); masks contiguous
 * [batch, nq] / [batch, nk] (f32/bf16/bool) or NULL (all kept). The result is the bias of
 * an xfh_dot_product_attention call with no mask. Replaces the bias construction of
 * CrossAttention.forward (xfold/nn/diffusion_transformer.py:318-339), whose positive 1e9
 * term makes a masked query attend to the masked keys only. */
int xfh_cross_attention_bias(const void *pair_logits, int logits_dtype, const int64_t *strides,
                             const void *mask_q, int mask_q_dtype, const void *mask_k, int mask_k_dtype,
                             int64_t batch, int64_t heads, int64_t nq, int64_t nk, float *out, void *stream);

/* y[i] = x[i] converted between f32 and bf16 (round to nearest even), both contiguous with n
 * elements. The activation cast that torch autocast inserts in front of each Linear
 * (xfold/fastnn/native.py:31-43 computes in the autocast dtype); the hip modules run it here
 * instead of in a torch kernel. */
int xfh_convert(const void *x, int x_dtype, void *y, int y_dtype, int64_t n, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* XFOLD_HIP_H */
