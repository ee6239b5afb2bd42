// Internal launch interfaces shared by the kernel files and the C-ABI layer.
#pragma once

#include "common.h"

namespace xfh {

// Attention-operand output of a fused [q | k | v | gate] projection (gemm_ring, bf16 out,
// store epilogue): row m = b*T + t, column n = part*c + h*Dh + d (c = H*Dh) goes to
//   part 0: q    [B][H][T][Dp]    times qscale
//   part 1: k    [B][H][Tpad][Dp]
//   part 2: vt   [B][H][Dp][Tpad] with the attention kernel's key order inside runs of 32
//   part 3: gate [B][T][c]        (the gating Linear, when N = 4c)
// The head-dim padding (d >= Dh) and key padding (t >= T) are never written.
struct AttnOut {
  bf16 *q, *k, *vt, *gate;   // q null: row-major output
  int T, Tpad, H, Dh, Dp;
  float qscale;
};

struct GemmArgs {
  const void *A;
  int64_t lda, sA;          // row stride, batch stride (elements)
  const void *B;
  int64_t ldb, sB;
  void *C;
  int64_t ldc, sC;
  const float *bias;        // [N] or null (batch b reads bias + b * sBias)
  int64_t sBias;
  const void *aux;          // epilogue operand in C's dtype, or null
  int64_t ldaux, sAux, aux_rows;
  int M, N, K;
  int epi;                  // XFH_EPI_*
  // gemm_ring tile placement: 0 = plain 2-D grid; g in {1, 2, 4, 8} = each XCD takes one
  // rectangle of tiles out of a (8/g row groups) x (g column groups) split of the output.
  int xcd_split;
  int glu_f;                // GLU output features (GLU launches only)
  // Row divisor: the value (acc + bias) of row m is divided by (row_div_eps + row_div[m])
  // before the epilogue (fp32 [M], null = none).
  const float *row_div;
  float row_div_eps;
  // Pair-block output layout (0 = row-major): with blk > 0 the element (m, n) of an
  // [M = I*blk] x [N = J*blk] product goes to C[((m/blk * J + n/blk) * blk + m%blk) * blk + n%blk],
  // i.e. the [I][blk] x [J][blk] result stored as [I][J][blk][blk] (ldc unused).
  int pair_blk;
  AttnOut attn;             // attention-operand layout (attn.q != null), gemm_ring only
};

// Address of element (m, n) of C (row-major, or the pair-block layout).
template <typename TO> __device__ __forceinline__ TO *c_element(const GemmArgs &p, TO *C, int m, int n) {
  if (p.pair_blk == 0) return C + int64_t(m) * p.ldc + n;
  const int blk = p.pair_blk, jn = p.N / blk;
  return C + ((int64_t(m / blk) * jn + n / blk) * blk + m % blk) * blk + n % blk;
}

int gemm_nt(const GemmArgs &p, int64_t batch, int dtype, int out_dtype, bool glu, hipStream_t s);
// dst = the rows of up to four row-major matrices of `cols` elements (es bytes each), stacked
// (16-byte aligned sources, each a multiple of 16 bytes; rows[i] = 0 skips src[i]).
int stack_rows(void *dst, const void *const src[4], const int64_t rows[4], int64_t cols, int es, hipStream_t s);
// bf16-input GEMM with a direct-load LDS ring (gemm_ring.hip); gemm_nt routes to it when
// gemm_ring_supported (k a multiple of 32, 16-byte aligned operand rows, 4-aligned output).
bool gemm_ring_supported(const GemmArgs &p, int out_dtype);
int gemm_ring(const GemmArgs &p, int64_t batch, int out_dtype, bool glu, hipStream_t s);
int glu_pack(const void *w, int64_t f, int64_t k, int dtype, void *packed, hipStream_t s);

int layer_norm_rows(const void *x, int xd, int64_t rows, int64_t C, const float *w, const float *b,
                    float eps, void *y, int yd, hipStream_t s);
int adaptive_layer_norm_rows(const void *x, int xd, int64_t rows, int64_t C, const void *scale,
                             const void *shift, int ad, int64_t cond_rows, float eps, void *y,
                             int yd, hipStream_t s);
int layer_norm_planes(const void *x, int xd, int64_t plane, int C, const float *w, const float *b,
                      float eps, void *y, int yd, hipStream_t s);

struct AttentionArgs {
  const void *q, *k, *v;
  void *o;
  const void *mask;
  const void *bias;
  int mask_dtype, bias_dtype, out_dtype;
  int64_t B, H, Q, K, D, Dv;
  int64_t qs[3], ks[3], vs[3], os[3];
  int64_t ms[4], bs[4];
  float scale;
};
int attention(const AttentionArgs &a, int dtype, hipStream_t s);
// dot_product_attention on the triangle-attention kernel (mha.hip).
int64_t mha_workspace_size(const AttentionArgs &a);
bool mha_supported(const AttentionArgs &a, int dtype);
int mha(const AttentionArgs &a, void *workspace, int64_t workspace_bytes, hipStream_t s);
int attention_bias_pack(const void *bias, int dtype, const int64_t *shape, const int64_t *strides, void *packed,
                        hipStream_t s);
// Self-attention on operands already in the pipelined kernel's layouts (mha.hip): padded
// head dim and key count, kept-key words, and the attention with an optional gate.
int attention_operands_dims(int64_t T, int64_t Dh, int *dp, int64_t *tpad);
int attention_mask_words(const void *mask, int dtype, int64_t stride, int64_t rows, int64_t T, uint64_t *words,
                         hipStream_t s);
int attention_operands(const bf16 *q, const bf16 *k, const bf16 *vt, const uint64_t *words, bool words_shared,
                       const void *bias, bool bias_bf16, const bf16 *gate, bf16 *out, int64_t B, int64_t T,
                       int64_t H, int64_t Dh, hipStream_t s);
// Linear(LayerNorm(pair)) straight into the packed attention-bias layout (pair_bias.hip).
struct PairBiasArgs {
  const void *pair;          // [n][n][128]
  const float *ln_w, *ln_b;
  float eps;
  const bf16 *w;             // [heads][128]
  void *packed;              // [heads][n][npad]: fp32 times log2(e), or bf16 (natural units)
  int packed_bf16 = 0;
  int n, npad, heads;
};
int pair_bias_max_heads();
int pair_bias(const PairBiasArgs &a, int pair_dtype, hipStream_t s);

// Triangle (grid) attention, bf16, head dim 32 (grid_attention.hip).
// Layouts (D = padded head dim, 32 or 64): q [B][H][Nq][D] pre-scaled by d^-0.5 * log2(e);
// k [B][H][Npad][D] and v^T [B][H][D][Npad] zero beyond the N keys (v^T keys permuted in
// runs of 32, see grid_project); bias [H][Nq][Npad] fp32 times log2(e), shared by all b.
struct GridAttentionArgs {
  const bf16 *q, *k, *vt;
  // [H][Nq][Npad]: fp32 times log2(e), or with bias_bf16 bf16 in natural units.
  const void *bias;
  const uint64_t *maskbits;  // word w of row b at maskbits[b*mbs + w] (mbs 0: one shared row)
  bf16 *out;
  int64_t osb, ost, ohs;     // out element (b, t, h, d) at out[b*osb + t*ost + h*ohs + d], d < Dv
  int64_t mbs;
  int B, H, Nq, N, Npad, Nblk, Dv;
  // Optional gate in out's layout: out = sigmoid(gate) * attention (the gating Linear of
  // SelfAttention applied at the store).
  const bf16 *gate = nullptr;
  int bias_bf16 = 0;
};
// Fused grid-attention projection / output (grid_fused.hip), bf16, c = 128, 4 x 32 heads.
struct GridProjectArgs {
  const void *pair;
  int n, heads, transpose;
  const float *ln_w, *ln_b;
  float eps;
  const bf16 *wq, *wk, *wv, *wb;  // nn.Linear weights [c][c] (wb: [heads][c])
  const void *mask;          // [n][n] (key k of row b at b*n + k), or null
  int mask_dtype;
  uint64_t *maskbits;        // [n][npad/64] kept-key words for the attention kernel
  float qscale;              // d^-0.5 * log2(e)
  bf16 *q, *k, *vt;
  float *bias;
  int npad;
};
struct GridOutputArgs {
  const void *pair;
  const bf16 *attn;          // [n*n][c], pair-row order
  const float *ln_w, *ln_b;
  float eps;
  const bf16 *w_gating, *w_out;
  void *out;
  int accumulate, n;
};
// One launch: the packed [q | k | v | bias] weight of grid_project and the 64-bit
// kept-key words of the attention kernel (bit s of word b*nblk + s/64 set iff key s < n of
// batch row b is kept, mask[b*n + s] != 0).
int grid_project(const GridProjectArgs &a, int pair_dtype, hipStream_t s);
int grid_output(const GridOutputArgs &a, int pair_dtype, int out_dtype, hipStream_t s);
int64_t grid_attention_pad(int64_t n);
// The same kernel for head dims 32 and 64 (d = 32 or 64) at the shapes of dot_product_attention.
int mha_attention(const GridAttentionArgs &a, int d, hipStream_t s);
// The grid attention's operands at head dim padded_dim(dh) from row-major [q | k | v]
// projection rows of stride ld (B = T batch rows, pair order; transpose: the ending node).
int qkv_repack(const bf16 *qkv, int64_t ld, int64_t B, int64_t T, int64_t H, int64_t dh, int transpose, float scale,
               bf16 *q, bf16 *k, bf16 *vt, hipStream_t s);
int64_t grid_attention_max_n();
int grid_attention(const GridAttentionArgs &a, hipStream_t s);

// Fused triangle multiplication, bf16 compute, c = 128 (trimul_fused.hip).
struct TriProjectArgs {
  const void *pair;
  const void *mask;
  int mask_dtype;
  const float *ln_w, *ln_b;
  float eps;
  const bf16 *w_proj, *w_gate;  // [2c][c] each (nn.Linear layout)
  bf16 *left, *right;        // contraction operands in the blocked operand layout, zero-padded
  int n, ld, outgoing;
};
struct TriOutputArgs {
  const void *pair;
  const bf16 *contracted;    // contraction result in the blocked result layout
  const float *ln_in_w, *ln_in_b;
  float eps_in;
  const float *ln_c_w, *ln_c_b;
  float eps_c;
  const bf16 *w_gating, *w_out;
  void *out;
  int accumulate, n;
};
// Fused pair transition (transition_fused.hip), bf16 compute, c = 128, hidden 512.
struct TransitionArgs {
  const void *x;
  int64_t rows;
  const float *ln_w, *ln_b;
  float eps;
  const bf16 *w1;            // GLU-packed transition1 weight [1024][128]
  const bf16 *w2;            // transition2 weight [128][512]
  void *out;
  int accumulate;
};
int transition_fused(const TransitionArgs &a, int x_dtype, int out_dtype, hipStream_t s);
// The in-place bf16 pair transition (a.x == a.out, accumulating) followed by the attention
// bias Linear(LayerNorm(pair)) of the updated pair, computed in the transition's epilogue
// from the values it stores: the result equals transition_fused then pair_bias (fp32 times
// log2(e), [heads][n][npad], zero pad columns) bit for bit; heads <= 16, a.rows == n * n.
struct TransitionBias {
  const float *ln_w, *ln_b;
  float eps;
  const bf16 *w;             // [heads][128]
  float *packed;             // [heads][n][npad]
  int n, npad, heads;
};
int transition_pair_bias(const TransitionArgs &a, const TransitionBias &b, hipStream_t s);

// Layouts of the triangle multiplication's contraction (c = channels, ld = contraction_ld(n)):
//   operand (left, right): element (ch, i, t) of the per-channel [n][ld] matrices in blocks of
//     16 rows x 32 t (1 KB): block (t/32, i/16) holds the blocks of all channels together,
//     element at ((t/32) * G + i/16) * op_group_stride + ch * 512 + (i % 16) * 32 + t % 32,
//     G = ceil(n/16); zero for t >= n;
//   result: element (ch, pos = i*n + j) at (pos/16) * res_block_stride + ch * 16 + pos % 16:
//     16 pair positions, all channels of them contiguous (4 KB).
// The contraction reads each k-step of 16 rows as one contiguous 1 KB piece; trimul_project's
// wavefronts write neighbouring grid lines of one k-slice at the same time (64-byte pieces
// that fill whole rows of a block); trimul_output reads 16 positions' channels as one
// contiguous block. Against channel-major [c][n][ld] operands and [c][n*n] results this
// took the contraction from 167 to 155 us and trimul_output from 123 to 101 us at n = 768.
// The result blocks are padded by 128 bytes so that the contraction's stores to the 16
// rows i of a tile are not a power of two apart.
constexpr int kOpGroupPad = 0, kResPad = 64;    // elements (multiples of 8)
__host__ __device__ inline int64_t op_groups(int64_t n) { return (n + 15) / 16; }
__host__ __device__ inline int64_t op_group_stride(int c) { return int64_t(c) * 512 + kOpGroupPad; }
__host__ __device__ inline int64_t op_step_stride(int64_t n, int c) { return op_groups(n) * op_group_stride(c); }
__host__ __device__ inline int64_t op_offset(int64_t n, int c, int ch, int64_t i, int64_t s) {
  return (s * op_groups(n) + (i >> 4)) * op_group_stride(c) + int64_t(ch) * 512 + (i & 15) * 32;
}
__host__ __device__ inline int64_t res_block_stride(int c) { return int64_t(c) * 16 + kResPad; }
__host__ __device__ inline int64_t res_offset(int c, int ch, int64_t pos) {
  return (pos >> 4) * res_block_stride(c) + int64_t(ch) * 16 + (pos & 15);
}
struct ContractionArgs {
  const bf16 *left, *right;  // blocked operand layout
  bf16 *out;                 // blocked result layout
  int n, ld, channels;
};
int64_t contraction_ld(int64_t n);
int64_t contraction_operand_elems(int64_t n, int64_t channels);
int64_t contraction_result_elems(int64_t n, int64_t channels);
int contraction(const ContractionArgs &a, hipStream_t s);
int trimul_project(const TriProjectArgs &a, int pair_dtype, hipStream_t s);
int trimul_output(const TriOutputArgs &a, int pair_dtype, int out_dtype, hipStream_t s);

// Triangle multiplication helpers.
int trimul_gate(const void *proj, const void *gate, int dtype, const void *mask, int mask_dtype,
                int64_t n, int64_t c, int outgoing, void *a_out, void *b_out, hipStream_t s);

}  // namespace xfh
