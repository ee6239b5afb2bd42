// The Evoformer's MSA-stack operators, composed from the library's GEMMs and LayerNorm and
// the small layout kernels below:
//   OuterProductMean (xfold/nn/primitives.py:40-72)
//     LN(msa) -> [left | right] projections (one GEMM) -> masked, sequence-contiguous
//     operands L^T, R^T [n][c][s] and the mask M^T [n][s] (opm_operands_kernel) ->
//     O = L^T R (one GEMM over the sequences, stored [i][j][c][e]) -> out = O W + b divided
//     row-wise by (eps + M^T M) (one GEMM, the divisor from one more GEMM over the mask).
//   MSAAttention (xfold/nn/attention.py:108-144)
//     pair logits Linear(LN(pair)) -> softmax over keys with the MSA key term
//     1e9 (max_s mask[s,k] - 1) (msa_key_term_kernel, msa_softmax_kernel), shared by every
//     MSA row -> v^T per head (GEMM) -> weights x v per head (GEMM over keys) -> rows back to
//     [s][q][h, c] (msa_gather_kernel) -> sigmoid(gating) x (GEMM epilogue) -> output GEMM.
#include <cstring>
#include <string>

#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int kOpmTile = 32;           // sequences per opm_operands workgroup

// lr [rows][n][2 co] (left = columns [0, co), right = [co, 2 co)); mask [rows][n] (null = ones).
// lt, rt [n][co][spad] = mask * lr for s < rows, 0 beyond; mt [n][spad] = mask, 0 beyond.
// Workgroup (sequence tile, residue i): the tile's rows go through LDS so that both the reads
// (2 co contiguous channels per sequence) and the writes (32 contiguous sequences per channel)
// are coalesced.
template <typename T>
__global__ __launch_bounds__(256) void opm_operands_kernel(const T *__restrict__ lr, const void *__restrict__ mask,
                                                           int mask_dtype, int rows, int n, int co, int spad,
                                                           T *__restrict__ lt, T *__restrict__ rt, T *__restrict__ mt) {
  __shared__ float tile[kOpmTile][129];         // 2 co <= 128 channels of 32 sequences
  __shared__ float mrow[kOpmTile];
  const int s0 = blockIdx.x * kOpmTile, i = blockIdx.y, tid = threadIdx.x;
  const int width = 2 * co;
  for (int idx = tid; idx < kOpmTile * width; idx += blockDim.x) {
    const int t = idx / width, ch = idx % width, s = s0 + t;
    tile[t][ch] = s < rows ? static_cast<float>(lr[(int64_t(s) * n + i) * width + ch]) : 0.f;
  }
  if (tid < kOpmTile) {
    const int s = s0 + tid;
    mrow[tid] = s < rows ? (mask ? load_any(mask, mask_dtype, int64_t(s) * n + i) : 1.f) : 0.f;
  }
  __syncthreads();
  for (int idx = tid; idx < kOpmTile * width; idx += blockDim.x) {
    const int ch = idx / kOpmTile, t = idx % kOpmTile;
    const float v = tile[t][ch] * mrow[t];
    T *dst = ch < co ? lt + (int64_t(i) * co + ch) * spad : rt + (int64_t(i) * co + ch - co) * spad;
    dst[s0 + t] = static_cast<T>(v);
  }
  if (tid < kOpmTile) mt[int64_t(i) * spad + s0 + tid] = static_cast<T>(mrow[tid]);
}

// kt[k] = 1e9 * (max over s of mask[s][k] - 1) (0 without a mask): the additive key term of
// xfold/nn/attention.py:129. Workgroup = 64 keys; its 16 wavefronts take every 16th MSA row
// (independent loads, several in flight per lane), then combine their maxima through LDS.
constexpr int kKeyTermWaves = 16;
__global__ __launch_bounds__(64 * kKeyTermWaves) void msa_key_term_kernel(const void *__restrict__ mask,
                                                                         int mask_dtype, int rows, int n,
                                                                         float *__restrict__ kt) {
  __shared__ float part[kKeyTermWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + lane;
  float m = -__builtin_inff();
  if (mask && k < n) {
#pragma unroll 4
    for (int s = wave; s < rows; s += kKeyTermWaves) m = fmaxf(m, load_any(mask, mask_dtype, int64_t(s) * n + k));
  }
  part[wave][lane] = m;
  __syncthreads();
  if (wave == 0 && k < n) {
#pragma unroll
    for (int w = 1; w < kKeyTermWaves; ++w) m = fmaxf(m, part[w][lane]);
    kt[k] = mask ? 1e9f * (m - 1.0f) : 0.f;
  }
}

// One wavefront per (head h, query q): w[h][q][k] = softmax over k < n of
// (logit(h, q, k) * scale + kt[k]), zero for n <= k < npad. logit(h, q, k) =
// logits[h * sh + q * sq + k * sk] (fp32 or bf16); scale converts it to natural-log units.
// All arithmetic in fp32, as the reference's softmax over fp32 logits.
template <typename T>
__global__ __launch_bounds__(256) void msa_softmax_kernel(const void *__restrict__ logits, int logit_dtype,
                                                          int64_t sh, int64_t sq, int64_t sk, float scale,
                                                          const float *__restrict__ kt, int heads, int n, int npad,
                                                          T *__restrict__ w) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (row >= int64_t(heads) * n) return;
  const int h = int(row / n), q = int(row % n);
  const int64_t base = h * sh + q * sq;
  float mx = -__builtin_inff();
  for (int k = lane; k < n; k += 64) mx = fmaxf(mx, load_any(logits, logit_dtype, base + k * sk) * scale + kt[k]);
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = 0.f;
  for (int k = lane; k < n; k += 64) sum += expf(load_any(logits, logit_dtype, base + k * sk) * scale + kt[k] - mx);
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  const float inv = 1.0f / sum;
  T *dst = w + row * npad;
  for (int k = lane; k < npad; k += 64)
    dst[k] = static_cast<T>(k < n ? expf(load_any(logits, logit_dtype, base + k * sk) * scale + kt[k] - mx) * inv : 0.f);
}

constexpr int kGatherRows = 256;      // sequences per msa_gather workgroup

// avg_t [heads][n][dv][rows] -> avg [rows][n][heads * dv]. Workgroup (query q, head h,
// sequence chunk): the dv x 256 source block is read contiguously into LDS, then each thread
// writes one sequence's dv contiguous channels.
template <typename T>
__global__ __launch_bounds__(kGatherRows) void msa_gather_kernel(const T *__restrict__ avg_t, int heads, int n, int dv,
                                                                 int rows, T *__restrict__ avg) {
  __shared__ T tile[16][kGatherRows];
  const int q = blockIdx.x % n, h = blockIdx.x / n, s0 = blockIdx.y * kGatherRows, tid = threadIdx.x;
  const T *src = avg_t + (int64_t(h) * n + q) * dv * int64_t(rows);
  for (int c = 0; c < dv; ++c)
    if (s0 + tid < rows) tile[c][tid] = src[int64_t(c) * rows + s0 + tid];
  __syncthreads();
  const int s = s0 + tid;
  if (s >= rows) return;
  T *dst = avg + (int64_t(s) * n + q) * int64_t(heads) * dv + int64_t(h) * dv;
  for (int c = 0; c < dv; ++c) dst[c] = tile[c][tid];
}

bool fdtype(int d) { return d == XFH_F32 || d == XFH_BF16; }
int64_t esize(int d) { return d == XFH_F32 ? 4 : 2; }

GemmArgs plain_gemm(const void *A, int64_t lda, const void *B, int64_t ldb, void *C, int64_t ldc, int64_t M,
                    int64_t N, int64_t K) {
  GemmArgs g;
  std::memset(&g, 0, sizeof(g));
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc;
  g.M = int(M); g.N = int(N); g.K = int(K);
  g.epi = XFH_EPI_STORE;
  return g;
}

struct OpmPlan {
  void *normed, *lr, *lt, *rt, *mt, *outer;
  float *norm;
};

int64_t opm_carve(Carver &cv, OpmPlan &p, int64_t rows, int64_t n, int64_t c_msa, int64_t co, int dtype) {
  const int64_t es = esize(dtype), spad = align_up(rows, int64_t(kOpmTile));
  p.normed = cv.take(rows * n * c_msa * es);
  p.lr = cv.take(rows * n * 2 * co * es);
  p.lt = cv.take(n * co * spad * es);
  p.rt = cv.take(n * co * spad * es);
  p.mt = cv.take(n * spad * es);
  p.outer = cv.take(n * n * co * co * es);
  p.norm = static_cast<float *>(cv.take(n * n * 4));
  return cv.used;
}

struct MsaPlan {
  void *normed, *pair_normed, *logits, *weights, *vt, *avg_t, *avg;
  float *kt;
};

int64_t msa_carve(Carver &cv, MsaPlan &p, int64_t rows, int64_t n, int64_t c_msa, int64_t c_pair, int64_t heads,
                  int dtype, bool packed) {
  const int64_t es = esize(dtype), npad = align_up(n, int64_t(64));
  p.normed = cv.take(rows * n * c_msa * es);
  p.pair_normed = packed ? nullptr : cv.take(n * n * c_pair * es);
  p.logits = packed ? cv.take(heads * n * npad * 4) : cv.take(n * n * heads * es);
  p.kt = static_cast<float *>(cv.take(npad * 4));
  p.weights = cv.take(heads * n * npad * es);
  p.vt = cv.take(rows * n * c_msa * es);
  p.avg_t = cv.take(rows * n * c_msa * es);
  p.avg = cv.take(rows * n * c_msa * es);
  return cv.used;
}

bool msa_packed_logits(int64_t n, int64_t c_pair, int64_t heads, int dtype) {
  return dtype == XFH_BF16 && c_pair == 128 && heads <= pair_bias_max_heads() && n <= 16384;
}

}  // namespace

}  // namespace xfh

using namespace xfh;

extern "C" {

int64_t xfh_outer_product_mean_workspace_size(int64_t rows, int64_t n, int64_t c_msa, int64_t c_outer, int dtype) {
  if (rows < 0 || n < 0 || c_msa < 0 || c_outer < 0 || !fdtype(dtype)) return -1;
  Carver cv(nullptr, 0);
  OpmPlan p;
  return opm_carve(cv, p, rows, n, c_msa, c_outer, dtype) + 256;
}

int xfh_outer_product_mean(const void *msa, int msa_dtype, const void *mask, int mask_dtype, int64_t rows,
                           int64_t n, int64_t c_msa, int64_t c_outer, int64_t c_out, const float *ln_w,
                           const float *ln_b, float ln_eps, const void *proj_w, const void *out_w,
                           const float *out_b, float norm_eps, int dtype, void *out, int out_dtype,
                           int accumulate, void *workspace, int64_t workspace_bytes, void *stream) {
  XFH_REQUIRE(rows > 0 && n >= 0 && c_msa > 0 && c_outer > 0 && c_out > 0,
              "outer_product_mean: needs at least one MSA row and positive channel counts");
  XFH_REQUIRE(c_outer <= 64 && c_outer % 4 == 0, "outer_product_mean: outer channels must be a multiple of 4, <= 64");
  XFH_REQUIRE(fdtype(msa_dtype) && fdtype(dtype) && fdtype(out_dtype), "outer_product_mean: dtypes must be f32/bf16");
  XFH_REQUIRE(!mask || mask_dtype == XFH_F32 || mask_dtype == XFH_BF16 || mask_dtype == XFH_BOOL,
              "outer_product_mean: bad mask dtype");
  XFH_REQUIRE(ln_eps >= 0.f && norm_eps >= 0.f, "outer_product_mean: eps must be nonnegative");
  if (n == 0) return XFH_OK;
  XFH_REQUIRE(n * c_outer < (int64_t(1) << 31) && n * n < (int64_t(1) << 31) && rows * n < (int64_t(1) << 31) &&
                  rows <= (int64_t(1) << 30),
              "outer_product_mean: sizes must fit in 32 bits");
  XFH_REQUIRE(msa && out && proj_w && out_w, "outer_product_mean: null tensor");
  Carver cv(workspace, workspace_bytes);
  OpmPlan p;
  const int64_t need = opm_carve(cv, p, rows, n, c_msa, c_outer, dtype);
  if (!workspace || need > workspace_bytes)
    return fail(XFH_EWORKSPACE, "outer_product_mean: workspace too small (need " + std::to_string(need) + " bytes)");
  hipStream_t s = as_stream(stream);
  const int64_t spad = align_up(rows, int64_t(kOpmTile)), co = c_outer;
  XFH_TRY(layer_norm_rows(msa, msa_dtype, rows * n, c_msa, ln_w, ln_b, ln_eps, p.normed, dtype, s));
  {
    GemmArgs g = plain_gemm(p.normed, c_msa, proj_w, c_msa, p.lr, 2 * co, rows * n, 2 * co, c_msa);
    XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
  }
  const dim3 grid(unsigned(spad / kOpmTile), unsigned(n));
  {
    if (dtype == XFH_BF16)
      opm_operands_kernel<bf16><<<grid, 256, 0, s>>>(static_cast<const bf16 *>(p.lr), mask, mask_dtype, int(rows),
                                                      int(n), int(co), int(spad), static_cast<bf16 *>(p.lt),
                                                      static_cast<bf16 *>(p.rt), static_cast<bf16 *>(p.mt));
    else
      opm_operands_kernel<float><<<grid, 256, 0, s>>>(static_cast<const float *>(p.lr), mask, mask_dtype, int(rows),
                                                       int(n), int(co), int(spad), static_cast<float *>(p.lt),
                                                       static_cast<float *>(p.rt), static_cast<float *>(p.mt));
    XFH_TRY(check_launch("opm_operands"));
  }
  {
    // outer[i][j][c][e] = sum_s lt[i][c][s] rt[j][e][s]
    GemmArgs g = plain_gemm(p.lt, spad, p.rt, spad, p.outer, 0, n * co, n * co, spad);
    g.pair_blk = int(co);
    XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
    // norm[i][j] = sum_s mask[s][i] mask[s][j]
    g = plain_gemm(p.mt, spad, p.mt, spad, p.norm, n, n, n, spad);
    XFH_TRY(gemm_nt(g, 1, dtype, XFH_F32, false, s));
  }
  // out[i][j] = (outer[i][j] . W + b) / (eps + norm[i][j]), stored or accumulated.
  GemmArgs g = plain_gemm(p.outer, co * co, out_w, co * co, out, c_out, n * n, c_out, co * co);
  g.bias = out_b;
  g.row_div = p.norm;
  g.row_div_eps = norm_eps;
  g.epi = accumulate ? XFH_EPI_ACCUMULATE : XFH_EPI_STORE;
  return gemm_nt(g, 1, dtype, out_dtype, false, s);
}

int64_t xfh_msa_attention_workspace_size(int64_t rows, int64_t n, int64_t c_msa, int64_t c_pair, int64_t heads,
                                         int dtype) {
  if (rows < 0 || n < 0 || c_msa < 0 || c_pair < 0 || heads <= 0 || !fdtype(dtype)) return -1;
  Carver cv(nullptr, 0);
  MsaPlan p;
  return msa_carve(cv, p, rows, n, c_msa, c_pair, heads, dtype, msa_packed_logits(n, c_pair, heads, dtype)) + 256;
}

int xfh_msa_attention(const void *msa, int msa_dtype, const void *mask, int mask_dtype, const void *pair,
                      int pair_dtype, int64_t rows, int64_t n, int64_t c_msa, int64_t c_pair, int64_t heads,
                      const float *ln_w, const float *ln_b, float ln_eps, const float *pair_ln_w,
                      const float *pair_ln_b, float pair_ln_eps, const void *logits_w, const void *v_w,
                      const void *gating_w, const void *out_w, int dtype, void *out, int out_dtype, int accumulate,
                      void *workspace, int64_t workspace_bytes, void *stream) {
  XFH_REQUIRE(rows >= 0 && n >= 0 && c_msa > 0 && c_pair > 0 && heads > 0 && c_msa % heads == 0,
              "msa_attention: bad size");
  const int64_t dv = c_msa / heads;
  XFH_REQUIRE(dv <= 16, "msa_attention: head dim must be <= 16");
  XFH_REQUIRE(fdtype(msa_dtype) && fdtype(pair_dtype) && fdtype(dtype) && fdtype(out_dtype),
              "msa_attention: dtypes must be f32/bf16");
  XFH_REQUIRE(!mask || mask_dtype == XFH_F32 || mask_dtype == XFH_BF16 || mask_dtype == XFH_BOOL,
              "msa_attention: bad mask dtype");
  if (rows == 0 || n == 0) return XFH_OK;
  XFH_REQUIRE(rows * n * c_msa < (int64_t(1) << 31) && n * n * c_pair < (int64_t(1) << 40) && n * n < (int64_t(1) << 31),
              "msa_attention: sizes must fit in 32 bits");
  XFH_REQUIRE(msa && pair && out && logits_w && v_w && gating_w && out_w, "msa_attention: null tensor");
  const bool packed = msa_packed_logits(n, c_pair, heads, dtype);
  Carver cv(workspace, workspace_bytes);
  MsaPlan p;
  const int64_t need = msa_carve(cv, p, rows, n, c_msa, c_pair, heads, dtype, packed);
  if (!workspace || need > workspace_bytes)
    return fail(XFH_EWORKSPACE, "msa_attention: workspace too small (need " + std::to_string(need) + " bytes)");
  hipStream_t s = as_stream(stream);
  const int64_t npad = align_up(n, int64_t(64));
  XFH_TRY(layer_norm_rows(msa, msa_dtype, rows * n, c_msa, ln_w, ln_b, ln_eps, p.normed, dtype, s));
  // logits(h, q, k) = Linear(LN(pair))[q][k][h]
  int logit_dtype;
  int64_t sh, sq, sk;
  float scale;
  if (packed) {
    PairBiasArgs pb;
    pb.pair = pair; pb.ln_w = pair_ln_w; pb.ln_b = pair_ln_b; pb.eps = pair_ln_eps;
    pb.w = static_cast<const bf16 *>(logits_w); pb.packed = p.logits; pb.packed_bf16 = 0;
    pb.n = int(n); pb.npad = int(npad); pb.heads = int(heads);
    XFH_TRY(pair_bias(pb, pair_dtype, s));
    logit_dtype = XFH_F32; sh = n * npad; sq = npad; sk = 1;
    scale = 0.6931471805599453f;                     // the packed logits are in log2 units
  } else {
    XFH_TRY(layer_norm_rows(pair, pair_dtype, n * n, c_pair, pair_ln_w, pair_ln_b, pair_ln_eps, p.pair_normed,
                            dtype, s));
    GemmArgs g = plain_gemm(p.pair_normed, c_pair, logits_w, c_pair, p.logits, heads, n * n, heads, c_pair);
    XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
    logit_dtype = dtype; sh = 1; sq = n * heads; sk = heads;
    scale = 1.0f;
  }
  msa_key_term_kernel<<<dim3(unsigned(ceil_div(n, 64))), 64 * kKeyTermWaves, 0, s>>>(mask, mask_dtype, int(rows),
                                                                                      int(n), p.kt);
  XFH_TRY(check_launch("msa_key_term"));
  const dim3 sgrid(unsigned(ceil_div(heads * n, 4)));
  if (dtype == XFH_BF16)
    msa_softmax_kernel<bf16><<<sgrid, 256, 0, s>>>(p.logits, logit_dtype, sh, sq, sk, scale, p.kt, int(heads), int(n),
                                                   int(npad), static_cast<bf16 *>(p.weights));
  else
    msa_softmax_kernel<float><<<sgrid, 256, 0, s>>>(p.logits, logit_dtype, sh, sq, sk, scale, p.kt, int(heads),
                                                    int(n), int(npad), static_cast<float *>(p.weights));
  XFH_TRY(check_launch("msa_softmax"));
  // vt[h][c][s n + k] = v_w[h dv + c] . LN(msa)[s][k]
  GemmArgs g = plain_gemm(v_w, c_msa, p.normed, c_msa, p.vt, rows * n, dv, rows * n, c_msa);
  g.sA = dv * c_msa; g.sB = 0; g.sC = dv * rows * n;
  XFH_TRY(gemm_nt(g, heads, dtype, dtype, false, s));
  // avg_t[h][q][c rows + s] = sum_k weights[h][q][k] vt[h][c][s n + k]
  g = plain_gemm(p.weights, npad, p.vt, n, p.avg_t, dv * rows, n, dv * rows, n);
  g.sA = n * npad; g.sB = dv * rows * n; g.sC = n * dv * rows;
  XFH_TRY(gemm_nt(g, heads, dtype, dtype, false, s));
  const dim3 ggrid(unsigned(n * heads), unsigned(ceil_div(rows, kGatherRows)));
  if (dtype == XFH_BF16)
    msa_gather_kernel<bf16><<<ggrid, kGatherRows, 0, s>>>(static_cast<const bf16 *>(p.avg_t), int(heads), int(n),
                                                          int(dv), int(rows), static_cast<bf16 *>(p.avg));
  else
    msa_gather_kernel<float><<<ggrid, kGatherRows, 0, s>>>(static_cast<const float *>(p.avg_t), int(heads), int(n),
                                                           int(dv), int(rows), static_cast<float *>(p.avg));
  XFH_TRY(check_launch("msa_gather"));
  // avg *= sigmoid(LN(msa) . gating_w^T), in place; out (+)= avg . out_w^T
  g = plain_gemm(p.normed, c_msa, gating_w, c_msa, p.avg, c_msa, rows * n, c_msa, c_msa);
  g.epi = XFH_EPI_SIGMOID_MUL_AUX; g.aux = p.avg; g.ldaux = c_msa;
  XFH_TRY(gemm_nt(g, 1, dtype, dtype, false, s));
  g = plain_gemm(p.avg, c_msa, out_w, c_msa, out, c_msa, rows * n, c_msa, c_msa);
  g.epi = accumulate ? XFH_EPI_ACCUMULATE : XFH_EPI_STORE;
  return gemm_nt(g, 1, dtype, out_dtype, false, s);
}

}  // extern "C"
