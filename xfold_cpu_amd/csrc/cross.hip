// Two small elementwise entry points:
//   xfh_cross_attention_bias: the attention bias of the atom CrossAttention
//     (xfold/nn/diffusion_transformer.py:318-339),
//       out[b][h][q][k] = pair_logits[b][h][q][k] + 1e9 * (mask_q[b][q] == 0 && mask_k[b][k] == 0)
//     in fp32, the logits' additive term in front of xfh_dot_product_attention. The 1e9 term
//     is the reference's: positive, on the pairs where both the query and the key are
//     masked, so a masked query attends to the masked keys and an unmasked query to every
//     key. One thread per 4 consecutive keys of one (b, h, q): the 16-byte fp32 stores of a
//     wavefront cover 1 KB of the output in row-major order.
//   xfh_convert: an activation's dtype change (fp32 <-> bf16), the cast torch.autocast puts
//     in front of a Linear, done here so that no per-call torch kernel remains on the path.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

__global__ __launch_bounds__(256) void cross_bias_kernel(const void *__restrict__ logits, int logits_dtype,
                                                         int64_t sb, int64_t sh, int64_t sq, int64_t sk,
                                                         const void *__restrict__ mask_q, int mq_dtype,
                                                         const void *__restrict__ mask_k, int mk_dtype,
                                                         int64_t batch, int64_t heads, int64_t nq, int64_t nk,
                                                         float *__restrict__ out) {
  const int64_t quads = (nk + 3) / 4;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= batch * heads * nq * quads) return;
  const int64_t k0 = (idx % quads) * 4, row = idx / quads;
  const int64_t q = row % nq, bh = row / nq, h = bh % heads, b = bh / heads;
  const bool q_masked = mask_q && load_any(mask_q, mq_dtype, b * nq + q) == 0.f;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t k = k0 + e;
    float x = 0.f;
    if (k < nk) {
      if (logits) x = load_any(logits, logits_dtype, b * sb + h * sh + q * sq + k * sk);
      if (q_masked && mask_k && load_any(mask_k, mk_dtype, b * nk + k) == 0.f) x += 1e9f;
    }
    v[e] = x;
  }
  float *dst = out + row * nk + k0;
  if (nk % 4 == 0) {
    *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (k0 + e < nk) dst[e] = v[e];
  }
}

bool mask_ok(int d) { return d == XFH_F32 || d == XFH_BF16 || d == XFH_BOOL; }

// y = x in another float dtype (round to nearest even into bf16), 8 elements per thread.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void convert_kernel(const TI *__restrict__ x, TO *__restrict__ y, int64_t n) {
  const int64_t i0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (i0 + e < n) y[i0 + e] = static_cast<TO>(static_cast<float>(x[i0 + e]));
}

}  // namespace

}  // namespace xfh

using namespace xfh;

extern "C" int xfh_cross_attention_bias(const void *pair_logits, int logits_dtype, const int64_t *strides,
                                        const void *mask_q, int mask_q_dtype, const void *mask_k, int mask_k_dtype,
                                        int64_t batch, int64_t heads, int64_t nq, int64_t nk, float *out,
                                        void *stream) {
  XFH_REQUIRE(batch >= 0 && heads >= 0 && nq >= 0 && nk >= 0, "cross_attention_bias: bad size");
  XFH_REQUIRE(!pair_logits || ((logits_dtype == XFH_F32 || logits_dtype == XFH_BF16) && strides),
              "cross_attention_bias: pair logits must be f32/bf16 with strides");
  XFH_REQUIRE((!mask_q || mask_ok(mask_q_dtype)) && (!mask_k || mask_ok(mask_k_dtype)),
              "cross_attention_bias: bad mask dtype");
  const int64_t total = batch * heads * nq * ceil_div(nk, 4);
  if (total == 0) return XFH_OK;
  XFH_REQUIRE(out && reinterpret_cast<uintptr_t>(out) % 16 == 0, "cross_attention_bias: out must be 16-byte aligned");
  const int64_t sb = pair_logits ? strides[0] : 0, sh = pair_logits ? strides[1] : 0;
  const int64_t sq = pair_logits ? strides[2] : 0, sk = pair_logits ? strides[3] : 0;
  cross_bias_kernel<<<dim3(unsigned(ceil_div(total, 256))), 256, 0, as_stream(stream)>>>(
      pair_logits, logits_dtype, sb, sh, sq, sk, mask_q, mask_q_dtype, mask_k, mask_k_dtype, batch, heads, nq, nk,
      out);
  return check_launch("cross_attention_bias");
}

extern "C" int xfh_convert(const void *x, int x_dtype, void *y, int y_dtype, int64_t n, void *stream) {
  XFH_REQUIRE(n >= 0, "convert: bad size");
  XFH_REQUIRE((x_dtype == XFH_F32 || x_dtype == XFH_BF16) && (y_dtype == XFH_F32 || y_dtype == XFH_BF16),
              "convert: dtypes must be f32/bf16");
  if (n == 0) return XFH_OK;
  XFH_REQUIRE(x && y, "convert: null tensor");
  const dim3 grid(unsigned(ceil_div(ceil_div(n, 8), 256)));
  hipStream_t s = as_stream(stream);
  if (x_dtype == XFH_F32 && y_dtype == XFH_BF16)
    convert_kernel<float, bf16><<<grid, 256, 0, s>>>(static_cast<const float *>(x), static_cast<bf16 *>(y), n);
  else if (x_dtype == XFH_BF16 && y_dtype == XFH_F32)
    convert_kernel<bf16, float><<<grid, 256, 0, s>>>(static_cast<const bf16 *>(x), static_cast<float *>(y), n);
  else if (x_dtype == XFH_F32)
    convert_kernel<float, float><<<grid, 256, 0, s>>>(static_cast<const float *>(x), static_cast<float *>(y), n);
  else
    convert_kernel<bf16, bf16><<<grid, 256, 0, s>>>(static_cast<const bf16 *>(x), static_cast<bf16 *>(y), n);
  return check_launch("convert");
}
