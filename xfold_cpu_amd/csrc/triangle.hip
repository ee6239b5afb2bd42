// Triangle-multiplication gating kernel.
//
// From the two projection GEMM outputs P = LN(z) Wp^T and G = LN(z) Wg^T ([n*n, 2c] each,
// row-major) it forms mask * P * sigmoid(G) and de-interleaves channel 2k -> a_k and
// 2k+1 -> b_k (xfold/nn/triangle_multiplication.py:83-95). The results are written
// channel-major in the operand layouts of one "NT" batched GEMM per direction:
//   outgoing  out[k,i,j] = sum_t a[k,i,t] b[k,j,t]   -> left = a,   right = b
//   incoming  out[k,i,j] = sum_t a[k,t,j] b[k,t,i]   -> left = b^T, right = a^T
// so the contraction kernel always reads k-contiguous rows.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void trimul_gate_kernel(const T *__restrict__ proj,
                                                          const T *__restrict__ gate,
                                                          const void *__restrict__ mask,
                                                          int mask_dtype, int64_t n, int64_t c,
                                                          int outgoing, T *__restrict__ left,
                                                          T *__restrict__ right) {
  const int64_t plane = n * n;
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= plane * c) return;
  const int64_t k = idx / plane, rem = idx % plane;
  const int64_t x = rem / n, y = rem % n;
  // Output element [k, x, y]; its source pair position is (x, y) outgoing, (y, x) incoming.
  const int64_t src = outgoing ? x * n + y : y * n + x;
  const float m = mask ? load_any(mask, mask_dtype, src) : 1.0f;
  const T *pr = proj + src * 2 * c + 2 * k;
  const T *gr = gate + src * 2 * c + 2 * k;
  const float a = to_f32(pr[0]) * m * sigmoidf_(to_f32(gr[0]));
  const float b = to_f32(pr[1]) * m * sigmoidf_(to_f32(gr[1]));
  left[idx] = from_f32<T>(outgoing ? a : b);
  right[idx] = from_f32<T>(outgoing ? b : a);
}

}  // namespace

int trimul_gate(const void *proj, const void *gate, int dtype, const void *mask, int mask_dtype,
                int64_t n, int64_t c, int outgoing, void *a_out, void *b_out, hipStream_t s) {
  const int64_t total = n * n * c;
  if (total == 0) return XFH_OK;
  dim3 grid(ceil_div(total, 256));
  if (dtype == XFH_BF16)
    trimul_gate_kernel<bf16><<<grid, 256, 0, s>>>((const bf16 *)proj, (const bf16 *)gate, mask,
                                                  mask_dtype, n, c, outgoing, (bf16 *)a_out,
                                                  (bf16 *)b_out);
  else
    trimul_gate_kernel<float><<<grid, 256, 0, s>>>((const float *)proj, (const float *)gate, mask,
                                                   mask_dtype, n, c, outgoing, (float *)a_out,
                                                   (float *)b_out);
  return check_launch("trimul_gate");
}

}  // namespace xfh
