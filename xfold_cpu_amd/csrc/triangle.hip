// Triangle-multiplication gating kernel.
//
// From the two projection GEMM outputs P = LN(z) Wp^T and G = LN(z) Wg^T ([n*n, 2c] each,
// row-major) it forms mask * P * sigmoid(G) and de-interleaves channel 2k -> a_k and
// 2k+1 -> b_k (xfold/nn/triangle_multiplication.py:83-95). The results are written
// channel-major in the operand layouts of one "NT" batched GEMM per direction:
//   outgoing  out[k,i,j] = sum_t a[k,i,t] b[k,j,t]   -> left = a,   right = b
//   incoming  out[k,i,j] = sum_t a[k,t,j] b[k,t,i]   -> left = b^T, right = a^T
// so the contraction kernel always reads k-contiguous rows.
//
// The tiled kernel takes one grid line x and TILE consecutive positions y per workgroup: it
// reads those positions' P and G rows whole (16-byte pieces), forms a and b, parks them in
// LDS as [channel][position] and writes every channel's TILE outputs as one 128-byte run.
// The per-element kernel (one output element per thread, 2-byte reads strided by the row
// length) remains for rows that are not a multiple of 16 bytes.
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

// Workgroup (y tile, x): positions y0 .. y0 + TILE - 1 of grid line x, all c channel pairs.
template <typename T, int TILE>
__global__ __launch_bounds__(256) void trimul_gate_tiled_kernel(const T *__restrict__ proj,
                                                                const T *__restrict__ gate,
                                                                const void *__restrict__ mask,
                                                                int mask_dtype, int n, int c, int outgoing,
                                                                T *__restrict__ left, T *__restrict__ right) {
  constexpr int VEC = 16 / sizeof(T);              // elements per 16-byte piece (VEC / 2 channel pairs)
  constexpr int LDP = TILE + 1;                    // LDS row stride, elements
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T *ta = reinterpret_cast<T *>(smem), *tb = ta + int64_t(c) * LDP;
  const int x = blockIdx.y, y0 = blockIdx.x * TILE;
  const int cpr = 2 * c / VEC;                     // pieces per row
  for (int i = threadIdx.x; i < TILE * cpr; i += 256) {
    const int p = i / cpr, piece = i - p * cpr, y = y0 + p;
    if (y >= n) continue;
    const int64_t src = outgoing ? int64_t(x) * n + y : int64_t(y) * n + x;
    const float m = mask ? load_any(mask, mask_dtype, src) : 1.0f;
    const int64_t off = src * 2 * c + int64_t(piece) * VEC;
    alignas(16) T pv[VEC];
    alignas(16) T gv[VEC];
    *reinterpret_cast<uint4 *>(pv) = *reinterpret_cast<const uint4 *>(proj + off);
    *reinterpret_cast<uint4 *>(gv) = *reinterpret_cast<const uint4 *>(gate + off);
#pragma unroll
    for (int e = 0; e < VEC / 2; ++e) {
      const int k = piece * (VEC / 2) + e;
      ta[k * LDP + p] = from_f32<T>(to_f32(pv[2 * e]) * m * sigmoidf_(to_f32(gv[2 * e])));
      tb[k * LDP + p] = from_f32<T>(to_f32(pv[2 * e + 1]) * m * sigmoidf_(to_f32(gv[2 * e + 1])));
    }
  }
  __syncthreads();
  T *la = outgoing ? left : right, *lb = outgoing ? right : left;
  const int64_t plane = int64_t(n) * n;
  for (int i = threadIdx.x; i < c * TILE; i += 256) {
    const int k = i / TILE, p = i - k * TILE, y = y0 + p;
    if (y >= n) continue;
    const int64_t dst = k * plane + int64_t(x) * n + y;
    la[dst] = ta[k * LDP + p];
    lb[dst] = tb[k * LDP + p];
  }
}

}  // namespace

int trimul_gate(const void *proj, const void *gate, int dtype, const void *mask, int mask_dtype,
                int64_t n, int64_t c, int outgoing, void *a_out, void *b_out, hipStream_t s) {
  const int64_t total = n * n * c;
  if (total == 0) return XFH_OK;
  // Tiled: whole 16-byte pieces per row, 128-byte output runs, LDS within 64 KB.
  const int es = dtype == XFH_BF16 ? 2 : 4, tile = 128 / es;
  const int64_t lds = 2 * c * (tile + 1) * es;
  if ((2 * c * es) % 16 == 0 && lds <= 65536 && n <= 65535 &&
      reinterpret_cast<uintptr_t>(proj) % 16 == 0 && reinterpret_cast<uintptr_t>(gate) % 16 == 0) {
    const dim3 tgrid(unsigned(ceil_div(n, tile)), unsigned(n));
    if (dtype == XFH_BF16)
      trimul_gate_tiled_kernel<bf16, 64><<<tgrid, 256, size_t(lds), s>>>(
          (const bf16 *)proj, (const bf16 *)gate, mask, mask_dtype, int(n), int(c), outgoing, (bf16 *)a_out,
          (bf16 *)b_out);
    else
      trimul_gate_tiled_kernel<float, 32><<<tgrid, 256, size_t(lds), s>>>(
          (const float *)proj, (const float *)gate, mask, mask_dtype, int(n), int(c), outgoing, (float *)a_out,
          (float *)b_out);
    return check_launch("trimul_gate");
  }
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
