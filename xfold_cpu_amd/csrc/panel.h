// Row-panel building blocks for the fused pair-stack kernels (bf16 compute, K = 128).
//
// A workgroup of 256 threads (4 wavefronts in a 2 x 2 grid) owns a panel of 128 rows of
// 128 channels. The panel is normalised once into an LDS tile, each wavefront lifts its
// 64 rows into registers as MFMA A fragments, and the weight matrix ([out, 128], nn.Linear
// layout) streams through LDS in chunks of 64 output columns, double-buffered, so every
// panel is read from HBM exactly once whatever the number of outputs. A chunk gives each
// wavefront a 64 x 32 block of results (4 x 2 MFMA 16x16 tiles) in fp32.
#pragma once

#include "common.h"

namespace xfh {
namespace panel {

constexpr int ROWS = 128;            // rows per panel
constexpr int K = 128;               // channels (reduction dim)
constexpr int CHUNK = 64;            // output columns per weight chunk
constexpr int PITCH = K + 8;         // LDS row pitch (bf16) of A and B tiles: 272 bytes
constexpr int A_ELEMS = ROWS * PITCH;
constexpr int B_ELEMS = CHUNK * PITCH;

// The 8 affine parameters a lane applies (channels sub*8 .. sub*8+7), loaded once.
struct LnParams {
  float w[8], b[8];
};

__device__ __forceinline__ void load_ln_params(const float *w, const float *b, int sub, LnParams &p) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p.w[i] = 1.f;
    p.b[i] = 0.f;
  }
  if (w) {
    const float4 lo = reinterpret_cast<const float4 *>(w + sub * 8)[0];
    const float4 hi = reinterpret_cast<const float4 *>(w + sub * 8)[1];
    p.w[0] = lo.x; p.w[1] = lo.y; p.w[2] = lo.z; p.w[3] = lo.w;
    p.w[4] = hi.x; p.w[5] = hi.y; p.w[6] = hi.z; p.w[7] = hi.w;
  }
  if (b) {
    const float4 lo = reinterpret_cast<const float4 *>(b + sub * 8)[0];
    const float4 hi = reinterpret_cast<const float4 *>(b + sub * 8)[1];
    p.b[0] = lo.x; p.b[1] = lo.y; p.b[2] = lo.z; p.b[3] = lo.w;
    p.b[4] = hi.x; p.b[5] = hi.y; p.b[6] = hi.z; p.b[7] = hi.w;
  }
}

// LayerNorm of one 128-channel row held by 16 lanes (8 channels each, fp32 statistics),
// written to the LDS A tile as bf16. `x` holds the lane's 8 inputs.
__device__ __forceinline__ void ln_row_to_lds(float x[8], const LnParams &p, float eps, int sub,
                                              bf16 *dst_row) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
  s = group_sum<16>(s);
  const float mean = s * (1.0f / K);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x[i] -= mean;
    q += x[i] * x[i];
  }
  q = group_sum<16>(q);
  const float rstd = rsqrtf(q * (1.0f / K) + eps);
  bf16x8 o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = bf16(x[i] * rstd * p.w[i] + p.b[i]);
  *reinterpret_cast<bf16x8 *>(dst_row + sub * 8) = o;
}

template <typename T> __device__ __forceinline__ void load8(const T *p, float *o);
template <> __device__ __forceinline__ void load8<bf16>(const bf16 *p, float *o) {
  const bf16x8 v = *reinterpret_cast<const bf16x8 *>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = static_cast<float>(v[i]);
}
template <> __device__ __forceinline__ void load8<float>(const float *p, float *o) {
  const float4 a = reinterpret_cast<const float4 *>(p)[0];
  const float4 c = reinterpret_cast<const float4 *>(p)[1];
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = c.x; o[5] = c.y; o[6] = c.z; o[7] = c.w;
}

// Normalises the panel rows into `a_tile` ([ROWS][PITCH] bf16). row_ptr(r) gives the
// address of row r's 128 channels, or nullptr for rows past the end (zero-filled).
// Each wavefront handles 4 rows per pass; loads for all 8 passes are issued first.
template <typename TIN, typename RowPtr>
__device__ __forceinline__ void ln_panel(RowPtr row_ptr, const float *w, const float *b, float eps,
                                         bf16 *a_tile) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane & 15, rsub = lane >> 4;
  LnParams prm;
  load_ln_params(w, b, sub, prm);
  float x[8][8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int r = p * 16 + wave * 4 + rsub;
    const TIN *src = row_ptr(r);
    if (src) {
      load8<TIN>(src + sub * 8, x[p]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[p][i] = 0.f;
    }
  }
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int r = p * 16 + wave * 4 + rsub;
    ln_row_to_lds(x[p], prm, eps, sub, a_tile + r * PITCH);
  }
}

// A fragments of a wavefront's 64 rows: frag[mt][ks] = rows wm*64 + mt*16 + (l%16),
// k = ks*32 + 8*(l/16) .. +8.
struct AFrags {
  bf16x8 f[4][4];
};

__device__ __forceinline__ void load_a_frags(const bf16 *a_tile, int wm, AFrags &a) {
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      a.f[mt][ks] = *reinterpret_cast<const bf16x8 *>(a_tile + (wm * 64 + mt * 16 + col) * PITCH + ks * 32 + grp * 8);
}

// Register staging of one weight chunk: rows [n0, n0+64) of W ([n_total, 128] bf16),
// 16 KB = 4 x 16 bytes per thread. Rows >= n_total are zero.
struct BStage {
  uint4 v[4];
};

__device__ __forceinline__ void fetch_b(const bf16 *W, int n0, int n_total, BStage &st) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + i * 256;           // 1024 chunks of 16 bytes
    const int r = idx >> 4, c = (idx & 15) * 8;
    st.v[i] = (n0 + r < n_total) ? *reinterpret_cast<const uint4 *>(W + int64_t(n0 + r) * K + c)
                                 : make_uint4(0, 0, 0, 0);
  }
}

// The same staging for a weight given row by row: row_ptr(r) is the address of row r's
// 128 inputs, or nullptr for a zero row (lets a kernel read several nn.Linear weights as
// one packed matrix without packing them first).
template <typename RowPtr>
__device__ __forceinline__ void fetch_rows(RowPtr row_ptr, int n0, BStage &st) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + i * 256;
    const int r = idx >> 4, c = (idx & 15) * 8;
    const bf16 *src = row_ptr(n0 + r);
    st.v[i] = src ? *reinterpret_cast<const uint4 *>(src + c) : make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ void stash_b(const BStage &st, bf16 *b_tile) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + i * 256;
    const int r = idx >> 4, c = (idx & 15) * 8;
    *reinterpret_cast<uint4 *>(b_tile + r * PITCH + c) = st.v[i];
  }
}

// acc[mt][nt] += A(rows wm*64+mt*16) . B(cols wn*32+nt*16)^T over K = 128.
__device__ __forceinline__ void mma_chunk(const AFrags &a, const bf16 *b_tile, int wn, f32x4 acc[4][2]) {
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    bf16x8 bf[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
      bf[nt] = *reinterpret_cast<const bf16x8 *>(b_tile + (wn * 32 + nt * 16 + col) * PITCH + ks * 32 + grp * 8);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma16(a.f[mt][ks], bf[nt], acc[mt][nt]);
  }
}

__device__ __forceinline__ void zero(f32x4 acc[4][2]) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
}

}  // namespace panel
}  // namespace xfh
