// Register-resident building blocks for the pair-stack kernels whose inputs and outputs
// are [positions][128 channels] rows (bf16 compute, K = 128).
//
// A wavefront works on 16 positions at a time ("step") with no LDS traffic for its
// activations and no barriers: lane l handles position l % 16 and channel group
// g = l / 16, and the activations live in one of two register layouts:
//   K-layout: channels 32 ks + 8 g + j (ks < 4, j < 8), the MFMA operand layout with
//             k = channels (a lane supplies 8 consecutive k per 16x16x32 step);
//   O-layout: channels 16 t + 4 g + e (t < 8, e < 4), the layout of a 16x16 MFMA result
//             tile whose columns are positions and whose rows are channels.
// An O-layout set is also a valid MFMA k-operand if the other operand lists its k in the
// order kperm(ks, g, j) below (tiles 2 ks and 2 ks + 1 side by side), so a result feeds
// the next GEMM without leaving the registers.
//
// Weights W[128 out][128 in] (nn.Linear layout) sit in LDS for the workgroup's lifetime,
// 256-byte rows with 16-byte chunk c of row n stored at chunk c ^ (n & 15), optionally with
// their input channels in kperm order. out^T[n][pos] = sum_k W[n][k] x[pos][k] then takes
// W as the A operand (row n = 16 t + l % 16) and x as the B operand, and lands in O-layout.
#pragma once

#include "common.h"

namespace xfh {
namespace rowstep {

constexpr int C = 128;                  // channels
constexpr int W_ELEMS = C * C;          // one weight matrix in LDS (bf16, 32 KB)

// Input channel of MFMA k-slot (ks, g, j) when the operand is an O-layout register set.
__host__ __device__ constexpr int kperm(int ks, int g, int j) {
  return j < 4 ? 32 * ks + 4 * g + j : 32 * ks + 16 + 4 * g + (j - 4);
}

// Weight rows ([rows][128] bf16, row-major) on their way into LDS with the chunk swizzle:
// load() issues every global load of the calling thread, store() writes them, so the copy
// costs one memory round trip (a loop that stores each chunk before loading the next pays
// one per iteration). Work is spread over T threads (the workgroup size); `src(row)` gives
// the row's source, or nullptr for a row of zeros; `permuted` reorders each row's input
// channels to kperm order.
template <int ROWS, int T> struct WeightStage {
  static constexpr int N = (ROWS * 16 + T - 1) / T;   // chunks per thread
  bf16x8 v[N];
  template <class Src> __device__ __forceinline__ void load(Src src, bool permuted) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int i = int(threadIdx.x) + j * T;
      v[j] = bf16x8{};
      if (i >= ROWS * 16) continue;
      const int n = i >> 4, c = i & 15;             // row, logical chunk
      const bf16 *w = src(n);
      if (!w) continue;
      if (permuted) {
        const int ks = c >> 2, g = c & 3;
        const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(w + kperm(ks, g, 0));
        const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(w + kperm(ks, g, 4));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[j][e] = lo[e];
          v[j][4 + e] = hi[e];
        }
      } else {
        v[j] = *reinterpret_cast<const bf16x8 *>(w + c * 8);
      }
    }
  }
  __device__ __forceinline__ void store(bf16 *dst) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int i = int(threadIdx.x) + j * T;
      if (i >= ROWS * 16) continue;
      const int n = i >> 4, c = i & 15;
      *reinterpret_cast<bf16x8 *>(dst + n * C + ((c ^ (n & 15)) * 8)) = v[j];
    }
  }
};

// Fragment of W for output tile t, k-step ks (lane: row 16 t + l % 16, chunk 4 ks + g):
// the A operand of out^T = W . x^T, or the B operand of out = x . W^T (same lane layout).
__device__ __forceinline__ bf16x8 weight_frag(const bf16 *w_lds, int t, int ks) {
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int n = 16 * t + r;
  return *reinterpret_cast<const bf16x8 *>(w_lds + n * C + (((4 * ks + g) ^ r) * 8));
}

// out^T tiles: acc[t] (+)= sum_ks W(t, ks) . x[ks]; x is a K-layout (or, with a permuted W,
// an O-layout) bf16 operand.
__device__ __forceinline__ void gemm_t(const bf16 *w_lds, const bf16x8 (&x)[4], f32x4 (&acc)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc[t] = mfma16(weight_frag(w_lds, t, ks), x[ks], acc[t]);
}

// out tile: acc (+)= sum_ks x[ks] . W(t, ks) — rows are positions, columns the 16 output
// channels of tile t; a lane ends up with 4 consecutive positions (4 g .. +3) of channel
// 16 t + l % 16.
__device__ __forceinline__ void gemm_n(const bf16 *w_lds, int t, const bf16x8 (&x)[4], f32x4 &acc) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) acc = mfma16(x[ks], weight_frag(w_lds, t, ks), acc);
}

// Sum over the four lanes of one position (l, l ^ 16, l ^ 32, l ^ 48). The swap results
// pass through an empty asm: the compiler otherwise folds arithmetic on the two results
// of one swap as if they were equal.
__device__ __forceinline__ float position_sum(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  uint32_t p0 = p[0], p1 = p[1];
  asm volatile("" : "+v"(p0), "+v"(p1));
  x = __builtin_bit_cast(float, p0) + __builtin_bit_cast(float, p1);
  u = __builtin_bit_cast(uint32_t, x);
  const auto q = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  uint32_t q0 = q[0], q1 = q[1];
  asm volatile("" : "+v"(q0), "+v"(q1));
  return __builtin_bit_cast(float, q0) + __builtin_bit_cast(float, q1);
}

// LayerNorm statistics of a position from this lane's 32 channels (fp32, two passes).
__device__ __forceinline__ void ln_stats(const float (&v)[32], float eps, float &mean, float &rstd) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) s += v[i];
  mean = position_sum(s) * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float d = v[i] - mean;
    q += d * d;
  }
  rstd = rsqrtf(position_sum(q) * (1.0f / C) + eps);
}

// Loads 8 consecutive channels of a row as floats.
template <typename T> __device__ __forceinline__ void load8f(const T *p, float *o);
template <> __device__ __forceinline__ void load8f<bf16>(const bf16 *p, float *o) {
  const bf16x8 v = *reinterpret_cast<const bf16x8 *>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = static_cast<float>(v[i]);
}
template <> __device__ __forceinline__ void load8f<float>(const float *p, float *o) {
  const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
template <typename T> __device__ __forceinline__ void load4f(const T *p, float *o);
template <> __device__ __forceinline__ void load4f<bf16>(const bf16 *p, float *o) {
  const bf16x4 v = *reinterpret_cast<const bf16x4 *>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = static_cast<float>(v[i]);
}
template <> __device__ __forceinline__ void load4f<float>(const float *p, float *o) {
  const float4 a = *reinterpret_cast<const float4 *>(p);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
}
template <typename T> __device__ __forceinline__ void store4f(T *p, const float *v);
template <> __device__ __forceinline__ void store4f<bf16>(bf16 *p, const float *v) {
  bf16x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = bf16(v[i]);
  *reinterpret_cast<bf16x4 *>(p) = o;
}
template <> __device__ __forceinline__ void store4f<float>(float *p, const float *v) {
  *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

// Four consecutive channels as loaded (bf16x4 or float4), converted only when used, so
// that loads can be issued early without holding fp32 copies.
template <typename T> struct Raw4;
template <> struct Raw4<bf16> {
  bf16x4 v;
  __device__ __forceinline__ void load(const bf16 *p) { v = *reinterpret_cast<const bf16x4 *>(p); }
  __device__ __forceinline__ float operator[](int i) const { return static_cast<float>(v[i]); }
};
template <> struct Raw4<float> {
  float4 v;
  __device__ __forceinline__ void load(const float *p) { v = *reinterpret_cast<const float4 *>(p); }
  __device__ __forceinline__ float operator[](int i) const { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
};

// K-layout row as loaded: r[2 ks + h] = channels 32 ks + 8 g + 4 h .. +3.
template <typename T> __device__ __forceinline__ void load_k(const T *row, Raw4<T> (&r)[8]) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    r[2 * ks].load(row + 32 * ks + 8 * g);
    r[2 * ks + 1].load(row + 32 * ks + 8 * g + 4);
  }
}
template <typename T> __device__ __forceinline__ void k_to_float(const Raw4<T> (&r)[8], float (&v)[32]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * i + e] = r[i][e];
}
// O-layout row as loaded: r[t] = channels 16 t + 4 g .. +3.
template <typename T> __device__ __forceinline__ void load_o(const T *row, Raw4<T> (&r)[8]) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t].load(row + 16 * t + 4 * g);
}

// LayerNorm of a K-layout position (affine parameters from LDS, fp32) to bf16 operands.
__device__ __forceinline__ void ln_k(float (&v)[32], const float *lnw, const float *lnb, float eps,
                                     bf16x8 (&x)[4]) {
  const int g = (threadIdx.x & 63) >> 4;
  float mean, rstd;
  ln_stats(v, eps, mean, rstd);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const float4 w0 = *reinterpret_cast<const float4 *>(lnw + 32 * ks + 8 * g);
    const float4 w1 = *reinterpret_cast<const float4 *>(lnw + 32 * ks + 8 * g + 4);
    const float4 b0 = *reinterpret_cast<const float4 *>(lnb + 32 * ks + 8 * g);
    const float4 b1 = *reinterpret_cast<const float4 *>(lnb + 32 * ks + 8 * g + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) x[ks][j] = bf16((v[8 * ks + j] - mean) * rstd * wv[j] + bv[j]);
  }
}

// Optional LayerNorm affine parameters (fp32[128], nullptr: 1 / 0) on their way into LDS,
// split like WeightStage; the workgroup has at least 128 threads.
struct LnStage {
  float w, b;
  __device__ __forceinline__ void load(const float *wp, const float *bp) {
    const int i = int(threadIdx.x);
    w = 1.f;
    b = 0.f;
    if (i < C) {
      if (wp) w = wp[i];
      if (bp) b = bp[i];
    }
  }
  __device__ __forceinline__ void store(float *w_lds, float *b_lds) const {
    if (threadIdx.x < C) {
      w_lds[threadIdx.x] = w;
      b_lds[threadIdx.x] = b;
    }
  }
};

// Identity fragments: as the A operand with a K-layout operand x[ks] as B, half h
// (0 or 1) gives O-layout tile t = 2 ks + h exactly (one nonzero product per output), so
// one MFMA both converts 16 bf16 channels per position to fp32 and moves them into O-layout.
__device__ __forceinline__ void identity_frags(bf16x8 (&id)[2]) {
  const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) id[h][j] = (8 * g + j == m + 16 * h) ? bf16(1.0f) : bf16(0.0f);
}
__device__ __forceinline__ void k_to_o(const bf16x8 (&id)[2], const bf16x8 (&x)[4], f32x4 (&o)[8]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int h = 0; h < 2; ++h) o[2 * ks + h] = mfma16(id[h], x[ks], f32x4{0.f, 0.f, 0.f, 0.f});
}

// Pairs the O-layout values of tiles 2 ks and 2 ks + 1 into k-operand ks (kperm order).
__device__ __forceinline__ void o_to_operand(const float (&y)[8][4], bf16x8 (&x)[4]) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[ks][e] = bf16(y[2 * ks][e]);
      x[ks][4 + e] = bf16(y[2 * ks + 1][e]);
    }
}

// Swap of `hi` across the two 32-lane halves (permlane32_swap: vdst's lanes 32-63 trade
// places with src0's lanes 0-31) or across rows 0/1 and 2/3 (permlane16_swap: vdst's odd
// rows trade places with src0's even rows). The results pass through an empty asm, as in
// position_sum.
__device__ __forceinline__ void swap32(uint32_t &vdst, uint32_t &src0) {
  const auto r = __builtin_amdgcn_permlane32_swap(vdst, src0, false, false);
  uint32_t a = r[0], b = r[1];
  asm volatile("" : "+v"(a), "+v"(b));
  vdst = a;
  src0 = b;
}
__device__ __forceinline__ void swap16(uint32_t &vdst, uint32_t &src0) {
  const auto r = __builtin_amdgcn_permlane16_swap(vdst, src0, false, false);
  uint32_t a = r[0], b = r[1];
  asm volatile("" : "+v"(a), "+v"(b));
  vdst = a;
  src0 = b;
}

// One k-step of a kperm-ordered operand (lane group g holds channels 32 ks + 4 g .. +3 in
// elements 0-3 and 32 ks + 16 + 4 g .. +3 in 4-7) into K-layout (lane group g holds
// 32 ks + 8 g .. + 7), in place. With g = 2 hi + lo, piece a (elements 0-3 or 4-7) of lane
// group 2 c + e belongs to lane group 2 a + c as its piece e: one swap across the halves
// moves piece a to half a, one swap across rows moves it to row c.
__device__ __forceinline__ void o_to_k_step(bf16x8 &x) {
  uint4 d = __builtin_bit_cast(uint4, x);
  swap32(d.x, d.z);                       // lower half: piece 0 of both halves,
  swap32(d.y, d.w);                       // upper half: piece 1 of both halves
  swap16(d.x, d.z);                       // row c: piece a of lane groups 2 c, 2 c + 1
  swap16(d.y, d.w);
  x = __builtin_bit_cast(bf16x8, d);
}

// O-layout tiles 2 ks and 2 ks + 1 (4 values each) as k-step ks of a kperm-ordered operand
// (one step of o_to_operand).
__device__ __forceinline__ bf16x8 pack_tiles(const float (&lo)[4], const float (&hi)[4]) {
  bf16x8 x;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = bf16(lo[e]);
    x[4 + e] = bf16(hi[e]);
  }
  return x;
}

}  // namespace rowstep
}  // namespace xfh
