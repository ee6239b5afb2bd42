// LayerNorm kernels: row-major rows (pair / single / diffusion activations) and
// channel-major planes (the triangle-multiplication centre norm).
//
// Row kernel: a row of C elements is owned by LPR consecutive lanes; each lane holds
// CHUNKS vectors of 8 elements (one 16-byte load for bf16, two for fp32), so every
// global access is a 128-bit load or store and the statistics need only log2(LPR)
// butterfly steps inside the wavefront. Statistics are fp32 and two-pass (mean, then
// the mean of squared deviations) from registers, matching F.layer_norm's biased
// variance (xfold/fastnn/layer_norm.py:56-59).
#include <type_traits>

#include "common.h"

namespace xfh {

template <typename T> struct Vec8;
template <> struct Vec8<bf16> {
  __device__ static void load(const bf16 *p, float *o) {
    bf16x8 v = *reinterpret_cast<const bf16x8 *>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = static_cast<float>(v[i]);
  }
  __device__ static void store(bf16 *p, const float *o) {
    bf16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<bf16>(o[i]);
    *reinterpret_cast<bf16x8 *>(p) = v;
  }
};
template <> struct Vec8<float> {
  __device__ static void load(const float *p, float *o) {
    float4 a = reinterpret_cast<const float4 *>(p)[0];
    float4 b = reinterpret_cast<const float4 *>(p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
  __device__ static void store(float *p, const float *o) {
    reinterpret_cast<float4 *>(p)[0] = make_float4(o[0], o[1], o[2], o[3]);
    reinterpret_cast<float4 *>(p)[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
};

// MODE 0: plain (optional affine). MODE 1: adaptive (sigmoid(scale) * xhat + shift).
template <typename TI, typename TO, typename TA, int LPR, int CHUNKS, int MODE>
__global__ __launch_bounds__(256) void ln_rows_vec(const TI *__restrict__ x, int64_t rows,
                                                   const float *__restrict__ w,
                                                   const float *__restrict__ b,
                                                   const TA *__restrict__ scale,
                                                   const TA *__restrict__ shift, int64_t cond_rows,
                                                   float eps, TO *__restrict__ y) {
  constexpr int C = LPR * CHUNKS * 8;
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPR;
  const int64_t row = (int64_t(blockIdx.x) * 256 + threadIdx.x) / LPR;
  if (row >= rows) return;
  const TI *xr = x + row * C;
  float v[CHUNKS][8];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    Vec8<TI>::load(xr + (c * LPR + sub) * 8, v[c]);
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[c][i];
  }
  s = group_sum<LPR>(s);
  const float mean = s * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[c][i] -= mean;
      q += v[c][i] * v[c][i];
    }
  q = group_sum<LPR>(q);
  const float rstd = rsqrtf(q * (1.0f / C) + eps);
  TO *yr = y + row * C;
  const int64_t crow = MODE == 1 ? (row % cond_rows) * C : 0;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int base = (c * LPR + sub) * 8;
    float o[8];
    if (MODE == 1) {
      float sc[8], sh[8];
      Vec8<TA>::load(scale + crow + base, sc);
      Vec8<TA>::load(shift + crow + base, sh);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = sigmoidf_(sc[i]) * (v[c][i] * rstd) + sh[i];
    } else {
      float wv[8], bv[8];
      if (w) {
        Vec8<float>::load(w + base, wv);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) wv[i] = 1.f;
      }
      if (b) {
        Vec8<float>::load(b + base, bv);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) bv[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = v[c][i] * rstd * wv[i] + bv[i];
    }
    Vec8<TO>::store(yr + base, o);
  }
}

// Generic fallback: one wavefront per row, any C, statistics re-read from memory.
template <typename TI, typename TO, typename TA, int MODE>
__global__ __launch_bounds__(256) void ln_rows_any(const TI *__restrict__ x, int64_t rows, int64_t C,
                                                   const float *__restrict__ w,
                                                   const float *__restrict__ b,
                                                   const TA *__restrict__ scale,
                                                   const TA *__restrict__ shift, int64_t cond_rows,
                                                   float eps, TO *__restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t(blockIdx.x) * 256 + threadIdx.x) / 64;
  if (row >= rows) return;
  const TI *xr = x + row * C;
  float s = 0.f;
  for (int64_t c = lane; c < C; c += 64) s += to_f32(xr[c]);
  const float mean = wave_sum(s) / float(C);
  float q = 0.f;
  for (int64_t c = lane; c < C; c += 64) {
    float d = to_f32(xr[c]) - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(wave_sum(q) / float(C) + eps);
  TO *yr = y + row * C;
  const int64_t crow = MODE == 1 ? (row % cond_rows) * C : 0;
  for (int64_t c = lane; c < C; c += 64) {
    float t = (to_f32(xr[c]) - mean) * rstd;
    if (MODE == 1) {
      t = sigmoidf_(to_f32(scale[crow + c])) * t + to_f32(shift[crow + c]);
    } else {
      if (w) t *= w[c];
      if (b) t += b[c];
    }
    yr[c] = from_f32<TO>(t);
  }
}

// Channel-major input: element (r, c) at x[c * plane + r]; output row-major y[r * C + c].
// One thread per row; neighbouring threads read neighbouring addresses for each channel.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void ln_planes(const TI *__restrict__ x, int64_t plane, int C,
                                                 const float *__restrict__ w,
                                                 const float *__restrict__ b, float eps,
                                                 TO *__restrict__ y) {
  const int64_t r = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (r >= plane) return;
  float s = 0.f;
  for (int c = 0; c < C; ++c) s += to_f32(x[c * plane + r]);
  const float mean = s / float(C);
  float q = 0.f;
  for (int c = 0; c < C; ++c) {
    float d = to_f32(x[c * plane + r]) - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(q / float(C) + eps);
  for (int c = 0; c < C; ++c) {
    float t = (to_f32(x[c * plane + r]) - mean) * rstd;
    if (w) t *= w[c];
    if (b) t += b[c];
    y[r * C + c] = from_f32<TO>(t);
  }
}

// The same through LDS for C <= kPlanesMaxC: a workgroup takes 64 rows, reads each plane's
// 64-element run of them (coalesced), keeps the [C][64] tile in LDS for the two passes of
// statistics (4 channel groups per row, summed in LDS) and writes the 64 rows' contiguous
// channel vectors (coalesced), instead of one thread per row storing with a stride of C.
// The tile is sized for at most MAXC channels (64, 128 or 256), so narrow pairs keep more
// workgroups per CU in flight (C = 64: 16.6 KB each).
constexpr int kPlaneRows = 64, kPlanesMaxC = 256;
template <typename TI, typename TO, int MAXC>
__global__ __launch_bounds__(256) void ln_planes_tiled(const TI *__restrict__ x, int64_t plane, int C,
                                                       const float *__restrict__ w,
                                                       const float *__restrict__ b, float eps,
                                                       TO *__restrict__ y) {
  constexpr int P = kPlaneRows + 1;                  // padded tile row (conflict-free transposed reads)
  __shared__ float tile[MAXC * P];
  __shared__ float part[4][kPlaneRows];
  __shared__ float mean_s[kPlaneRows], rstd_s[kPlaneRows];
  const int64_t r0 = int64_t(blockIdx.x) * kPlaneRows;
  const int l = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int rows = int(plane - r0 < kPlaneRows ? plane - r0 : kPlaneRows);
  if (plane % 4 == 0) {
    // 4 rows of one plane per load (8 or 16 bytes; plane % 4 == 0 keeps them aligned)
    for (int i = threadIdx.x; i < C * (kPlaneRows / 4); i += 256) {
      const int c = i / (kPlaneRows / 4), l4 = (i - c * (kPlaneRows / 4)) * 4;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      const TI *src = x + int64_t(c) * plane + r0 + l4;
      if (l4 + 4 <= rows) {
        if constexpr (std::is_same<TI, float>::value) {
          const float4 u = *reinterpret_cast<const float4 *>(src);
          v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
        } else {
          const bf16x4 u = *reinterpret_cast<const bf16x4 *>(src);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = static_cast<float>(u[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = l4 + e < rows ? to_f32(src[e]) : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) tile[c * P + l4 + e] = v[e];
    }
  } else {
    for (int c = grp; c < C; c += 4) tile[c * P + l] = l < rows ? to_f32(x[int64_t(c) * plane + r0 + l]) : 0.f;
  }
  __syncthreads();
  float s = 0.f;
  for (int c = grp; c < C; c += 4) s += tile[c * P + l];
  part[grp][l] = s;
  __syncthreads();
  if (grp == 0) mean_s[l] = (part[0][l] + part[1][l] + part[2][l] + part[3][l]) / float(C);
  __syncthreads();
  const float mean = mean_s[l];
  float q = 0.f;
  for (int c = grp; c < C; c += 4) {
    const float d = tile[c * P + l] - mean;
    q += d * d;
  }
  part[grp][l] = q;                                  // (read before the previous barrier)
  __syncthreads();
  if (grp == 0) rstd_s[l] = rsqrtf((part[0][l] + part[1][l] + part[2][l] + part[3][l]) / float(C) + eps);
  __syncthreads();
  if (C % 4 == 0) {                                 // 4 channels of one row per store
    const int c4s = C / 4;
    for (int i = threadIdx.x; i < rows * c4s; i += 256) {
      const int row = i / c4s, c = (i - row * c4s) * 4;
      float t[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        t[e] = (tile[(c + e) * P + row] - mean_s[row]) * rstd_s[row];
        if (w) t[e] *= w[c + e];
        if (b) t[e] += b[c + e];
      }
      TO *dst = y + (r0 + row) * int64_t(C) + c;
      if constexpr (std::is_same<TO, float>::value) {
        *reinterpret_cast<float4 *>(dst) = make_float4(t[0], t[1], t[2], t[3]);
      } else {
        bf16x4 u;
#pragma unroll
        for (int e = 0; e < 4; ++e) u[e] = bf16(t[e]);
        *reinterpret_cast<bf16x4 *>(dst) = u;
      }
    }
    return;
  }
  const int total = rows * C;
  for (int i = threadIdx.x; i < total; i += 256) {
    const int row = i / C, c = i - row * C;
    float t = (tile[c * P + row] - mean_s[row]) * rstd_s[row];
    if (w) t *= w[c];
    if (b) t += b[c];
    y[(r0 + row) * int64_t(C) + c] = from_f32<TO>(t);
  }
}

template <typename TI, typename TO, typename TA, int MODE>
static int launch_rows(const void *x, int64_t rows, int64_t C, const float *w, const float *b,
                       const void *scale, const void *shift, int64_t cond_rows, float eps, void *y,
                       hipStream_t stream) {
  if (rows == 0 || C == 0) return XFH_OK;
  const TI *xi = static_cast<const TI *>(x);
  TO *yo = static_cast<TO *>(y);
  const TA *sc = static_cast<const TA *>(scale);
  const TA *sh = static_cast<const TA *>(shift);
  const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                       (MODE == 0 || (reinterpret_cast<uintptr_t>(scale) % 16 == 0 &&
                                      reinterpret_cast<uintptr_t>(shift) % 16 == 0));
#define XFH_LN_VEC(LPR, CH)                                                                      \
  do {                                                                                           \
    int64_t blocks = ceil_div(rows * (LPR), 256);                                                \
    ln_rows_vec<TI, TO, TA, LPR, CH, MODE><<<dim3(blocks), dim3(256), 0, stream>>>(              \
        xi, rows, w, b, sc, sh, cond_rows, eps, yo);                                             \
    return check_launch("layer_norm");                                                           \
  } while (0)
  if (aligned) {
    if (C == 128) XFH_LN_VEC(16, 1);
    if (C == 64) XFH_LN_VEC(8, 1);
    if (C == 256) XFH_LN_VEC(32, 1);
    if (C == 384) XFH_LN_VEC(16, 3);
    if (C == 768) XFH_LN_VEC(32, 3);
    if (C == 512) XFH_LN_VEC(64, 1);
    if (C == 1536) XFH_LN_VEC(64, 3);
  }
#undef XFH_LN_VEC
  int64_t blocks = ceil_div(rows * 64, 256);
  ln_rows_any<TI, TO, TA, MODE><<<dim3(blocks), dim3(256), 0, stream>>>(xi, rows, C, w, b, sc, sh,
                                                                         cond_rows, eps, yo);
  return check_launch("layer_norm");
}

template <int MODE, typename TA>
static int dispatch_rows(const void *x, int xd, int64_t rows, int64_t C, const float *w,
                         const float *b, const void *sc, const void *sh, int64_t cr, float eps,
                         void *y, int yd, hipStream_t s) {
  if (xd == XFH_F32 && yd == XFH_F32) return launch_rows<float, float, TA, MODE>(x, rows, C, w, b, sc, sh, cr, eps, y, s);
  if (xd == XFH_F32 && yd == XFH_BF16) return launch_rows<float, bf16, TA, MODE>(x, rows, C, w, b, sc, sh, cr, eps, y, s);
  if (xd == XFH_BF16 && yd == XFH_F32) return launch_rows<bf16, float, TA, MODE>(x, rows, C, w, b, sc, sh, cr, eps, y, s);
  if (xd == XFH_BF16 && yd == XFH_BF16) return launch_rows<bf16, bf16, TA, MODE>(x, rows, C, w, b, sc, sh, cr, eps, y, s);
  return fail(XFH_EUNSUPPORTED, "layer_norm: dtypes must be f32 or bf16");
}

int layer_norm_rows(const void *x, int xd, int64_t rows, int64_t C, const float *w, const float *b,
                    float eps, void *y, int yd, hipStream_t s) {
  KernelTimer timer("layer_norm", s);
  return dispatch_rows<0, float>(x, xd, rows, C, w, b, nullptr, nullptr, 1, eps, y, yd, s);
}

int adaptive_layer_norm_rows(const void *x, int xd, int64_t rows, int64_t C, const void *scale,
                             const void *shift, int ad, int64_t cond_rows, float eps, void *y,
                             int yd, hipStream_t s) {
  if (ad == XFH_F32) return dispatch_rows<1, float>(x, xd, rows, C, nullptr, nullptr, scale, shift, cond_rows, eps, y, yd, s);
  if (ad == XFH_BF16) return dispatch_rows<1, bf16>(x, xd, rows, C, nullptr, nullptr, scale, shift, cond_rows, eps, y, yd, s);
  return fail(XFH_EUNSUPPORTED, "adaptive_layer_norm: aux dtype must be f32 or bf16");
}

template <int MAXC>
static int launch_planes_tiled(const void *x, int xd, int64_t plane, int C, const float *w, const float *b,
                               float eps, void *y, int yd, dim3 tiles, hipStream_t s) {
  if (xd == XFH_F32 && yd == XFH_F32)
    ln_planes_tiled<float, float, MAXC><<<tiles, 256, 0, s>>>((const float *)x, plane, C, w, b, eps, (float *)y);
  else if (xd == XFH_BF16 && yd == XFH_BF16)
    ln_planes_tiled<bf16, bf16, MAXC><<<tiles, 256, 0, s>>>((const bf16 *)x, plane, C, w, b, eps, (bf16 *)y);
  else if (xd == XFH_F32 && yd == XFH_BF16)
    ln_planes_tiled<float, bf16, MAXC><<<tiles, 256, 0, s>>>((const float *)x, plane, C, w, b, eps, (bf16 *)y);
  else
    return fail(XFH_EUNSUPPORTED, "layer_norm_planes: unsupported dtypes");
  return check_launch("layer_norm_planes");
}

int layer_norm_planes(const void *x, int xd, int64_t plane, int C, const float *w, const float *b,
                      float eps, void *y, int yd, hipStream_t s) {
  if (plane == 0) return XFH_OK;
  if (C <= kPlanesMaxC) {
    dim3 tiles(ceil_div(plane, int64_t(kPlaneRows)));
    if (C <= 64) return launch_planes_tiled<64>(x, xd, plane, C, w, b, eps, y, yd, tiles, s);
    if (C <= 128) return launch_planes_tiled<128>(x, xd, plane, C, w, b, eps, y, yd, tiles, s);
    return launch_planes_tiled<kPlanesMaxC>(x, xd, plane, C, w, b, eps, y, yd, tiles, s);
  }
  dim3 grid(ceil_div(plane, 256));
  if (xd == XFH_F32 && yd == XFH_F32)
    ln_planes<float, float><<<grid, 256, 0, s>>>((const float *)x, plane, C, w, b, eps, (float *)y);
  else if (xd == XFH_BF16 && yd == XFH_BF16)
    ln_planes<bf16, bf16><<<grid, 256, 0, s>>>((const bf16 *)x, plane, C, w, b, eps, (bf16 *)y);
  else if (xd == XFH_F32 && yd == XFH_BF16)
    ln_planes<float, bf16><<<grid, 256, 0, s>>>((const float *)x, plane, C, w, b, eps, (bf16 *)y);
  else
    return fail(XFH_EUNSUPPORTED, "layer_norm_planes: unsupported dtypes");
  return check_launch("layer_norm_planes");
}

}  // namespace xfh
