// Batched "NT" GEMM on MFMA: C[b][m][n] = epilogue(sum_k A[b][m][k] * B[b][n][k]).
//
// Both operands are k-contiguous, which is torch.nn.Linear's weight layout ([out, in]) and
// also the layout the triangle-multiplication contraction is written in, so one kernel
// serves every projection and the per-channel N x N x N products.
//
// Tiling: 128 x 128 block tile, k-step 32, 256 threads = 4 wavefronts in a 2 x 2 grid,
// each owning a 64 x 64 sub-tile = 4 x 4 MFMA 16x16 tiles (bf16: v_mfma_f32_16x16x32_bf16;
// fp32: 8 x v_mfma_f32_16x16x4f32 per k-step). Problems with fewer 128 x 128 tiles than two
// per CU take 64 x 64 tiles (32 x 32 per wavefront) instead, four times as many workgroups. Global -> register prefetch of the next
// k-step overlaps the MFMAs of the current one; LDS rows are padded by 16 bytes so the
// 16 rows a fragment read touches fall in distinct banks.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int BK = 32, THREADS = 256;

template <typename T, int BT> struct GemmSmem {
  static constexpr int kChunk = 16 / sizeof(T);      // elements per 16-byte vector
  static constexpr int kPitch = BK + kChunk;          // padded LDS row (elements)
  T a[BT * kPitch];
  T b[BT * kPitch];
};

template <typename T> __device__ __forceinline__ typename Frag<T>::type read_frag(const T *p);
template <> __device__ __forceinline__ bf16x8 read_frag<bf16>(const bf16 *p) {
  return *reinterpret_cast<const bf16x8 *>(p);
}
template <> __device__ __forceinline__ f32x8 read_frag<float>(const float *p) {
  f32x8 f;
  float4 lo = reinterpret_cast<const float4 *>(p)[0];
  float4 hi = reinterpret_cast<const float4 *>(p)[1];
  f.v[0] = lo.x; f.v[1] = lo.y; f.v[2] = lo.z; f.v[3] = lo.w;
  f.v[4] = hi.x; f.v[5] = hi.y; f.v[6] = hi.z; f.v[7] = hi.w;
  return f;
}

// Loads one 16-byte chunk (kChunk elements) of row `row`, columns [k, k + kChunk).
template <typename T, bool VEC>
__device__ __forceinline__ uint4 load_chunk(const T *base, int64_t ld, int row, int rows, int k,
                                            int K) {
  constexpr int kChunk = 16 / sizeof(T);
  uint4 out = make_uint4(0, 0, 0, 0);
  if (row >= rows) return out;
  const T *p = base + int64_t(row) * ld + k;
  if (VEC) {
    if (k < K) out = *reinterpret_cast<const uint4 *>(p);
  } else {
    T tmp[kChunk];
#pragma unroll
    for (int e = 0; e < kChunk; ++e) tmp[e] = (k + e < K) ? p[e] : T(0);
    __builtin_memcpy(&out, tmp, 16);
  }
  return out;
}

template <typename TO>
__device__ __forceinline__ float apply_epilogue(int epi, float acc, TO *c, const TO *aux) {
  switch (epi) {
    case XFH_EPI_MUL_SIGMOID_AUX: return acc * sigmoidf_(to_f32(*aux));
    case XFH_EPI_SIGMOID_MUL_AUX: return sigmoidf_(acc) * to_f32(*aux);
    case XFH_EPI_ACCUMULATE: return to_f32(*c) + acc;
    case XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE: return to_f32(*c) + acc * sigmoidf_(to_f32(*aux));
    default: return acc;
  }
}

// BT x BT block tile (BT = 128 or 64), each wavefront BT/2 x BT/2 = TW x TW MFMA tiles.
template <typename T, typename TO, bool VEC, bool GLU, int BT>
__global__ __launch_bounds__(THREADS) void gemm_nt_kernel(GemmArgs p) {
  constexpr int BM = BT, BN = BT, WT = BT / 2, TW = WT / 16;
  typedef GemmSmem<T, BT> Smem;
  constexpr int kChunk = Smem::kChunk;
  constexpr int kPitch = Smem::kPitch;
  constexpr int kChunksPerRow = BK / kChunk;
  constexpr int kLoads = BM * kChunksPerRow / THREADS;
  __shared__ Smem smem;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int64_t batch = blockIdx.z;
  const T *A = static_cast<const T *>(p.A) + batch * p.sA + int64_t(m0) * p.lda;
  const T *B = static_cast<const T *>(p.B) + batch * p.sB + int64_t(n0) * p.ldb;
  const int rowsA = p.M - m0, rowsB = p.N - n0;

  f32x4 acc[TW][TW];
#pragma unroll
  for (int i = 0; i < TW; ++i)
#pragma unroll
    for (int j = 0; j < TW; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 ra[kLoads], rb[kLoads];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int ci = tid + i * THREADS;
      const int r = ci / kChunksPerRow, kc = (ci % kChunksPerRow) * kChunk;
      ra[i] = load_chunk<T, VEC>(A, p.lda, r, rowsA, k0 + kc, p.K);
      rb[i] = load_chunk<T, VEC>(B, p.ldb, r, rowsB, k0 + kc, p.K);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int ci = tid + i * THREADS;
      const int r = ci / kChunksPerRow, kc = (ci % kChunksPerRow) * kChunk;
      *reinterpret_cast<uint4 *>(&smem.a[r * kPitch + kc]) = ra[i];
      *reinterpret_cast<uint4 *>(&smem.b[r * kPitch + kc]) = rb[i];
    }
  };

  const int fr = lane & 15, fk = (lane >> 4) * 8;
  fetch(0);
  for (int k0 = 0; k0 < p.K; k0 += BK) {
    __syncthreads();
    stash();
    __syncthreads();
    if (k0 + BK < p.K) fetch(k0 + BK);
    typename Frag<T>::type fa[TW], fb[TW];
#pragma unroll
    for (int i = 0; i < TW; ++i) fa[i] = read_frag<T>(&smem.a[(wm * WT + i * 16 + fr) * kPitch + fk]);
#pragma unroll
    for (int j = 0; j < TW; ++j) fb[j] = read_frag<T>(&smem.b[(wn * WT + j * 16 + fr) * kPitch + fk]);
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
      for (int j = 0; j < TW; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
  }

  TO *C = static_cast<TO *>(p.C) + batch * p.sC;
  const TO *aux = static_cast<const TO *>(p.aux);
  const int col_lane = lane & 15, row_lane = (lane >> 4) * 4;
  if (GLU) {
    // Packed GLU weight: 32-column groups = 16 gate columns then the 16 matching value
    // columns, so sub-tiles (2q, 2q + 1) of a wave hold gate/value of the same features.
#pragma unroll
    for (int q = 0; q < TW / 2; ++q) {
      const int f = (n0 + wn * WT) / 2 + q * 16 + col_lane;
      if (f >= p.glu_f) continue;
#pragma unroll
      for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + wm * WT + i * 16 + row_lane + e;
          if (m >= p.M) continue;
          const float g = acc[i][2 * q][e], v = acc[i][2 * q + 1][e];
          C[int64_t(m) * p.ldc + f] = from_f32<TO>(siluf_(g) * v);
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    const int n = n0 + wn * WT + j * 16 + col_lane;
    if (n >= p.N) continue;
    const float bias = p.bias ? p.bias[batch * p.sBias + n] : 0.f;
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * WT + i * 16 + row_lane + e;
        if (m >= p.M) continue;
        TO *c = c_element(p, C, m, n);
        const TO *a = nullptr;
        if (aux) {
          const int64_t ar = p.aux_rows > 0 ? (m % p.aux_rows) : m;
          a = aux + batch * p.sAux + ar * p.ldaux + n;
        }
        float v = acc[i][j][e] + bias;
        if (p.row_div) v /= p.row_div_eps + p.row_div[m];
        *c = from_f32<TO>(apply_epilogue<TO>(p.epi, v, c, a));
      }
  }
}

template <typename T, typename TO>
int launch_typed(const GemmArgs &p, int64_t batch, bool glu, hipStream_t s) {
  constexpr int kChunk = 16 / sizeof(T);
  const bool vec = (p.K % kChunk == 0) && (p.lda % kChunk == 0) && (p.ldb % kChunk == 0) &&
                   (p.sA % kChunk == 0) && (p.sB % kChunk == 0) &&
                   (reinterpret_cast<uintptr_t>(p.A) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(p.B) % 16 == 0);
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const bool small = ceil_div(p.N, int64_t(128)) * ceil_div(p.M, int64_t(128)) * batch < 2 * int64_t(cus);
  if (small) {
    dim3 grid(ceil_div(p.N, 64), ceil_div(p.M, 64), batch);
    if (glu) {
      if (vec) gemm_nt_kernel<T, TO, true, true, 64><<<grid, THREADS, 0, s>>>(p);
      else gemm_nt_kernel<T, TO, false, true, 64><<<grid, THREADS, 0, s>>>(p);
    } else {
      if (vec) gemm_nt_kernel<T, TO, true, false, 64><<<grid, THREADS, 0, s>>>(p);
      else gemm_nt_kernel<T, TO, false, false, 64><<<grid, THREADS, 0, s>>>(p);
    }
    return check_launch("gemm_nt");
  }
  dim3 grid(ceil_div(p.N, 128), ceil_div(p.M, 128), batch);
  if (glu) {
    if (vec) gemm_nt_kernel<T, TO, true, true, 128><<<grid, THREADS, 0, s>>>(p);
    else gemm_nt_kernel<T, TO, false, true, 128><<<grid, THREADS, 0, s>>>(p);
  } else {
    if (vec) gemm_nt_kernel<T, TO, true, false, 128><<<grid, THREADS, 0, s>>>(p);
    else gemm_nt_kernel<T, TO, false, false, 128><<<grid, THREADS, 0, s>>>(p);
  }
  return check_launch("gemm_nt");
}

// Up to four row-major matrices stacked into dst (a GEMM's B operand built from separate
// Linear weights): thread = 16 bytes of dst.
__global__ void stack_rows_kernel(char *__restrict__ dst, const char *s0, const char *s1, const char *s2,
                                  const char *s3, int64_t b1, int64_t b2, int64_t b3, int64_t total) {
  const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 16;
  if (i >= total) return;
  const char *src = i < b1 ? s0 + i : i < b2 ? s1 + (i - b1) : i < b3 ? s2 + (i - b2) : s3 + (i - b3);
  *reinterpret_cast<uint4 *>(dst + i) = *reinterpret_cast<const uint4 *>(src);
}

}  // namespace

int gemm_nt(const GemmArgs &p, int64_t batch, int dtype, int out_dtype, bool glu, hipStream_t s) {
  if (p.M == 0 || p.N == 0 || batch == 0) return XFH_OK;
  if (p.M < 0 || p.N < 0 || p.K < 0) return fail(XFH_EINVAL, "gemm: negative size");
  if (int64_t(ceil_div(p.M, 128)) > 65535) return fail(XFH_EUNSUPPORTED, "gemm: M too large for one launch");
  if (dtype == XFH_BF16 && (out_dtype == XFH_BF16 || out_dtype == XFH_F32) && ceil_div(p.N, 64) <= 65535 &&
      batch <= 65535 && gemm_ring_supported(p, out_dtype))
    return gemm_ring(p, batch, out_dtype, glu, s);
  if (dtype == XFH_BF16 && out_dtype == XFH_BF16) return launch_typed<bf16, bf16>(p, batch, glu, s);
  if (dtype == XFH_BF16 && out_dtype == XFH_F32) return launch_typed<bf16, float>(p, batch, glu, s);
  if (dtype == XFH_F32 && out_dtype == XFH_F32) return launch_typed<float, float>(p, batch, glu, s);
  if (dtype == XFH_F32 && out_dtype == XFH_BF16) return launch_typed<float, bf16>(p, batch, glu, s);
  return fail(XFH_EUNSUPPORTED, "gemm: dtype must be f32 or bf16");
}

// GLU weight packing: rows of the packed matrix in groups of 32 = 16 gate rows (features
// 16t..16t+15 of the first half) followed by the 16 matching value rows; zero rows pad.
template <typename T>
__global__ void glu_pack_kernel(const T *__restrict__ w, int64_t f, int64_t k, T *__restrict__ out,
                                int64_t rows_out) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows_out * k) return;
  const int64_t r = idx / k, c = idx % k;
  const int64_t group = r / 32, within = r % 32;
  const int64_t feature = group * 16 + (within % 16);
  const bool value = within >= 16;
  T v = T(0);
  if (feature < f) v = w[(value ? f + feature : feature) * k + c];
  out[idx] = v;
}

int glu_pack(const void *w, int64_t f, int64_t k, int dtype, void *packed, hipStream_t s) {
  const int64_t rows = 2 * align_up(f, 16);
  const int64_t total = rows * k;
  if (total == 0) return XFH_OK;
  dim3 grid(ceil_div(total, 256));
  if (dtype == XFH_BF16)
    glu_pack_kernel<bf16><<<grid, 256, 0, s>>>((const bf16 *)w, f, k, (bf16 *)packed, rows);
  else if (dtype == XFH_F32)
    glu_pack_kernel<float><<<grid, 256, 0, s>>>((const float *)w, f, k, (float *)packed, rows);
  else
    return fail(XFH_EUNSUPPORTED, "glu_pack: dtype must be f32 or bf16");
  return check_launch("glu_pack");
}

int stack_rows(void *dst, const void *const src[4], const int64_t rows[4], int64_t cols, int es, hipStream_t s) {
  const int64_t b1 = rows[0] * cols * es, b2 = b1 + rows[1] * cols * es, b3 = b2 + rows[2] * cols * es;
  const int64_t total = b3 + rows[3] * cols * es;
  for (int i = 0; i < 4; ++i)
    if (rows[i] && reinterpret_cast<uintptr_t>(src[i]) % 16)
      return fail(XFH_EUNSUPPORTED, "stack_rows: sources must be 16-byte aligned");
  if (b1 % 16 || b2 % 16 || b3 % 16 || total % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return fail(XFH_EUNSUPPORTED, "stack_rows: matrices must be multiples of 16 bytes");
  if (total == 0) return XFH_OK;
  stack_rows_kernel<<<dim3(unsigned(ceil_div(total / 16, 256))), 256, 0, s>>>(
      static_cast<char *>(dst), static_cast<const char *>(src[0]), static_cast<const char *>(src[1]),
      static_cast<const char *>(src[2]), static_cast<const char *>(src[3]), b1, b2, b3, total);
  return check_launch("stack_rows");
}

}  // namespace xfh
