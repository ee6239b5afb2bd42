// bf16 "NT" GEMM, C[b][m][n] = epilogue(sum_k A[b][m][k] * B[b][n][k]), for the shapes of
// the projections and transitions (k a multiple of 32, 16-byte aligned rows). Same contract
// as gemm_nt (gemm.hip), which keeps every other case.
//
// Tiling: 128 x 128 output tile per workgroup, 4 wavefronts in a 2 x 2 grid each owning
// 64 x 64 (4 x 4 MFMA 16x16x32 tiles). Per k-step of 32 both 128 x 32 operand tiles go
// global -> LDS with direct loads (global_load_lds_dwordx4, no registers) into a 4-slot
// ring: the loads of steps s+1..s+3 are in flight while step s is multiplied, one barrier
// per step. Rows are 64 B in LDS with the 16-byte slots XOR-swizzled (slot c of row r
// holds chunk c ^ ((r >> 2) & 3)) so the 16 rows of an MFMA operand read hit distinct
// bank groups. Rows past M or N read the last row (their results are never stored).
// The MFMA takes the B rows as its A operand, so a lane ends up with four consecutive
// output columns of one row: bias, auxiliary operand, accumulation and the GLU pairing
// all work on 4-element vectors and the stores are 8 (bf16) or 16 (fp32) bytes.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int TB = 128;                  // tile edge
constexpr int TK = 32;                   // k-step
constexpr int SLOTS = 4;                 // ring of operand stages
constexpr int OP_ELEMS = TB * TK;        // one operand tile (bf16), 8 KB
constexpr int SLOT_ELEMS = 2 * OP_ELEMS;
constexpr int PIECES = 2 * TB / 16;      // 1 KB loads per k-step (16), 4 per wavefront
constexpr int PIECES_PER_WAVE = PIECES / 4;
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

template <int N> __device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <typename TO> struct Vec4;
template <> struct Vec4<bf16> {
  __device__ static void load(const bf16 *p, float (&v)[4]) {
    const bf16x4 x = *reinterpret_cast<const bf16x4 *>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = static_cast<float>(x[e]);
  }
  __device__ static void store(bf16 *p, const float (&v)[4]) {
    bf16x4 x;
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = bf16(v[e]);
    *reinterpret_cast<bf16x4 *>(p) = x;
  }
};
template <> struct Vec4<float> {
  __device__ static void load(const float *p, float (&v)[4]) {
    const float4 x = *reinterpret_cast<const float4 *>(p);
    v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  }
  __device__ static void store(float *p, const float (&v)[4]) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

__device__ __forceinline__ float epilogue(int epi, float acc, float c, float aux) {
  switch (epi) {
    case XFH_EPI_MUL_SIGMOID_AUX: return acc * sigmoidf_(aux);
    case XFH_EPI_SIGMOID_MUL_AUX: return sigmoidf_(acc) * aux;
    case XFH_EPI_ACCUMULATE: return c + acc;
    case XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE: return c + acc * sigmoidf_(aux);
    default: return acc;
  }
}

template <typename TO, bool GLU>
__global__ __launch_bounds__(256, 2) void gemm_ring_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) bf16 lds[SLOTS * SLOT_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
  const int m0 = blockIdx.y * TB, n0 = blockIdx.x * TB;
  const int64_t batch = blockIdx.z;
  const bf16 *A = static_cast<const bf16 *>(p.A) + batch * p.sA;
  const bf16 *B = static_cast<const bf16 *>(p.B) + batch * p.sB;

  // Piece q of a k-step: operand q / 8 (A, B), rows 16 (q % 8) .. +15; lane -> row
  // 16 (q % 8) + lane / 4, LDS slot lane % 4 holding chunk (lane % 4) ^ ((lane >> 4) & 3).
  const int chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const bf16 *src[PIECES_PER_WAVE];
#pragma unroll
  for (int j = 0; j < PIECES_PER_WAVE; ++j) {
    const int q = wave + 4 * j;
    const int row = (q % 8) * 16 + (lane >> 2);
    if (q < 8) {
      const int m = m0 + row;
      src[j] = A + int64_t(m < p.M ? m : p.M - 1) * p.lda + chunk * 8;
    } else {
      const int n = n0 + row;
      src[j] = B + int64_t(n < p.N ? n : p.N - 1) * p.ldb + chunk * 8;
    }
  }
  auto issue = [&](int step, int slot) {
#pragma unroll
    for (int j = 0; j < PIECES_PER_WAVE; ++j) {
      const int q = wave + 4 * j;
      bf16 *dst = lds + slot * SLOT_ELEMS + (q < 8 ? 0 : OP_ELEMS) + (q % 8) * 16 * TK;
      __builtin_amdgcn_global_load_lds((global_void *)(src[j] + step * TK), (lds_void *)dst, 16, 0, 0);
    }
  };

  // Fragment offset: row base + col of an operand tile, k-chunk grp, lives at
  // row * TK + (grp ^ ((col >> 2) & 3)) * 8 for a base that is a multiple of 16.
  const int frag = col * TK + ((grp ^ ((col >> 2) & 3)) * 8);

  f32x4 acc[4][4];   // [jt][it]: rows n (A operand = B rows), cols m (B operand = A rows)
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int steps = p.K / TK;
#pragma unroll
  for (int s = 0; s < SLOTS - 1; ++s)
    if (s < steps) issue(s, s);
  for (int s = 0; s < steps; ++s) {
    // This wavefront's loads of step s have landed (the younger steps may still fly), then
    // every wavefront's have, and every wavefront is done with step s - 1.
    const int younger = steps - 1 - s;
    if (younger >= 2) wait_vmcnt<2 * PIECES_PER_WAVE>();
    else if (younger == 1) wait_vmcnt<PIECES_PER_WAVE>();
    else wait_vmcnt<0>();
    __syncthreads();
    if (s + SLOTS - 1 < steps) issue(s + SLOTS - 1, (s + SLOTS - 1) % SLOTS);
    const bf16 *ta = lds + (s % SLOTS) * SLOT_ELEMS, *tb = ta + OP_ELEMS;
    bf16x8 fa[4], fb[4];
#pragma unroll
    for (int y = 0; y < 4; ++y) fa[y] = *reinterpret_cast<const bf16x8 *>(ta + (wm * 64 + y * 16) * TK + frag);
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      fb[x] = *reinterpret_cast<const bf16x8 *>(tb + (wn * 64 + x * 16) * TK + frag);
#pragma unroll
      for (int y = 0; y < 4; ++y) acc[x][y] = mfma16(fb[x], fa[y], acc[x][y]);
    }
  }

  // acc[x][y][e] = C[m = m0 + wm*64 + y*16 + col][n = n0 + wn*64 + x*16 + grp*4 + e]
  TO *C = static_cast<TO *>(p.C) + batch * p.sC;
  if constexpr (GLU) {
    // Packed GLU weight: 32-column groups = 16 gate columns then the 16 matching value
    // columns, so tiles (0, 1) and (2, 3) of a wavefront hold gate/value of the same features.
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int f = (n0 + wn * 64) / 2 + q * 16 + grp * 4;
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        const int m = m0 + wm * 64 + y * 16 + col;
        if (m >= p.M) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = siluf_(acc[2 * q][y][e]) * acc[2 * q + 1][y][e];
        TO *dst = C + int64_t(m) * p.ldc + f;
        if (f + 4 <= p.glu_f) {
          Vec4<TO>::store(dst, v);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (f + e < p.glu_f) dst[e] = from_f32<TO>(v[e]);
        }
      }
    }
    return;
  }
  const TO *aux = static_cast<const TO *>(p.aux);
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int n = n0 + wn * 64 + x * 16 + grp * 4;
    if (n >= p.N) continue;
    const bool full = n + 4 <= p.N;
    float bias[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.bias)
#pragma unroll
      for (int e = 0; e < 4; ++e) bias[e] = n + e < p.N ? p.bias[batch * p.sBias + n + e] : 0.f;
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int m = m0 + wm * 64 + y * 16 + col;
      if (m >= p.M) continue;
      TO *c = C + int64_t(m) * p.ldc + n;
      const TO *a = nullptr;
      if (aux) {
        const int64_t ar = p.aux_rows > 0 ? (m % p.aux_rows) : m;
        a = aux + batch * p.sAux + ar * p.ldaux + n;
      }
      const bool reads_c = p.epi == XFH_EPI_ACCUMULATE || p.epi == XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE;
      float cv[4] = {0.f, 0.f, 0.f, 0.f}, av[4] = {0.f, 0.f, 0.f, 0.f}, out[4];
      if (full) {
        if (reads_c) Vec4<TO>::load(c, cv);
        if (a) Vec4<TO>::load(a, av);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (n + e >= p.N) continue;
          if (reads_c) cv[e] = to_f32(c[e]);
          if (a) av[e] = to_f32(a[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] = epilogue(p.epi, acc[x][y][e] + bias[e], cv[e], av[e]);
      if (full) {
        Vec4<TO>::store(c, out);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < p.N) c[e] = from_f32<TO>(out[e]);
      }
    }
  }
}

bool aligned(const void *ptr, int bytes) { return reinterpret_cast<uintptr_t>(ptr) % bytes == 0; }

}  // namespace

bool gemm_ring_supported(const GemmArgs &p, int out_dtype) {
  const int ob = out_dtype == XFH_BF16 ? 2 : 4;
  const bool vec_out = p.ldc % 4 == 0 && p.sC % 4 == 0 && aligned(p.C, 4 * ob) &&
                       (!p.aux || (p.ldaux % 4 == 0 && p.sAux % 4 == 0 && aligned(p.aux, 4 * ob)));
  return p.K > 0 && p.K % TK == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 && p.sA % 8 == 0 &&
         p.sB % 8 == 0 && aligned(p.A, 16) && aligned(p.B, 16) && vec_out;
}

int gemm_ring(const GemmArgs &p, int64_t batch, int out_dtype, bool glu, hipStream_t s) {
  const dim3 grid(unsigned(ceil_div(p.N, TB)), unsigned(ceil_div(p.M, TB)), unsigned(batch));
  KernelTimer timer("gemm_ring", s);
  if (out_dtype == XFH_BF16) {
    if (glu) gemm_ring_kernel<bf16, true><<<grid, 256, 0, s>>>(p);
    else gemm_ring_kernel<bf16, false><<<grid, 256, 0, s>>>(p);
  } else {
    if (glu) gemm_ring_kernel<float, true><<<grid, 256, 0, s>>>(p);
    else gemm_ring_kernel<float, false><<<grid, 256, 0, s>>>(p);
  }
  return check_launch("gemm_ring");
}

}  // namespace xfh
