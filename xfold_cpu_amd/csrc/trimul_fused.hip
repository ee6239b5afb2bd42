// Fused triangle-multiplication kernels (bf16 compute, c = 128), around the per-channel
// contraction (xfold/nn/triangle_multiplication.py:71-105):
//
//   trimul_project: LN_in(z) -> [projection | gate] (one GEMM over a packed weight) ->
//       mask * proj * sigmoid(gate) -> channel 2k = a_k, 2k+1 = b_k -> written channel-major
//       in the contraction's operand layouts (left/right, see triangle.hip).
//   trimul_output: centre LN over the channel-major contraction result -> output_projection,
//       times sigmoid(gating_linear(LN_in(z))) (recomputed from z, which this kernel reads
//       anyway for the residual) -> z += update (or update stored).
//
// Both are row-panel kernels (panel.h): 128 pair positions per workgroup.
#include "common.h"
#include "kernels.h"
#include "panel.h"

namespace xfh {

namespace {

using namespace panel;

constexpr int SPITCH = ROWS + 8;     // staging row pitch (bf16): [channel][position]

template <typename TIN>
__global__ __launch_bounds__(256, 2) void trimul_project_kernel(TriProjectArgs a) {
  __shared__ bf16 lds_a[A_ELEMS];                 // A tile, later two B buffers
  __shared__ bf16 stage[32 * SPITCH];             // 32 channels x 128 positions
  __shared__ float mval[ROWS];
  auto bbuf = [&](int i) -> bf16 * { return lds_a + (i & 1) * B_ELEMS; };

  const int n = a.n;
  const int ppx = (n + ROWS - 1) / ROWS;          // panels per grid line
  const int x = blockIdx.x / ppx, y0 = (blockIdx.x % ppx) * ROWS;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
  const TIN *z = static_cast<const TIN *>(a.pair);
  // Pair position of panel row r: (x, y) outgoing, (y, x) incoming.
  auto pos_of = [&](int r) -> int64_t {
    const int64_t y = y0 + r;
    return a.outgoing ? int64_t(x) * n + y : y * n + x;
  };
  if (tid < ROWS) {
    float m = 0.f;
    if (y0 + tid < n) m = a.mask ? load_any(a.mask, a.mask_dtype, pos_of(tid)) : 1.f;
    mval[tid] = m;
  }
  ln_panel<TIN>([&](int r) -> const TIN * { return (y0 + r < n) ? z + pos_of(r) * K : nullptr; },
                a.ln_w, a.ln_b, a.eps, lds_a);
  __syncthreads();
  AFrags af;
  load_a_frags(lds_a, wm, af);
  BStage st;
  const int nout = 4 * K;                          // projection + gate, 2c each
  fetch_b(a.w_packed, 0, nout, st);
  __syncthreads();                                 // A tile consumed; reuse as B buffers
  stash_b(st, bbuf(0));
  __syncthreads();

  bf16 *left = a.left, *right = a.right;
  const int64_t plane = int64_t(n) * a.ld;
  const int chunks = nout / CHUNK;
  for (int j = 0; j < chunks; ++j) {
    if (j + 1 < chunks) fetch_b(a.w_packed, (j + 1) * CHUNK, nout, st);
    f32x4 acc[4][2];
    zero(acc);
    mma_chunk(af, bbuf(j), wn, acc);
    // Sub-tile 0 = projection, 1 = gate of projection channel 32j + 16*wn + col.
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int r0 = wm * 64 + mt * 16 + grp * 4;
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = bf16(acc[mt][0][e] * sigmoidf_(acc[mt][1][e]) * mval[r0 + e]);
      *reinterpret_cast<bf16x4 *>(&stage[(wn * 16 + col) * SPITCH + r0]) = v;
    }
    __syncthreads();
    // 32 projection channels x 128 positions -> left/right[k][x][y0 + ...], with zeros in
    // the pad columns y in [n, ld) (ld is a multiple of 32, so a chunk of 8 is either all
    // below ld or all above).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + i * 256;
      const int ch = idx >> 4, yc = (idx & 15) * 8;
      const int y = y0 + yc;
      if (y >= a.ld) continue;
      const int p = j * 32 + ch;                    // projection channel
      const bool is_a = (p & 1) == 0;
      bf16 *dst = ((a.outgoing != 0) == is_a ? left : right) + int64_t(p >> 1) * plane +
                  int64_t(x) * a.ld + y;
      bf16x8 v = *reinterpret_cast<const bf16x8 *>(&stage[ch * SPITCH + yc]);
      if (y + 8 > n) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (y + e >= n) v[e] = bf16(0.0f);
      }
      *reinterpret_cast<bf16x8 *>(dst) = v;
    }
    if (j + 1 < chunks) stash_b(st, bbuf(j + 1));
    __syncthreads();
  }
}

// Channel-major LayerNorm of a 128-channel x 128-position tile into the A tile.
// Thread t holds channels 8*(t%16) .. +7 of positions 8*(t/16) .. +7, so the 16 lanes of
// a DPP row hold all 128 channels of the same 8 positions: the statistics need no LDS
// round trip, and each position's normalised channels leave as 16-byte rows.
__device__ __forceinline__ void ln_channel_major(const bf16 *x, int64_t plane, int64_t pos0, int valid,
                                                 const float *w, const float *b, float eps,
                                                 bf16 *a_tile) {
  const int tid = threadIdx.x;
  const int kc = (tid & 15) * 8, pc = (tid >> 4) * 8;
  const bool full = pc + 8 <= valid;
  float v[8][8];                                   // [channel kc + i][position pc + e]
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bf16 *src = x + int64_t(kc + i) * plane + pos0 + pc;
    if (full) {
      load8<bf16>(src, v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = (pc + e < valid) ? static_cast<float>(src[e]) : 0.f;
    }
  }
  float mean[8], rstd[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) t += v[i][e];
    mean[e] = row16_sum(t) * (1.0f / K);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float d = v[i][e] - mean[e];
      t += d * d;
    }
    rstd[e] = rsqrtf(row16_sum(t) * (1.0f / K) + eps);
  }
  LnParams prm;
  load_ln_params(w, b, tid & 15, prm);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    bf16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = bf16((v[i][e] - mean[e]) * rstd[e] * prm.w[i] + prm.b[i]);
    *reinterpret_cast<bf16x8 *>(a_tile + (pc + e) * PITCH + kc) = o;
  }
}

template <typename TIN, typename TOUT>
__global__ __launch_bounds__(256, 2) void trimul_output_kernel(TriOutputArgs a) {
  __shared__ bf16 lds_a[A_ELEMS];                  // A tile / output staging
  __shared__ bf16 lds_b[2 * B_ELEMS];              // weight chunks
  auto bbuf = [&](int i) -> bf16 * { return lds_b + (i & 1) * B_ELEMS; };

  const int64_t plane = int64_t(a.n) * a.n;
  const int64_t pos0 = int64_t(blockIdx.x) * ROWS;
  const int valid = int(plane - pos0 < ROWS ? plane - pos0 : ROWS);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
  const TIN *z = static_cast<const TIN *>(a.pair);

  // 1) gate = sigmoid(LN_in(z) Wgating^T), kept in registers for this wavefront's block.
  ln_panel<TIN>([&](int r) -> const TIN * { return r < valid ? z + (pos0 + r) * K : nullptr; },
                a.ln_in_w, a.ln_in_b, a.eps_in, lds_a);
  __syncthreads();
  AFrags af;
  load_a_frags(lds_a, wm, af);
  BStage st;
  fetch_b(a.w_gating, 0, K, st);
  stash_b(st, bbuf(0));
  fetch_b(a.w_gating, CHUNK, K, st);
  stash_b(st, bbuf(1));
  __syncthreads();
  f32x4 gate[2][4][2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    zero(gate[j]);
    mma_chunk(af, bbuf(j), wn, gate[j]);
  }
  __syncthreads();                                 // everyone done with lds_a and lds_b

  // 2) centre LN of the contraction result -> A fragments; output projection.
  ln_channel_major(a.contracted, plane, pos0, valid, a.ln_c_w, a.ln_c_b, a.eps_c, lds_a);
  fetch_b(a.w_out, 0, K, st);
  stash_b(st, bbuf(0));
  fetch_b(a.w_out, CHUNK, K, st);
  stash_b(st, bbuf(1));
  __syncthreads();
  load_a_frags(lds_a, wm, af);
  __syncthreads();                                 // A tile free for output staging
  bf16 *stage = lds_a;                             // [128 positions][PITCH]
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    f32x4 acc[4][2];
    zero(acc);
    mma_chunk(af, bbuf(j), wn, acc);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int c = j * CHUNK + wn * 32 + nt * 16 + col;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = wm * 64 + mt * 16 + grp * 4 + e;
          stage[r * PITCH + c] = bf16(acc[mt][nt][e] * sigmoidf_(gate[j][mt][nt][e]));
        }
      }
  }
  __syncthreads();
  // 3) residual: 128 positions x 128 channels, 8 channels per thread-chunk.
  TOUT *out = static_cast<TOUT *>(a.out);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid + i * 256;
    const int r = idx >> 4, c = (idx & 15) * 8;
    if (r >= valid) continue;
    TOUT *dst = out + (pos0 + r) * K + c;
    float u[8];
    load8<bf16>(&stage[r * PITCH + c], u);
    float o[8];
    if (a.accumulate) {
      load8<TOUT>(dst, o);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += u[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = u[e];
    }
    if constexpr (sizeof(TOUT) == 2) {
      bf16x8 w;
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = bf16(o[e]);
      *reinterpret_cast<bf16x8 *>(dst) = w;
    } else {
      reinterpret_cast<float4 *>(dst)[0] = make_float4(o[0], o[1], o[2], o[3]);
      reinterpret_cast<float4 *>(dst)[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
  }
}

// Packed [4c][c] weight: chunk j (64 rows) = projection rows 32j..32j+15, gate rows
// 32j..32j+15, projection rows 32j+16..32j+31, gate rows 32j+16..32j+31.
__global__ void trimul_pack_kernel(const bf16 *__restrict__ proj, const bf16 *__restrict__ gate,
                                   int c, bf16 *__restrict__ packed) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = int64_t(4) * c * c;
  if (idx >= total) return;
  const int r = int(idx / c), k = int(idx % c);
  const int j = r / 64, s = (r % 64) / 16, i = r % 16;
  const int src_row = 32 * j + (s >= 2 ? 16 : 0) + i;
  const bf16 *src = (s & 1) ? gate : proj;
  packed[idx] = src[int64_t(src_row) * c + k];
}

}  // namespace

int trimul_pack(const void *proj, const void *gate, int c, void *packed, hipStream_t s) {
  const int64_t total = int64_t(4) * c * c;
  trimul_pack_kernel<<<dim3(ceil_div(total, 256)), 256, 0, s>>>((const bf16 *)proj, (const bf16 *)gate, c,
                                                                 (bf16 *)packed);
  return check_launch("trimul_pack");
}

int trimul_project(const TriProjectArgs &a, int pair_dtype, hipStream_t s) {
  const int64_t panels = int64_t(a.n) * ceil_div(a.n, ROWS);
  KernelTimer timer("trimul_project", s);
  if (pair_dtype == XFH_BF16)
    trimul_project_kernel<bf16><<<dim3(panels), 256, 0, s>>>(a);
  else
    trimul_project_kernel<float><<<dim3(panels), 256, 0, s>>>(a);
  return check_launch("trimul_project");
}

int trimul_output(const TriOutputArgs &a, int pair_dtype, int out_dtype, hipStream_t s) {
  const int64_t panels = ceil_div(int64_t(a.n) * a.n, ROWS);
  KernelTimer timer("trimul_output", s);
  if (pair_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    trimul_output_kernel<bf16, bf16><<<dim3(panels), 256, 0, s>>>(a);
  else if (pair_dtype == XFH_BF16 && out_dtype == XFH_F32)
    trimul_output_kernel<bf16, float><<<dim3(panels), 256, 0, s>>>(a);
  else if (pair_dtype == XFH_F32 && out_dtype == XFH_F32)
    trimul_output_kernel<float, float><<<dim3(panels), 256, 0, s>>>(a);
  else
    trimul_output_kernel<float, bf16><<<dim3(panels), 256, 0, s>>>(a);
  return check_launch("trimul_output");
}

}  // namespace xfh
