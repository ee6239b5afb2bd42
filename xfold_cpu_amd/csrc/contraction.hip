// Per-channel triangle contraction: out[k][i][j] = sum_t L[k][i][t] * R[k][j][t]
// (bf16 operands, fp32 accumulation, bf16 result), the N x N x N product at the centre
// of xfold/nn/triangle_multiplication.py:96 for both directions (the operand layouts are
// prepared by trimul_project).
//
// Tiling: 128 x 128 output tile per workgroup, k-step 64, 4 wavefronts in a 2 x 2 grid
// each owning 64 x 64 (4 x 4 MFMA 16x16x32 tiles). Both operand tiles are double-buffered
// in LDS: the global loads of step s+1 are in flight while step s is multiplied, one
// barrier per step. The MFMA takes R rows as its A operand so that a lane ends up with
// four consecutive j of one i and writes them as one 8-byte store. Channels are numbered
// so that each XCD works through a contiguous run of channels (their operands stay in
// that XCD's L2).
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int TB = 128;                 // tile edge
constexpr int TK = 64;                  // k-step
constexpr int TPITCH = TK + 8;          // LDS row pitch (bf16): 144 bytes
constexpr int TILE_ELEMS = TB * TPITCH;

__global__ __launch_bounds__(256, 2) void contraction_kernel(ContractionArgs a) {
  __shared__ bf16 lds[4 * TILE_ELEMS];   // [stage][L, R] tiles
  const int n = a.n;
  const int tiles = (n + TB - 1) / TB;
  const int64_t per_channel = int64_t(tiles) * tiles;
  const int64_t total = per_channel * a.channels;
  const int64_t per_xcd = (total + 7) / 8;
  const int64_t logical = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (logical >= total) return;
  const int64_t ch = logical / per_channel;
  const int tile = int(logical % per_channel);
  const int i0 = (tile / tiles) * TB, j0 = (tile % tiles) * TB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wi = wave >> 1, wj = wave & 1, col = lane & 15, grp = lane >> 4;
  const int64_t plane = int64_t(n) * n;
  const bf16 *L = a.left + ch * plane;
  const bf16 *R = a.right + ch * plane;
  const bool vec = (n % 8) == 0;

  // 128 rows x 64 k of each operand per stage: 1024 chunks of 16 B -> 4 per thread each.
  uint4 rl[4], rr[4];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int r = idx >> 3, kc = (idx & 7) * 8;
      const int k = k0 + kc;
      rl[c] = make_uint4(0, 0, 0, 0);
      rr[c] = make_uint4(0, 0, 0, 0);
      if (vec) {
        if (i0 + r < n && k < n) rl[c] = *reinterpret_cast<const uint4 *>(L + int64_t(i0 + r) * n + k);
        if (j0 + r < n && k < n) rr[c] = *reinterpret_cast<const uint4 *>(R + int64_t(j0 + r) * n + k);
      } else {
        bf16 tl[8], tr[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          tl[e] = (i0 + r < n && k + e < n) ? L[int64_t(i0 + r) * n + k + e] : bf16(0.0f);
          tr[e] = (j0 + r < n && k + e < n) ? R[int64_t(j0 + r) * n + k + e] : bf16(0.0f);
        }
        __builtin_memcpy(&rl[c], tl, 16);
        __builtin_memcpy(&rr[c], tr, 16);
      }
    }
  };
  auto stash = [&](int stage) {
    bf16 *tl = lds + (2 * stage) * TILE_ELEMS, *tr = tl + TILE_ELEMS;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + c * 256;
      const int r = idx >> 3, kc = (idx & 7) * 8;
      *reinterpret_cast<uint4 *>(tl + r * TPITCH + kc) = rl[c];
      *reinterpret_cast<uint4 *>(tr + r * TPITCH + kc) = rr[c];
    }
  };

  f32x4 acc[4][4];   // [jt][it]: rows j (A operand = R), cols i (B operand = L)
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int steps = (n + TK - 1) / TK;
  fetch(0);
  stash(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    if (s + 1 < steps) fetch((s + 1) * TK);
    const bf16 *tl = lds + (2 * (s & 1)) * TILE_ELEMS, *tr = tl + TILE_ELEMS;
#pragma unroll
    for (int kk = 0; kk < TK / 32; ++kk) {
      bf16x8 fr[4], fl[4];
#pragma unroll
      for (int x = 0; x < 4; ++x)
        fr[x] = *reinterpret_cast<const bf16x8 *>(tr + (wj * 64 + x * 16 + col) * TPITCH + kk * 32 + grp * 8);
#pragma unroll
      for (int y = 0; y < 4; ++y)
        fl[y] = *reinterpret_cast<const bf16x8 *>(tl + (wi * 64 + y * 16 + col) * TPITCH + kk * 32 + grp * 8);
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = mfma16(fr[x], fl[y], acc[x][y]);
    }
    if (s + 1 < steps) stash((s + 1) & 1);
    __syncthreads();
  }

  // acc[x][y][e] = out[i = i0 + wi*64 + y*16 + col][j = j0 + wj*64 + x*16 + grp*4 + e]
  bf16 *O = a.out + ch * plane;
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    const int i = i0 + wi * 64 + y * 16 + col;
    if (i >= n) continue;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int j = j0 + wj * 64 + x * 16 + grp * 4;
      bf16 *dst = O + int64_t(i) * n + j;
      if (vec && j + 4 <= n) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = bf16(acc[x][y][e]);
        *reinterpret_cast<bf16x4 *>(dst) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (j + e < n) dst[e] = bf16(acc[x][y][e]);
      }
    }
  }
}

}  // namespace

int contraction(const ContractionArgs &a, hipStream_t s) {
  if (a.n == 0 || a.channels == 0) return XFH_OK;
  const int64_t tiles = ceil_div(a.n, TB);
  const int64_t total = tiles * tiles * a.channels;
  const int64_t grid = ceil_div(total, 8) * 8;
  KernelTimer timer("trimul_contract", s);
  contraction_kernel<<<dim3(grid), 256, 0, s>>>(a);
  return check_launch("contraction");
}

}  // namespace xfh
