// Per-channel triangle contraction: out[k][i][j] = sum_t L[k][i][t] * R[k][j][t]
// (bf16 operands, fp32 accumulation, bf16 result), the N x N x N product at the centre
// of xfold/nn/triangle_multiplication.py:96 for both directions (the operand layouts are
// prepared by trimul_project).
//
// Operands: L, R in the blocked operand layout (kernels.h): 16 rows x 32 t of one channel
// are one contiguous 1 KB block, ld = contraction_ld(n), zeros for t in [n, ld) so that the
// last k-step needs no bounds. The result goes to the blocked result layout: 16 pair
// positions' channels contiguous.
//
// Tiling: 192 x 192 output tile per workgroup, 4 wavefronts in a 2 x 2 grid each owning
// 96 x 96 (6 x 6 MFMA 16x16x32 tiles). Per k-step of 32 both 192 x 32 operand tiles go
// global -> LDS with global_load_lds_dwordx4 (no registers) into a 3-slot ring, so the
// loads of step s+2 are in flight while step s is multiplied; one barrier per step. Rows
// are 64 B in LDS with the 16-byte slots XOR-swizzled (slot c of row r holds chunk
// c ^ ((r >> 2) & 3)), so the 16 rows of an MFMA operand read hit distinct bank groups.
// The MFMA takes R rows as its A operand so that a lane ends up with four consecutive j
// of one i and writes them as one 8-byte store. Channels are numbered so that each XCD
// works through a contiguous run of tiles: the workgroups in flight on an XCD cover a few
// consecutive channels, whose k-slices share 128-byte lines and DRAM pages.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int TB = 192;                 // tile edge
constexpr int WT = 96;                  // wavefront tile edge
constexpr int NT = WT / 16;             // MFMA tiles per wavefront edge (6)
constexpr int TK = 32;                  // k-step
constexpr int SLOTS = 3;                // ring of operand stages
constexpr int OP_ELEMS = TB * TK;       // one operand tile (bf16)
constexpr int SLOT_ELEMS = 2 * OP_ELEMS;
constexpr int PIECES = 2 * TB / 16;     // 1 KB loads per k-step (24), 6 per wavefront
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

__global__ __launch_bounds__(256, 2) void contraction_kernel(ContractionArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 lds[SLOTS * SLOT_ELEMS];
  const int n = a.n, ld = a.ld;
  const int tiles = (n + TB - 1) / TB;
  const int64_t per_channel = int64_t(tiles) * tiles;
  const int64_t total = per_channel * a.channels;
  const int64_t per_xcd = (total + 7) / 8;
  const int64_t logical = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (logical >= total) return;
  const int64_t ch = logical / per_channel;
  const int tile = int(logical % per_channel);
  const int i0 = (tile / tiles) * TB, j0 = (tile % tiles) * TB;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wi = wave >> 1, wj = wave & 1, col = lane & 15, grp = lane >> 4;
  // k-step s of row g of channel ch at op_offset(n, c, ch, g, 0) + s * step_stride.
  const int64_t step_stride = op_step_stride(n, a.channels);

  // Piece p of a k-step: operand p / 12 (L, R), rows 16 (p % 12) .. +15 (one 1 KB block); lane -> row
  // 16 (p % 12) + lane / 4, LDS slot lane % 4 holding chunk (lane % 4) ^ ((lane >> 4) & 3).
  // Rows beyond n read row n-1 (their results are never stored).
  const int chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const bf16 *src[PIECES / 4];
#pragma unroll
  for (int j = 0; j < PIECES / 4; ++j) {
    const int p = wave + 4 * j;
    const int row = (p % 12) * 16 + (lane >> 2);
    const int g = (p < 12 ? i0 : j0) + row;
    src[j] = (p < 12 ? a.left : a.right) + op_offset(n, a.channels, int(ch), g < n ? g : n - 1, 0) + chunk * 8;
  }
  auto issue = [&](int step, int slot) {
#pragma unroll
    for (int j = 0; j < PIECES / 4; ++j) {
      const int p = wave + 4 * j;
      bf16 *dst = lds + slot * SLOT_ELEMS + (p < 12 ? 0 : OP_ELEMS) + (p % 12) * 16 * TK;
      __builtin_amdgcn_global_load_lds((global_void *)(src[j] + step * step_stride), (lds_void *)dst, 16, 0, 0);
    }
  };

  // Fragment offsets: row r of an operand tile, k-chunk grp, lives at r*TK + slot*8 with
  // slot = grp ^ ((r >> 2) & 3); for r = base + col with base a multiple of 16 that is
  // grp ^ ((col >> 2) & 3).
  const int frag = col * TK + ((grp ^ ((col >> 2) & 3)) * 8);

  f32x4 acc[NT][NT];   // [jt][it]: rows j (A operand = R), cols i (B operand = L)
#pragma unroll
  for (int x = 0; x < NT; ++x)
#pragma unroll
    for (int y = 0; y < NT; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int steps = ld / TK;
  issue(0, 0);
  if (steps > 1) issue(1, 1);
  for (int s = 0; s < steps; ++s) {
    // This wavefront's loads of step s have landed (those of step s+1 may still fly),
    // then every wavefront's have, and every wavefront is done with step s-1.
    if (s + 1 < steps) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    ring_barrier();
    if (s + 2 < steps) issue(s + 2, (s + 2) % SLOTS);
    const bf16 *tl = lds + (s % SLOTS) * SLOT_ELEMS, *tr = tl + OP_ELEMS;
    // All L fragments and the first two R fragments, then each pair of R fragments is read
    // while the previous pair's 12 MFMAs run (scheduling barriers keep the compiler from
    // sinking the reads next to their use).
    bf16x8 fl[NT], fr[NT];
#pragma unroll
    for (int y = 0; y < NT; ++y)
      fl[y] = *reinterpret_cast<const bf16x8 *>(tl + (wi * WT + y * 16) * TK + frag);
#pragma unroll
    for (int x = 0; x < 2; ++x) fr[x] = *reinterpret_cast<const bf16x8 *>(tr + (wj * WT + x * 16) * TK + frag);
#pragma unroll
    for (int xp = 0; xp < NT / 2; ++xp) {
      __builtin_amdgcn_sched_barrier(0);
      if (xp + 1 < NT / 2) {
#pragma unroll
        for (int x = 2 * xp + 2; x < 2 * xp + 4; ++x)
          fr[x] = *reinterpret_cast<const bf16x8 *>(tr + (wj * WT + x * 16) * TK + frag);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int x = 2 * xp; x < 2 * xp + 2; ++x)
#pragma unroll
        for (int y = 0; y < NT; ++y) acc[x][y] = mfma16(fr[x], fl[y], acc[x][y]);
    }
  }

  // acc[x][y][e] = out[i = i0 + wi*96 + y*16 + col][j = j0 + wj*96 + x*16 + grp*4 + e],
  // pair position pos = i n + j at res_offset (16 positions' channels contiguous).
  auto at = [&](int64_t pos) { return a.out + res_offset(a.channels, int(ch), pos); };
  const bool vec = (n % 4) == 0;                    // then pos % 4 == 0: 4 positions in one block
#pragma unroll
  for (int y = 0; y < NT; ++y) {
    const int i = i0 + wi * WT + y * 16 + col;
    if (i >= n) continue;
#pragma unroll
    for (int x = 0; x < NT; ++x) {
      const int j = j0 + wj * WT + x * 16 + grp * 4;
      const int64_t pos = int64_t(i) * n + j;
      if (vec && j + 4 <= n) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = bf16(acc[x][y][e]);
        *reinterpret_cast<bf16x4 *>(at(pos)) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (j + e < n) *at(pos + e) = bf16(acc[x][y][e]);
      }
    }
  }
}

}  // namespace

int64_t contraction_ld(int64_t n) { return align_up(n, TK); }
int64_t contraction_operand_elems(int64_t n, int64_t channels) {
  return (contraction_ld(n) / TK) * op_step_stride(n, int(channels));
}
int64_t contraction_result_elems(int64_t n, int64_t channels) {
  return ceil_div(n * n, 16) * res_block_stride(int(channels));
}

int contraction(const ContractionArgs &a, hipStream_t s) {
  if (a.n == 0 || a.channels == 0) return XFH_OK;
  if (a.ld != contraction_ld(a.n)) return fail(XFH_EINVAL, "contraction: operand rows must be padded to 32");
  const int64_t tiles = ceil_div(a.n, TB);
  const int64_t total = tiles * tiles * a.channels;
  const int64_t grid = ceil_div(total, 8) * 8;
  KernelTimer timer("trimul_contract", s);
  contraction_kernel<<<dim3(grid), 256, 0, s>>>(a);
  return check_launch("contraction");
}

}  // namespace xfh
