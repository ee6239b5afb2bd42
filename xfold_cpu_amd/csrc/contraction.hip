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
// Tiling: 192 x 384 output tiles, one workgroup of 8 wavefronts per CU (N <= 1024), or
// 192 x 192 tiles, two workgroups of 4 wavefronts per CU; each wavefront owns 96 x 96 (6 x 6
// MFMA 16x16x32 tiles). Per k-step of 32 both operand tiles go global -> LDS with
// global_load_lds_dwordx4 (no registers) into a ring of 4 or 3 slots, so the loads of the
// next 2 or 1 steps are in flight while step s is multiplied; one barrier per step. Rows
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

constexpr int WT = 96;                  // wavefront tile edge
constexpr int NT = WT / 16;             // MFMA tiles per wavefront edge (6)
constexpr int TK = 32;                  // k-step
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

template <int N> __device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most `younger` k-steps of this wavefront's loads (P each) are in flight.
template <int P, int MAXY> __device__ __forceinline__ void wait_younger(int younger) {
  if constexpr (MAXY == 0) {
    wait_vmcnt<0>();
  } else {
    if (younger >= MAXY) wait_vmcnt<MAXY * P>();
    else wait_younger<P, MAXY - 1>(younger);
  }
}

// TBI x TBJ output tiles (rows i of L, rows j of R), 2 x WJ wavefronts of WT x WT each,
// SLOTS ring stages, WGS workgroups per CU.
template <int TBI_, int TBJ_, int WJ_, int SLOTS_, int WGS_> struct Tiling {
  static constexpr int TBI = TBI_, TBJ = TBJ_, WJ = WJ_, W = 2 * WJ_, SLOTS = SLOTS_, WGS = WGS_;
  static constexpr int RBI = TBI / 16, RBJ = TBJ / 16;   // 16-row (1 KB) blocks per operand tile
  static constexpr int PIECES = RBI + RBJ;               // 1 KB direct loads per k-step
  static constexpr int PMAX = (PIECES + W - 1) / W;      // per wavefront (the first PIECES % W one more)
  static constexpr int SLOT_ELEMS = (TBI + TBJ) * TK;
  static_assert(TBI == 2 * WT && TBJ == WJ * WT, "wavefront grid");
  static_assert(SLOTS * SLOT_ELEMS * 2 * WGS <= 160 * 1024, "LDS budget");
};
// 192 x 192, two independent workgroups per CU.
using TileSquare = Tiling<192, 192, 2, 3, 2>;
// 192 x 384, one workgroup of 8 wavefronts per CU: each R row band serves twice the
// columns, so a k-step moves 36 instead of 48 KB of operands per CU for the same MFMAs.
using TileWide = Tiling<192, 384, 4, 4, 1>;

template <class T>
__global__ __launch_bounds__(64 * T::W, T::WGS) void contraction_kernel(ContractionArgs a) {
  constexpr int TBI = T::TBI, TBJ = T::TBJ, WJ = T::WJ, W = T::W, SLOTS = T::SLOTS;
  constexpr int RBI = T::RBI, PIECES = T::PIECES, PMAX = T::PMAX, SLOT_ELEMS = T::SLOT_ELEMS;
  __shared__ __attribute__((aligned(16))) bf16 lds[SLOTS * SLOT_ELEMS];
  const int n = a.n, ld = a.ld;
  const int tiles_i = (n + TBI - 1) / TBI, tiles_j = (n + TBJ - 1) / TBJ;
  const int64_t per_channel = int64_t(tiles_i) * tiles_j;
  const int64_t total = per_channel * a.channels;
  const int64_t per_xcd = (total + 7) / 8;
  const int64_t logical = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (logical >= total) return;
  const int64_t ch = logical / per_channel;
  const int tile = int(logical % per_channel);
  const int i0 = (tile / tiles_j) * TBI, j0 = (tile % tiles_j) * TBJ;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wi = wave / WJ, wj = wave % WJ, col = lane & 15, grp = lane >> 4;
  // k-step s of row g of channel ch at op_offset(n, c, ch, g, 0) + s * step_stride.
  const int64_t step_stride = op_step_stride(n, a.channels);

  // Piece p of a k-step (wavefront w loads p = w, w + W, ...): L row block p (p < RBI) or R
  // row block p - RBI, 16 rows each (one 1 KB block); lane -> row 16 (block) + lane / 4, LDS
  // slot lane % 4 holding chunk (lane % 4) ^ ((lane >> 4) & 3). Rows beyond n read row n-1
  // (their results are never stored).
  const int chunk = (lane & 3) ^ ((lane >> 4) & 3);
  const bool full = wave < PIECES - (PMAX - 1) * W;  // this wavefront loads PMAX pieces
  const bf16 *src[PMAX];
#pragma unroll
  for (int j = 0; j < PMAX; ++j) {
    const int p = wave + W * j < PIECES ? wave + W * j : PIECES - 1;
    const bool lp = p < RBI;
    const int g = (lp ? i0 + p * 16 : j0 + (p - RBI) * 16) + (lane >> 2);
    src[j] = (lp ? a.left : a.right) + op_offset(n, a.channels, int(ch), g < n ? g : n - 1, 0) + chunk * 8;
  }
  auto issue = [&](int step, int slot) {
#pragma unroll
    for (int j = 0; j < PMAX; ++j) {
      const int p = wave + W * j;
      if (p >= PIECES) continue;
      bf16 *dst = lds + slot * SLOT_ELEMS + p * 16 * TK;   // L blocks, then R blocks
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
#pragma unroll
  for (int s = 0; s < SLOTS - 1; ++s)
    if (s < steps) issue(s, s);
  for (int s = 0; s < steps; ++s) {
    // This wavefront's loads of step s have landed (those of the younger steps, up to
    // SLOTS - 2 of them, may still fly), then every wavefront's have, and every wavefront
    // is done with step s-1.
    const int younger = steps - 1 - s < SLOTS - 2 ? steps - 1 - s : SLOTS - 2;
    if (full) wait_younger<PMAX, SLOTS - 2>(younger);
    else wait_younger<PMAX - 1, SLOTS - 2>(younger);
    ring_barrier();
    if (s + SLOTS - 1 < steps) issue(s + SLOTS - 1, (s + SLOTS - 1) % SLOTS);
    const bf16 *tl = lds + (s % SLOTS) * SLOT_ELEMS, *tr = tl + TBI * TK;
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

template <class T> int launch(const ContractionArgs &a, hipStream_t s) {
  const int64_t total = ceil_div(a.n, T::TBI) * ceil_div(a.n, T::TBJ) * a.channels;
  const int64_t grid = ceil_div(total, 8) * 8;
  KernelTimer timer("trimul_contract", s, 2.0 * double(a.channels) * a.n * a.n * a.n, true);
  timer.launch(contraction_kernel<T>, dim3(grid), dim3(64 * T::W), 0, a);
  return check_launch("contraction");
}

// Wide tiles up to N = 1024: measured (same box, libraries alternated) the C2 block (N=384)
// 0.579 -> 0.553 ms and the N=768 contraction 155 -> 152 us; at N=1536 the square tile's
// two independent workgroups per CU are 7% faster.
constexpr int kWideTileMaxN = 1024;

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
  return a.n <= kWideTileMaxN ? launch<TileWide>(a, s) : launch<TileSquare>(a, s);
}

}  // namespace xfh
