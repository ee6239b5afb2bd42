// Triangle (grid) attention core for bf16, head dim 32: the Pairformer's hot kernel.
//
// For batch row b (a row of the pair grid, or a column for the ending node), head h,
// query t and key s:  o[b,t,h,:] = softmax_s(q.k + bias[h,t,s], keys with mask[b,s]==0
// removed) @ v, which equals xfold/fastnn/attention.py:45-66 with its -1e9 fill whenever
// a row keeps at least one key (a masked key then gets probability exactly 0 in fp32);
// a row whose keys are all masked averages v uniformly over all keys, as -1e9 does.
//
// Operand layouts (written by grid_project):
//   q   [B][H][N][32] bf16, pre-multiplied by d^-0.5 * log2(e)
//   k   [B][H][Npad][32] bf16, zero for keys >= N
//   vt  [B][H][32][Npad] bf16, zero for keys >= N; inside every run of 32 keys, position
//       8g + j holds key 4g + j (j < 4) or 16 + 4g + j - 4 (j >= 4), the key order of a
//       lane's P^T fragment
//   bias [H][N][Npad] fp32, pre-multiplied by log2(e)
//   maskbits [B][Npad/64] uint64: bit s%64 of word s/64 set iff key s < N is kept
//
// One workgroup = one head, 64 queries (4 wavefronts x 16) and R = 4 batch rows; keys go
// in blocks of 64 through a double-buffered LDS stage filled by direct global->LDS loads
// (one barrier per block). Per block:
//   - the bias tile [16 q x 64 keys] is loaded once (prefetched a block ahead) and is the
//     accumulator input of the Q.K^T MFMA of every row: the bias add costs no VALU work;
//   - the MFMA computes S^T = K Q^T, so a lane holds 16 keys of one query, which is the B
//     operand of O^T = V^T P^T without any data movement; a constant ones row appended to
//     V^T makes the same MFMA produce the softmax denominator;
//   - the running maximum is rescaled lazily: o and the denominator are only rescaled
//     when some key's logit exceeds the maximum in use by more than kRescaleSlack (log2
//     units), so exp2(s - m) <= 2^kRescaleSlack always, and the final o / l is the same
//     quotient as with the exact running maximum. The test needs only each lane's own
//     maximum (v_maximum3); the maximum over a query's four lanes (gfx950 permlane
//     swaps) is taken only when rescaling;
//   - the Q.K^T of all rows of the group is issued first, then their softmax and P.V,
//     giving the scheduler independent MFMA and VALU chains;
//   - masked keys of a partly kept block get -1e30 added through one more MFMA per key
//     tile (a rank-1 product), blocks with no kept key are skipped.
// Workgroups are numbered so that one XCD walks the row groups of one head, keeping that
// head's bias in its L2 (from 1024 queries on, in runs of 8 row groups: see below).
#include <string>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int GKB = 64;              // keys per block
constexpr int MB_ZERO = 64;          // zeros read by the lanes that supply no mask value
// Mask words of a row group are kept in registers (lane w holds word w of each row): a
// global read inside the key loop would wait (vmcnt) for the block prefetch issued before it.
constexpr int kMaxKeyBlocks = 64;    // N <= 4096
constexpr float kRescaleSlack = 8.0f;
// Initial running maximum: finite, so that a block whose keys are all masked (logits near
// kMaskedLogit) neither triggers a rescale nor gets any weight, whatever came before it.
constexpr float kInitialMax = -1.0e20f;
constexpr float kMaskedLogit = -1.0e30f;
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

// Workgroup shape: R batch rows, W wavefronts, TQ tiles of 16 queries per wavefront, head
// dim D (16, 32 or 64; other heads are zero-padded to the next). At D = 16 the Q.K^T MFMA
// takes its k = 16 .. 31 half as zeros (the lanes of k-groups 2 and 3 supply zero fragments).
template <int R_, int W_, int TQ_, int D_> struct Shape {
  static constexpr int R = R_, W = W_, TQ = TQ_, D = D_;
  static constexpr int Q = 16 * TQ * W;                     // queries per workgroup
  static constexpr int T = 64 * W;                          // threads
  static constexpr int K_ELEMS = GKB * D;                   // K tile of one row: [64 keys][D]
  static constexpr int V_ELEMS = D * GKB;                   // V^T tile of one row: [D][64 keys]
  static constexpr int STAGE = R * (K_ELEMS + V_ELEMS + GKB); // + one additive mask row per row
  static constexpr int KPIECES = D / 8, PIECES = 2 * KPIECES; // 1 KB direct loads per row
  static constexpr int KPP = 512 / D;                       // keys per K piece
  static constexpr int DT = D / 16;                         // output tiles (+ 1 denominator)
  static constexpr int KS = D == 16 ? 1 : D / 32;           // k-steps of Q.K^T
  static constexpr int BLOCKS = (8 / W) * (R == 1 ? 2 : 1); // workgroups per CU
  static_assert(D == 16 || D == 32 || D == 64, "head dim 16, 32 or 64");
  static_assert(W >= R, "wavefront r writes row r's mask row");
  static_assert(PIECES % W == 0, "each wavefront loads the same number of pieces of a row");
};
using GridShape = Shape<4, 4, 1, 32>;

// K slot swizzle: 16-byte slot s of key j holds chunk s ^ kswz(j), so that the 16 keys of an
// MFMA operand read (one chunk each) hit distinct bank groups for 32-byte (D = 16), 64-byte
// (D = 32) and 128-byte (D = 64) rows.
template <int D> __host__ __device__ constexpr int kswz(int key) {
  return D == 16 ? (key >> 3) & 1 : D == 32 ? (key >> 2) & 3 : (key >> 1) & 7;
}

__device__ __forceinline__ uint32_t xcd_logical(uint32_t physical, uint32_t per_xcd) {
  return (physical % 8) * per_xcd + physical / 8;
}

// IEEE maximum (NaN-propagating): lowers to v_maximum3_f32 with no operand quieting.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Maximum over lanes col, col+16, col+32, col+48 (the four key groups of one query).
__device__ __forceinline__ float query_max(float x) {
  // The swap results pass through an empty asm: without it the compiler folds the float
  // maximum of the two results of a swap to the first one, dropping the exchange.
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  uint32_t p0 = p[0], p1 = p[1];
  asm volatile("" : "+v"(p0), "+v"(p1));
  x = vmax(__builtin_bit_cast(float, p0), __builtin_bit_cast(float, p1));
  u = __builtin_bit_cast(uint32_t, x);
  const auto q = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  uint32_t q0 = q[0], q1 = q[1];
  asm volatile("" : "+v"(q0), "+v"(q1));
  return vmax(__builtin_bit_cast(float, q0), __builtin_bit_cast(float, q1));
}

__device__ __forceinline__ float max16(const f32x4 (&s)[4]) {
  float m = vmax(vmax(s[0][0], s[0][1]), s[0][2]);
  m = vmax(vmax(m, s[0][3]), s[1][0]);
  m = vmax(vmax(m, s[1][1]), s[1][2]);
  m = vmax(vmax(m, s[1][3]), s[2][0]);
  m = vmax(vmax(m, s[2][1]), s[2][2]);
  m = vmax(vmax(m, s[2][3]), s[3][0]);
  m = vmax(vmax(m, s[3][1]), s[3][2]);
  return vmax(m, s[3][3]);
}

template <typename BT> __device__ __forceinline__ f32x4 bias_quad(const BT *p);
template <> __device__ __forceinline__ f32x4 bias_quad<float>(const float *p) {
  return *reinterpret_cast<const f32x4 *>(p);
}
// bf16 bias in natural units: widened and taken to log2 units here.
template <> __device__ __forceinline__ f32x4 bias_quad<bf16>(const bf16 *p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4 *>(p);
  constexpr float kLog2e = 1.4426950408889634f;
  return f32x4{static_cast<float>(v[0]) * kLog2e, static_cast<float>(v[1]) * kLog2e,
               static_cast<float>(v[2]) * kLog2e, static_cast<float>(v[3]) * kLog2e};
}

template <class S, typename BT = float>
__global__ __launch_bounds__(S::T, S::BLOCKS) void grid_attention_kernel(GridAttentionArgs a) {
  constexpr int R = S::R, W = S::W, TQ = S::TQ, GQ = S::Q, STAGE = S::STAGE, D = S::D;
  constexpr int K_ELEMS = S::K_ELEMS, V_ELEMS = S::V_ELEMS, DT = S::DT, KS = S::KS;
  constexpr int PW = S::PIECES / W;                  // pieces of a row per wavefront
  __shared__ __attribute__((aligned(16))) bf16 lds[2 * STAGE + MB_ZERO];
  auto kbuf = [&](int stage, int r) -> bf16 * { return lds + stage * STAGE + r * K_ELEMS; };
  auto vbuf = [&](int stage, int r) -> bf16 * { return lds + stage * STAGE + R * K_ELEMS + r * V_ELEMS; };
  auto mbuf = [&](int stage, int r) -> bf16 * {
    return lds + stage * STAGE + R * (K_ELEMS + V_ELEMS) + r * GKB;
  };
  bf16 *const mzero = lds + 2 * STAGE;

  // 32-bit work decomposition (the launcher keeps the grid below 2^31).
  const uint32_t qblocks = (a.Nq + GQ - 1) / GQ;
  const uint32_t rgroups = (a.B + R - 1) / R;
  const uint32_t total = qblocks * rgroups * uint32_t(a.H);
  const uint32_t logical = xcd_logical(blockIdx.x, (total + 7) / 8);
  if (logical >= total) return;
  // Within a head the query blocks run fastest (the workgroups in flight on an XCD share
  // the K/V of a few row groups). From 1024 queries on, a head's bias no longer fits an
  // XCD's L2, and the head is walked in runs of 8 row groups instead (query block, then row
  // group in the run): the workgroups in flight then read the bias of a few query blocks
  // (measured at N=1536: attention 4.56 -> 4.51 ms per launch; no change at N <= 768).
  int qblk, h, rg;
  if (a.Nq >= 1024 && rgroups % 8 == 0) {
    const uint32_t per_head = qblocks * rgroups, hh = logical / per_head, idx = logical - hh * per_head;
    const uint32_t run = idx / (qblocks * 8), inner = idx - run * (qblocks * 8);
    h = int(hh);
    qblk = int(inner / 8);
    rg = int(run * 8 + inner % 8);
  } else {
    const uint32_t rest = logical / qblocks;
    qblk = int(logical - rest * qblocks);
    h = int(rest / rgroups);
    rg = int(rest - uint32_t(h) * rgroups);
  }

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  // query tile tq of this wavefront: queries q0 + 16 tq + col
  const int q0 = qblk * GQ + wave * 16 * TQ;

  // Per-(row, query tile) state.
  bf16x8 qf[R][TQ][KS];
  f32x4 o[R][TQ][DT + 1];
  float m[R][TQ];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int b = rg * R + r;
#pragma unroll
    for (int tq = 0; tq < TQ; ++tq) {
      const int q = q0 + 16 * tq + col;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        bf16x8 z = {};
        qf[r][tq][ks] = z;
        if (b < a.B && q < a.Nq && (D != 16 || grp < 2))
          qf[r][tq][ks] = *reinterpret_cast<const bf16x8 *>(a.q + ((int64_t(b) * a.H + h) * a.Nq + q) * D + ks * 32 + grp * 8);
      }
#pragma unroll
      for (int t = 0; t <= DT; ++t) o[r][tq][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      m[r][tq] = kInitialMax;
    }
  }
  if (tid < MB_ZERO) mzero[tid] = bf16(0.0f);       // (LDS stores go before any direct load)
  // Lane w holds word w (key block w) of each row of the group.
  uint64_t wr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int b = rg * R + r;
    wr[r] = b < a.B && lane < a.Nblk ? a.maskbits[int64_t(b) * a.mbs + lane] : 0;
  }


  // Swizzled LDS offsets of this lane's K fragments (key kt*16 + col, chunk 4 ks + grp; the
  // swizzle of key kt*16 + col depends on col only) and V^T fragments (row t*16 + col,
  // chunk 4c + grp); the mask fragment (key kt*16 + col in k-slot 0) is read by the grp 0
  // lanes, the others read zeros.
  int kslot[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kslot[ks] = ((4 * ks + grp) ^ kswz<D>(col)) * 8;
  const int vslot[2] = {((0 + grp) ^ ((col >> 1) & 7)) * 8, ((4 + grp) ^ ((col >> 1) & 7)) * 8};

  // A operand of the denominator MFMA: V^T row D = ones, rows D+1..D+15 = zeros.
  // B operand of the mask MFMA: k = 0 is one for every query, the other k are zero.
  bf16x8 ones_a, ones_b;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    ones_a[s] = col == 0 ? bf16(1.0f) : bf16(0.0f);
    ones_b[s] = (grp == 0 && s == 0) ? bf16(1.0f) : bf16(0.0f);
  }

  // One key block goes global -> LDS without passing through registers
  // (global_load_lds_dwordx4: lane i of a wavefront writes bytes [16i, 16i + 16) of a
  // 1 KB LDS segment): per row, D/8 1 KB pieces of K and D/8 of V^T, spread over the
  // wavefronts. The 16-byte slots are XOR-swizzled so that the 16 lanes of an MFMA
  // operand read hit 16 distinct bank groups:
  //   K:   slot s of key j holds its 8-element chunk s ^ kswz(j)
  //   V^T: slot s of row d holds its 8-element chunk s ^ ((d >> 1) & 7)
  // K and V^T are zero for keys >= N (their logits are masked). Each lane's source is a
  // per-(row, block) uniform base plus a per-lane byte offset fixed for the kernel.
  // From the first block that needs the mask on, wavefront r < R also turns row r's mask
  // word into the additive mask row (0 or -1e30), before the loads: an LDS store after
  // them would wait for them to land.
  uint32_t piece_off[PW];                            // bytes, per piece of this wavefront
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int piece = wave + j * W;
    if (piece < S::KPIECES) {                        // keys KPP*piece .., D/8 lanes per key
      const int key = piece * S::KPP + lane / (D / 8), slot = lane % (D / 8);
      piece_off[j] = uint32_t(key * D + (slot ^ kswz<D>(key)) * 8) * 2;
    } else {                                         // V^T rows 8 (piece - KPIECES) ..
      const int d = (piece - S::KPIECES) * 8 + (lane >> 3), vchunk = (lane & 7) ^ ((d >> 1) & 7);
      piece_off[j] = uint32_t(d * a.Npad + vchunk * 8) * 2;
    }
  }
  // Row status, set in the prologue from the mask words (block 0's loads go out before
  // them): a row is present if b < B, active if it also keeps some key; first_masked is the
  // first key block in which some row of the group does not keep all 64 keys.
  bool all_masked[R];
  int active = 0, present = 0, first_masked = 0;
  uint32_t row_lo = 0, row_hi = 0;                   // this wavefront's row word, lane w = block w
  // Additive mask row (0 or -1e30 per key) of block kb for wavefront r < R's row.
  auto mask_row = [&](int kb, int stage) {
    if (kb >= first_masked && wave < R) {
      const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(row_hi), kb));
      const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(row_lo), kb));
      const uint64_t word = (uint64_t(hi) << 32) | lo;
      mbuf(stage, wave)[lane] = ((word >> lane) & 1ull) ? bf16(0.0f) : bf16(kMaskedLogit);
    }
  };
  auto issue_kv = [&](int kb, int stage) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int b = rg * R + r;
      if (b >= a.B) continue;                        // absent row: its tiles are never read
      const int64_t bh = int64_t(b) * a.H + h;
#pragma unroll
      for (int j = 0; j < PW; ++j) {
        const int piece = wave + j * W;
        const bool kp = piece < S::KPIECES;
        const char *base = kp
            ? reinterpret_cast<const char *>(a.k + (bh * a.Npad + int64_t(kb) * GKB) * D)
            : reinterpret_cast<const char *>(a.vt + bh * D * a.Npad + int64_t(kb) * GKB);
        bf16 *dst = kp ? kbuf(stage, r) + piece * 512 : vbuf(stage, r) + (piece - S::KPIECES) * 512;
        __builtin_amdgcn_global_load_lds((global_void *)(base + piece_off[j]), (lds_void *)dst, 16, 0, 0);
      }
    }
  };
  // Block kb into a stage: the mask row first (an LDS store after the direct loads would wait
  // for them), then K and V^T.
  auto issue = [&](int kb, int stage) {
    mask_row(kb, stage);
    issue_kv(kb, stage);
  };
  // Waits for this thread's outstanding global loads (LDS transfers included).
  auto drain = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
  // Bias tile of query tile tq: [16 queries x 64 keys], lane (col, grp) holds keys
  // kt*16 + grp*4 + 0..3 of query q0 + 16 tq + col.
  const BT *bias_rows[TQ];
#pragma unroll
  for (int tq = 0; tq < TQ; ++tq) {
    const int q = q0 + 16 * tq + col;
    bias_rows[tq] = static_cast<const BT *>(a.bias) + (int64_t(h) * a.Nq + (q < a.Nq ? q : a.Nq - 1)) * a.Npad;
  }
  f32x4 bias[TQ][4];
  auto load_bias = [&](int kb) {
#pragma unroll
    for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        bias[tq][kt] = bias_quad<BT>(bias_rows[tq] + kb * GKB + kt * 16 + grp * 4);
  };

  // S^T of row r (+ the additive mask row when masked), both query tiles.
  auto scores = [&](int cur, int r, f32x4 (&s)[TQ][4], bool masked) {
    const bf16 *kr = kbuf(cur, r);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      bf16x8 kf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kf[ks] = *reinterpret_cast<const bf16x8 *>(D == 16 && grp >= 2 ? mzero
                                                                       : kr + (kt * 16 + col) * D + kslot[ks]);
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq) {
        s[tq][kt] = mfma16(kf[0], qf[r][tq][0], bias[tq][kt]);
#pragma unroll
        for (int ks = 1; ks < KS; ++ks) s[tq][kt] = mfma16(kf[ks], qf[r][tq][ks], s[tq][kt]);
      }
    }
    if (masked) {
      const bf16 *mr = grp == 0 ? mbuf(cur, r) + col : mzero;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const uint32_t mv = *reinterpret_cast<const uint16_t *>(grp == 0 ? mr + kt * 16 : mr);
        const bf16x8 mf = __builtin_bit_cast(bf16x8, make_uint4(mv, 0u, 0u, 0u));
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq) s[tq][kt] = mfma16(mf, ones_b, s[tq][kt]);
      }
    }
  };
  // Lazy rescale of (row, tile), called when some lane's maximum exceeds m + slack: the
  // new m is the maximum over the query's four lanes, so it stays the same in all four.
  auto rescale = [&](int r, int tq, float lane_max) {
    const float mn = vmax(m[r][tq], query_max(lane_max));
    const float alpha = __builtin_amdgcn_exp2f(m[r][tq] - mn);
#pragma unroll
    for (int t = 0; t <= DT; ++t) o[r][tq][t] *= alpha;
    m[r][tq] = mn;
  };
  // P = exp2(S - m), then O^T += V^T P^T and l += 1^T P^T, both query tiles.
  auto pv = [&](int cur, int r, const f32x4 (&s)[TQ][4]) {
    bf16x8 pf[TQ][2];
#pragma unroll
    for (int tq = 0; tq < TQ; ++tq)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pf[tq][c][e] = bf16(__builtin_amdgcn_exp2f(s[tq][2 * c][e] - m[r][tq]));
          pf[tq][c][4 + e] = bf16(__builtin_amdgcn_exp2f(s[tq][2 * c + 1][e] - m[r][tq]));
        }
    const bf16 *vr = vbuf(cur, r);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8 *>(vr + (t * 16 + col) * GKB + vslot[c]);
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq) o[r][tq][t] = mfma16(vf, pf[tq][c], o[r][tq][t]);
      }
#pragma unroll
      for (int tq = 0; tq < TQ; ++tq) o[r][tq][DT] = mfma16(ones_a, pf[tq][c], o[r][tq][DT]);
    }
  };
  // Row with every key masked: P = 1 on every key of the block. V^T is zero for keys
  // >= N, so o collects the sum over the keys that exist; the denominator is N.
  auto uniform_pv = [&](int cur, int r) {
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = bf16(1.0f);
    const bf16 *vr = vbuf(cur, r);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8 *>(vr + (t * 16 + col) * GKB + vslot[c]);
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq) o[r][tq][t] = mfma16(vf, ones, o[r][tq][t]);
      }
  };
  // One key block for the whole group: the Q.K^T of all (active) rows first, then the next
  // block's bias into the registers they have just consumed, one rescale test for all
  // rows, then the exponentials and P.V (independent chains the scheduler interleaves).
  // MIXED groups (some rows absent or fully masked) test every row's status.
  auto rows = [&](int cur, int kb, auto masked_c, auto mixed_c) {
    constexpr bool masked = decltype(masked_c)::value, mixed = decltype(mixed_c)::value;
    f32x4 s[R][TQ][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (!mixed || (active & (1 << r))) scores(cur, r, s[r], masked);
    if (kb + 1 < a.Nblk) load_bias(kb + 1);
    float lane_max[R][TQ];
    bool need = false;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (!mixed || (active & (1 << r)))
#pragma unroll
        for (int tq = 0; tq < TQ; ++tq) {
          lane_max[r][tq] = max16(s[r][tq]);
          need = need || lane_max[r][tq] > m[r][tq] + kRescaleSlack;
        }
    if (__any(need)) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (!mixed || (active & (1 << r)))
#pragma unroll
          for (int tq = 0; tq < TQ; ++tq) rescale(r, tq, lane_max[r][tq]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (!mixed || (active & (1 << r))) pv(cur, r, s[r]);
      else if (present & (1 << r)) uniform_pv(cur, r);
    }
  };
  // One key block: prefetch the next one into the other stage, compute, hand over.
  auto step = [&](int kb, auto compute) {
    const int cur = kb & 1;
    if (kb + 1 < a.Nblk) issue(kb + 1, cur ^ 1);   // that stage was last read before the previous barrier
    compute(cur);
    drain();
    __syncthreads();
  };

  // Block 0's K/V and bias go out together with the q and mask-word loads above; one wait.
  issue_kv(0, 0);
  load_bias(0);
  drain();
  // Row status from the mask words, in every wavefront at once.
  uint64_t full_blocks = a.Nblk == 64 ? ~0ull : ((1ull << a.Nblk) - 1);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint64_t w = wr[r];
    const bool any = __ballot(w != 0) != 0;
    full_blocks &= __ballot(w == ~0ull);
    const bool here = rg * R + r < a.B;
    all_masked[r] = here && !any;
    if (here) present |= 1 << r;
    if (here && any) active |= 1 << r;
  }
  first_masked = full_blocks == ~0ull ? a.Nblk : __builtin_ctzll(~full_blocks);
  // This wavefront's row word (wavefront r < R writes row r's additive mask rows).
  uint64_t row_word = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (wave == r) row_word = wr[r];
  row_lo = uint32_t(row_word);
  row_hi = uint32_t(row_word >> 32);
  mask_row(0, 0);                                    // after the wait: no extra wait
  __syncthreads();

  using T_ = std::true_type;
  using F_ = std::false_type;
  const int all_rows = (1 << R) - 1;
  if (active == all_rows) {
    // Leading blocks in which every row keeps every key need no mask; the rest get it.
    int kb = 0;
    for (; kb < first_masked; ++kb) step(kb, [&](int cur) { rows(cur, kb, F_{}, F_{}); });
    for (; kb < a.Nblk; ++kb) step(kb, [&](int cur) { rows(cur, kb, T_{}, F_{}); });
  } else if (active == 0) {
    for (int kb = 0; kb < a.Nblk; ++kb)
      step(kb, [&](int cur) {
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (present & (1 << r)) uniform_pv(cur, r);
      });
  } else {
    for (int kb = 0; kb < a.Nblk; ++kb) step(kb, [&](int cur) { rows(cur, kb, T_{}, T_{}); });
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int b = rg * R + r;
#pragma unroll
    for (int tq = 0; tq < TQ; ++tq) {
      const int q = q0 + 16 * tq + col;
      const float l = __shfl(o[r][tq][DT][0], col, 64);  // denominator sits in lane `col`, grp 0
      if (b >= a.B || q >= a.Nq) continue;
      const float inv = 1.0f / (all_masked[r] ? float(a.N) : l);
      const int64_t off = int64_t(b) * a.osb + int64_t(q) * a.ost + int64_t(h) * a.ohs + grp * 4;
      bf16 *dst = a.out + off;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int d = t * 16 + grp * 4;
        float g[4] = {1.f, 1.f, 1.f, 1.f};
        if (a.gate) {
          if (d + 4 <= a.Dv) {
            const bf16x4 gv = *reinterpret_cast<const bf16x4 *>(a.gate + off + t * 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) g[e] = sigmoidf_(static_cast<float>(gv[e]));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (d + e < a.Dv) g[e] = sigmoidf_(static_cast<float>(a.gate[off + t * 16 + e]));
          }
        }
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = bf16(g[e] * (o[r][tq][t][e] * inv));
        if (d + 4 <= a.Dv) {
          *reinterpret_cast<bf16x4 *>(dst + t * 16) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (d + e < a.Dv) dst[t * 16 + e] = v[e];
        }
      }
    }
  }
}

int64_t grid_attention_pad_(int64_t n) { return align_up(n, GKB); }

template <class S, typename BT = float> int launch(const GridAttentionArgs &a, const char *name, hipStream_t s) {
  if (a.B == 0 || a.Nq == 0 || a.N == 0) return XFH_OK;
  if (a.Nblk > kMaxKeyBlocks) return fail(XFH_EUNSUPPORTED, std::string(name) + ": more than 4096 keys");
  const int64_t qblocks = ceil_div(a.Nq, S::Q), rgroups = ceil_div(a.B, S::R);
  const int64_t total = qblocks * rgroups * a.H;
  const int64_t grid = ceil_div(total, 8) * 8;
  if (grid > (int64_t(1) << 31) - 1) return fail(XFH_EUNSUPPORTED, std::string(name) + ": problem too large");
  // Algorithmic work: Q.K^T and P.V over every (row, head, query, key) at the value head dim.
  KernelTimer timer(name, s, 4.0 * double(a.B) * a.H * a.Nq * a.N * a.Dv, true);
  timer.launch(grid_attention_kernel<S, BT>, dim3(grid), dim3(S::T), 0, a);
  return check_launch(name);
}

}  // namespace

int grid_attention(const GridAttentionArgs &a, hipStream_t s) {
  if (a.bias_bf16) return fail(XFH_EUNSUPPORTED, "grid_attention: fp32 bias only");
  return launch<GridShape>(a, "grid_attention", s);
}

int mha_attention(const GridAttentionArgs &a, int d, hipStream_t s) {
  // Rows (batch entries) per workgroup share the bias tile; a single row keeps more
  // workgroups per CU instead (at head dim 64 always: measured 5% faster on the diffusion
  // transformer's 5 x 16 heads). At head dim 64, 8 wavefronts (128 queries) share each K/V
  // block: 11% faster per call there than 4.
  if (d == 32) {
    if (a.B == 1)
      return a.bias_bf16 ? launch<Shape<1, 4, 1, 32>, bf16>(a, "mha_attention", s)
                         : launch<Shape<1, 4, 1, 32>>(a, "mha_attention", s);
    return a.bias_bf16 ? launch<Shape<4, 4, 1, 32>, bf16>(a, "mha_attention", s)
                       : launch<Shape<4, 4, 1, 32>>(a, "mha_attention", s);
  }
  if (d == 64)
    return a.bias_bf16 ? launch<Shape<1, 8, 1, 64>, bf16>(a, "mha_attention", s)
                       : launch<Shape<1, 8, 1, 64>>(a, "mha_attention", s);
  if (d == 16) {
    if (a.B == 1)
      return a.bias_bf16 ? launch<Shape<1, 4, 1, 16>, bf16>(a, "mha_attention", s)
                         : launch<Shape<1, 4, 1, 16>>(a, "mha_attention", s);
    return a.bias_bf16 ? launch<Shape<4, 4, 1, 16>, bf16>(a, "mha_attention", s)
                       : launch<Shape<4, 4, 1, 16>>(a, "mha_attention", s);
  }
  return fail(XFH_EUNSUPPORTED, "mha_attention: head dim must be 16, 32 or 64");
}

int64_t grid_attention_pad(int64_t n) { return grid_attention_pad_(n); }

int64_t grid_attention_max_n() { return int64_t(kMaxKeyBlocks) * GKB; }

}  // namespace xfh
