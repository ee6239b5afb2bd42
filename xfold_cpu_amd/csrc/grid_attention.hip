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
//   k   [B][H][N][32] bf16
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
//   - the row maximum uses v_maximum3 and the gfx950 permlane swaps (no LDS round trip);
//   - the running maximum is rescaled lazily: o and the denominator are only rescaled
//     when a block's maximum exceeds the one in use by more than kRescaleSlack (log2
//     units), so exp2(s - m) <= 2^kRescaleSlack always, and the final o / l is the same
//     quotient as with the exact running maximum;
//   - the Q.K^T of row r+1 is issued before the softmax of row r, so MFMA and VALU work
//     overlap inside one wavefront;
//   - masked keys of a partly kept block get -1e30 added through one more MFMA per key
//     tile (a rank-1 product), blocks with no kept key are skipped.
// Workgroups are numbered so that one XCD walks the row groups of one head, keeping that
// head's bias in its L2.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int GD = 32;               // head dim
constexpr int GKB = 64;              // keys per block
constexpr int GR = 4;                // batch rows per workgroup
constexpr int K_ELEMS = GKB * GD;    // K tile of one row: [64 keys][32], 64 B per key
constexpr int V_ELEMS = GD * GKB;    // V^T tile of one row: [32 d][64 keys], 128 B per d
constexpr int STAGE_ELEMS = GR * (K_ELEMS + V_ELEMS + GKB);   // + one additive mask row per row
constexpr int MB_ZERO = 64;
// Mask words of a row group are kept in LDS: a global read inside the key loop would wait
// (vmcnt) for the block prefetch issued before it.
constexpr int kMaxKeyBlocks = 64;     // N <= 4096          // zeros read by the lanes that supply no mask value
constexpr float kRescaleSlack = 8.0f;
// Initial running maximum: finite, so that a block whose keys are all masked (logits near
// kMaskedLogit) neither triggers a rescale nor gets any weight, whatever came before it.
constexpr float kInitialMax = -1.0e20f;
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;
constexpr float kMaskedLogit = -1.0e30f;

__device__ __forceinline__ int64_t xcd_logical(int64_t physical, int64_t per_xcd) {
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

__global__ __launch_bounds__(256, 2) void grid_attention_kernel(GridAttentionArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 lds[2 * STAGE_ELEMS + MB_ZERO];
  auto kbuf = [&](int stage, int r) -> bf16 * { return lds + stage * STAGE_ELEMS + r * K_ELEMS; };
  auto vbuf = [&](int stage, int r) -> bf16 * {
    return lds + stage * STAGE_ELEMS + GR * K_ELEMS + r * V_ELEMS;
  };
  auto mbuf = [&](int stage, int r) -> bf16 * {
    return lds + stage * STAGE_ELEMS + GR * (K_ELEMS + V_ELEMS) + r * GKB;
  };
  bf16 *const mzero = lds + 2 * STAGE_ELEMS;         // MB_ZERO zeros
  __shared__ uint64_t words[GR][kMaxKeyBlocks];      // the group's mask words

  const int qblocks = (a.N + 63) / 64;
  const int rgroups = (a.B + GR - 1) / GR;
  const int64_t total = int64_t(qblocks) * rgroups * a.H;
  const int64_t logical = xcd_logical(blockIdx.x, (total + 7) / 8);
  if (logical >= total) return;
  const int qblk = int(logical % qblocks);
  const int rg = int((logical / qblocks) % rgroups);
  const int h = int(logical / (int64_t(qblocks) * rgroups));

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int q = qblk * 64 + wave * 16 + col;
  const int qc = q < a.N ? q : a.N - 1;

  // Per-row state. A row is active if it exists (b < B) and keeps at least one key.
  bf16x8 qf[GR];
  f32x4 o[GR][3];
  float m[GR];
  bool all_masked[GR];
  int active = 0, present = 0;
#pragma unroll
  for (int r = 0; r < GR; ++r) {
    const int b = rg * GR + r;
    bf16x8 z = {};
    qf[r] = z;
    if (b < a.B && q < a.N)
      qf[r] = *reinterpret_cast<const bf16x8 *>(a.q + ((int64_t(b) * a.H + h) * a.N + q) * GD + grp * 8);
#pragma unroll
    for (int t = 0; t < 3; ++t) o[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[r] = kInitialMax;
    uint64_t any = 0;
    if (b < a.B)
      for (int w = 0; w < a.Nblk; ++w) any |= a.maskbits[int64_t(b) * a.Nblk + w];
    all_masked[r] = (b < a.B) && any == 0;
    if (b < a.B) present |= 1 << r;
    if (b < a.B && any != 0) active |= 1 << r;
  }
  if (tid < MB_ZERO) mzero[tid] = bf16(0.0f);
  for (int i = tid; i < GR * a.Nblk; i += 256) {
    const int r = i / a.Nblk, w = i % a.Nblk, b = rg * GR + r;
    words[r][w] = b < a.B ? a.maskbits[int64_t(b) * a.Nblk + w] : 0;
  }

  // Swizzled LDS offsets of this lane's K fragment (key kt*16 + col, chunk grp) and V^T
  // fragments (row t*16 + col, chunk 4c + grp); the mask fragment (key kt*16 + col in
  // k-slot 0) is read by the grp 0 lanes, the others read zeros.
  const int kslot = (grp ^ ((col >> 2) & 3)) * 8;
  const int vslot[2] = {((0 + grp) ^ ((col >> 1) & 7)) * 8, ((4 + grp) ^ ((col >> 1) & 7)) * 8};

  // A operand of the denominator MFMA: V^T row 32 = ones, rows 33..47 = zeros.
  // B operand of the mask MFMA: k = 0 is one for every query, the other k are zero.
  bf16x8 ones_a, ones_b;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    ones_a[s] = col == 0 ? bf16(1.0f) : bf16(0.0f);
    ones_b[s] = (grp == 0 && s == 0) ? bf16(1.0f) : bf16(0.0f);
  }

  // One key block goes global -> LDS without passing through registers
  // (global_load_lds_dwordx4: lane i of a wavefront writes bytes [16i, 16i + 16) of a
  // 1 KB LDS segment). The 16-byte slots are XOR-swizzled so that the 16 lanes of an
  // MFMA operand read hit 16 distinct bank groups:
  //   K:   slot s of key j holds its 8-element chunk s ^ ((j >> 2) & 3)
  //   V^T: slot s of row d holds its 8-element chunk s ^ ((d >> 1) & 7)
  // Keys >= N of K are read from key N-1 (their logits are masked); V^T is zero there.
  // Wavefront r also turns row r's mask word into the additive mask row (0 or -1e30),
  // before the loads: an LDS store after them would wait for them to land.
  auto issue = [&](int kb, int stage) {
    const uint64_t word = words[wave][kb];
    mbuf(stage, wave)[lane] = ((word >> lane) & 1ull) ? bf16(0.0f) : bf16(kMaskedLogit);
#pragma unroll
    for (int r = 0; r < GR; ++r) {
      const int b = rg * GR + r;
      if (b >= a.B) continue;                          // absent row: its tiles are never read
      const int64_t bh = int64_t(b) * a.H + h;
      const int key = kb * GKB + wave * 16 + (lane >> 2);
      const int kchunk = (lane & 3) ^ ((lane >> 4) & 3);
      const bf16 *ksrc = a.k + (bh * a.N + (key < a.N ? key : a.N - 1)) * GD + kchunk * 8;
      __builtin_amdgcn_global_load_lds((global_void *)ksrc, (lds_void *)(kbuf(stage, r) + wave * 16 * GD),
                                       16, 0, 0);
      const int d = wave * 8 + (lane >> 3);
      const int vchunk = (lane & 7) ^ ((d >> 1) & 7);
      const bf16 *vsrc = a.vt + (bh * GD + d) * a.Npad + int64_t(kb) * GKB + vchunk * 8;
      __builtin_amdgcn_global_load_lds((global_void *)vsrc, (lds_void *)(vbuf(stage, r) + wave * 8 * GKB),
                                       16, 0, 0);
    }
  };
  // Waits for this thread's outstanding global loads (LDS transfers included).
  auto drain = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
  const float *bias_row = a.bias + (int64_t(h) * a.N + qc) * a.Npad;
  auto load_bias = [&](int kb, f32x4 (&bias)[4]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
      bias[kt] = *reinterpret_cast<const f32x4 *>(bias_row + kb * GKB + kt * 16 + grp * 4);
  };
  // Every row of the group keeps all 64 keys of block kb.
  auto block_full = [&](int kb) {
    bool full = true;
#pragma unroll
    for (int r = 0; r < GR; ++r) full = full && words[r][kb] == ~0ull;
    return full;
  };

  f32x4 bias[4], bias_next[4];

  // S^T of row r (+ the additive mask row when MASKED) into s.
  auto scores = [&](int cur, int r, f32x4 (&s)[4], bool masked) {
    const bf16 *kr = kbuf(cur, r);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(kr + (kt * 16 + col) * GD + kslot);
      s[kt] = mfma16(kf, qf[r], bias[kt]);
    }
    if (masked) {
      const bf16 *mr = grp == 0 ? mbuf(cur, r) + col : mzero;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const uint32_t mv = *reinterpret_cast<const uint16_t *>(grp == 0 ? mr + kt * 16 : mr);
        const uint4 frag = make_uint4(mv, 0u, 0u, 0u);
        s[kt] = mfma16(__builtin_bit_cast(bf16x8, frag), ones_b, s[kt]);
      }
    }
  };
  // P = exp2(S - m) (lazy rescale), then O^T += V^T P^T and l += 1^T P^T.
  auto softmax_pv = [&](int cur, int r, const f32x4 (&s)[4]) {
    const float mx = query_max(max16(s));
    if (__any(mx > m[r] + kRescaleSlack)) {
      const float mn = vmax(m[r], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[r] - mn);
#pragma unroll
      for (int t = 0; t < 3; ++t) o[r][t] *= alpha;
      m[r] = mn;
    }
    bf16x8 pf[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pf[c][e] = bf16(__builtin_amdgcn_exp2f(s[2 * c][e] - m[r]));
        pf[c][4 + e] = bf16(__builtin_amdgcn_exp2f(s[2 * c + 1][e] - m[r]));
      }
    const bf16 *vr = vbuf(cur, r);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8 *>(vr + (t * 16 + col) * GKB + vslot[c]);
        o[r][t] = mfma16(vf, pf[c], o[r][t]);
      }
      o[r][2] = mfma16(ones_a, pf[c], o[r][2]);
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
      for (int t = 0; t < 2; ++t) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8 *>(vr + (t * 16 + col) * GKB + vslot[c]);
        o[r][t] = mfma16(vf, ones, o[r][t]);
      }
  };
  // All rows active: the Q.K^T of row r+1 is issued before the softmax of row r.
  auto rows_active = [&](int cur, bool masked) {
    f32x4 s0[4], s1[4];
    scores(cur, 0, s0, masked);
#pragma unroll
    for (int r = 0; r < GR; ++r) {
      f32x4 (&sc)[4] = (r & 1) ? s1 : s0;
      f32x4 (&sn)[4] = (r & 1) ? s0 : s1;
      if (r + 1 < GR) scores(cur, r + 1, sn, masked);
      softmax_pv(cur, r, sc);
    }
  };
  // Mixed group (some rows absent or fully masked): row by row.
  auto rows_mixed = [&](int cur) {
#pragma unroll
    for (int r = 0; r < GR; ++r) {
      if (active & (1 << r)) {
        f32x4 sr[4];
        scores(cur, r, sr, true);
        softmax_pv(cur, r, sr);
      } else if (present & (1 << r)) {
        uniform_pv(cur, r);
      }
    }
  };
  // One key block: prefetch the next one into the other stage, compute, hand over.
  auto step = [&](int kb, auto compute) {
    const int cur = kb & 1;
    const bool more = kb + 1 < a.Nblk;
    if (more) {
      issue(kb + 1, cur ^ 1);    // that stage was last read before the previous barrier
      load_bias(kb + 1, bias_next);
    }
    compute(cur);
    drain();
    __syncthreads();
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) bias[kt] = bias_next[kt];
  };

  __syncthreads();                                   // words, mzero
  issue(0, 0);
  load_bias(0, bias);
  drain();
  __syncthreads();

  const int all_rows = (1 << GR) - 1;
  if (active == all_rows) {
    // Leading blocks in which every row keeps every key need no mask; the rest get it.
    int kb = 0;
    for (; kb < a.Nblk && block_full(kb); ++kb) step(kb, [&](int cur) { rows_active(cur, false); });
    for (; kb < a.Nblk; ++kb) step(kb, [&](int cur) { rows_active(cur, true); });
  } else if (active == 0) {
    for (int kb = 0; kb < a.Nblk; ++kb)
      step(kb, [&](int cur) {
#pragma unroll
        for (int r = 0; r < GR; ++r)
          if (present & (1 << r)) uniform_pv(cur, r);
      });
  } else {
    for (int kb = 0; kb < a.Nblk; ++kb) step(kb, rows_mixed);
  }

#pragma unroll
  for (int r = 0; r < GR; ++r) {
    const int b = rg * GR + r;
    const float l = __shfl(o[r][2][0], col, 64);     // denominator sits in lane `col`, grp 0
    if (b >= a.B || q >= a.N) continue;
    const float inv = 1.0f / (all_masked[r] ? float(a.N) : l);
    bf16 *dst = a.out + int64_t(b) * a.osb + int64_t(q) * a.ost + h * GD + grp * 4;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = bf16(o[r][t][e] * inv);
      *reinterpret_cast<bf16x4 *>(dst + t * 16) = v;
    }
  }
}

}  // namespace

int64_t grid_attention_pad(int64_t n) { return align_up(n, GKB); }

int64_t grid_attention_max_n() { return int64_t(kMaxKeyBlocks) * GKB; }

int grid_attention(const GridAttentionArgs &a, hipStream_t s) {
  if (a.B == 0 || a.N == 0) return XFH_OK;
  if (a.Nblk > kMaxKeyBlocks) return fail(XFH_EUNSUPPORTED, "grid_attention: more than 4096 keys");
  const int64_t qblocks = ceil_div(a.N, 64), rgroups = ceil_div(a.B, GR);
  const int64_t total = qblocks * rgroups * a.H;
  const int64_t grid = ceil_div(total, 8) * 8;
  if (grid > (int64_t(1) << 31) - 1) return fail(XFH_EUNSUPPORTED, "grid_attention: problem too large");
  KernelTimer timer("grid_attention", s);
  grid_attention_kernel<<<dim3(grid), 256, 0, s>>>(a);
  return check_launch("grid_attention");
}

}  // namespace xfh
