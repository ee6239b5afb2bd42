// bf16 "NT" GEMM, C[b][m][n] = epilogue(sum_k A[b][m][k] * B[b][n][k]), for the shapes of
// the projections and transitions (k a multiple of 32, 16-byte aligned rows). Same contract
// as gemm_nt (gemm.hip), which keeps every other case.
//
// Tiling: BM x BN output tile per workgroup (BM = 128 or 256, BN = 64 .. 192), 4 wavefronts
// in a 2 x 2 grid each owning BM/2 x BN/2 (BM/32 x BN/32 MFMA 16x16x32 tiles). Per k-step of TK (32 or 64)
// both operand tiles go global -> LDS with direct loads (global_load_lds_dwordx4, no
// registers) into a ring of SLOTS stages: the loads of steps s+1 .. s+SLOTS-1 are in
// flight while step s is multiplied, one barrier per step. A TK-deep row is CH = TK/8
// 16-byte chunks; chunk c of row r sits in slot c ^ sw(r), sw(r) = (r / (16 / CH)) % CH,
// so the 16 rows of an MFMA operand read (one chunk each) hit 16 distinct bank groups.
// Rows past M or N read the last row (their results are never stored).
// The MFMA takes the B rows as its A operand, so a lane ends up with four consecutive
// output columns of one row: bias, auxiliary operand, accumulation and the GLU pairing
// all work on 4-element vectors and the stores are 8 (bf16) or 16 (fp32) bytes.
// The launcher picks the tile width, depth and ring from the problem's shape (more
// workgroups for narrow outputs, deeper k-steps when k allows).
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

template <int BN_, int TK_, int SLOTS_, int WGS_, int BM_ = 128> struct Ring {
  static constexpr int BM = BM_, BN = BN_, TK = TK_, SLOTS = SLOTS_, WGS = WGS_;
  static constexpr int WM = BM / 2;                   // rows per wavefront (2 x 2 wavefront grid)
  static constexpr int MT = WM / 16;                  // MFMA tiles per wavefront along m
  static constexpr int CH = TK / 8;                   // 16-byte chunks per LDS row
  static constexpr int ROWS_PER_PIECE = 1024 / (2 * TK);   // rows per 1 KB direct load
  static constexpr int PIECES = (BM + BN) / ROWS_PER_PIECE; // per k-step
  static constexpr int PPW = PIECES / 4;              // per wavefront
  static constexpr int NT = BN / 32;                  // MFMA tiles per wavefront along n
  static constexpr int KS = TK / 32;                  // MFMA k-substeps per k-step
  static constexpr int SLOT_ELEMS = (BM + BN) * TK;
  static_assert(PIECES % 4 == 0, "direct-load pieces must split evenly over 4 wavefronts");
  static_assert(SLOTS * SLOT_ELEMS * 2 * WGS <= 160 * 1024, "LDS budget");
  __host__ __device__ static constexpr int sw(int r) { return (r / (16 / CH)) % CH; }
};

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

template <int EPI> __device__ __forceinline__ float epilogue(float acc, float c, float aux) {
  if constexpr (EPI == XFH_EPI_MUL_SIGMOID_AUX) return acc * sigmoidf_(aux);
  else if constexpr (EPI == XFH_EPI_SIGMOID_MUL_AUX) return sigmoidf_(acc) * aux;
  else if constexpr (EPI == XFH_EPI_ACCUMULATE) return c + acc;
  else if constexpr (EPI == XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE) return c + acc * sigmoidf_(aux);
  else return acc;
}

// Stores one wavefront's 64 x (16 NT) sub-tile (rows mw + 16 y + col, columns nw + 16 x +
// 4 grp + e) through epilogue EPI. The epilogue kind is a template parameter and the row
// quantities (row divisor, auxiliary row) are taken once per row: a runtime switch per
// element made this code ~10x larger than the main loop, and its instruction-cache misses
// cost ~10 us per launch whatever the grid.
template <int EPI, typename TO, int NT, int MT>
__device__ __forceinline__ void store_tile(const GemmArgs &p, const f32x4 (&acc)[NT][MT], int64_t batch, int mw,
                                           int nw, int col, int grp) {
  constexpr bool READS_C = EPI == XFH_EPI_ACCUMULATE || EPI == XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE;
  constexpr bool AUX = EPI == XFH_EPI_MUL_SIGMOID_AUX || EPI == XFH_EPI_SIGMOID_MUL_AUX ||
                       EPI == XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE;
  TO *C = static_cast<TO *>(p.C) + batch * p.sC;
  int m[MT];
  float rs[MT];
  const TO *arow[MT];
#pragma unroll
  for (int y = 0; y < MT; ++y) {
    m[y] = mw + y * 16 + col;
    rs[y] = p.row_div && m[y] < p.M ? 1.0f / (p.row_div_eps + p.row_div[m[y]]) : 1.0f;
    arow[y] = nullptr;
    if constexpr (AUX) {
      const int ar = p.aux_rows > 0 ? m[y] % int(p.aux_rows) : m[y];
      arow[y] = static_cast<const TO *>(p.aux) + batch * p.sAux + int64_t(ar) * p.ldaux;
    }
  }
  if (p.pair_blk == 0 && mw + 16 * MT <= p.M && nw + 16 * NT <= p.N) {
    // Interior sub-tile (every tile of the usual shapes): straight-line code, no per-element
    // bounds, row-major addresses.
#pragma unroll
    for (int x = 0; x < NT; ++x) {
      const int n = nw + x * 16 + grp * 4;
      float bias[4] = {0.f, 0.f, 0.f, 0.f};
      if (p.bias)
#pragma unroll
        for (int e = 0; e < 4; ++e) bias[e] = p.bias[batch * p.sBias + n + e];
#pragma unroll
      for (int y = 0; y < MT; ++y) {
        TO *c = C + int64_t(m[y]) * p.ldc + n;
        float cv[4] = {0.f, 0.f, 0.f, 0.f}, av[4] = {0.f, 0.f, 0.f, 0.f}, out[4];
        if constexpr (READS_C) Vec4<TO>::load(c, cv);
        if constexpr (AUX) Vec4<TO>::load(arow[y] + n, av);
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = epilogue<EPI>((acc[x][y][e] + bias[e]) * rs[y], cv[e], av[e]);
        Vec4<TO>::store(c, out);
      }
    }
    return;
  }
#pragma unroll
  for (int x = 0; x < NT; ++x) {
    const int n = nw + x * 16 + grp * 4;
    if (n >= p.N) continue;
    const bool full = n + 4 <= p.N;
    float bias[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.bias)
#pragma unroll
      for (int e = 0; e < 4; ++e) bias[e] = n + e < p.N ? p.bias[batch * p.sBias + n + e] : 0.f;
#pragma unroll
    for (int y = 0; y < MT; ++y) {
      if (m[y] >= p.M) continue;
      TO *c = c_element(p, C, m[y], n);
      float cv[4] = {0.f, 0.f, 0.f, 0.f}, av[4] = {0.f, 0.f, 0.f, 0.f}, out[4];
      if (full) {
        if constexpr (READS_C) Vec4<TO>::load(c, cv);
        if constexpr (AUX) Vec4<TO>::load(arow[y] + n, av);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (n + e >= p.N) continue;
          if constexpr (READS_C) cv[e] = to_f32(c[e]);
          if constexpr (AUX) av[e] = to_f32(arow[y][n + e]);
        }
      }
      // (acc + bias) * 1.0f is exact, so rows without a divisor keep acc + bias.
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] = epilogue<EPI>((acc[x][y][e] + bias[e]) * rs[y], cv[e], av[e]);
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

// Position of key t inside the attention kernel's V^T rows: within each run of 32 keys,
// key 4g + j goes to 8g + j and key 16 + 4g + j to 8g + 4 + j (g, j < 4).
__device__ __forceinline__ int vt_position(int t) {
  const int w = t & 31;
  return (t & ~31) + ((w & 15) >> 2) * 8 + ((w >> 4) << 2) + (w & 3);
}

// Store epilogue into the attention-operand layouts (AttnOut): (acc + bias), times qscale
// for the q columns. Four consecutive columns share one part and head (Dh % 4 == 0): q, k
// and gate take one 8-byte store, V^T four 2-byte stores (one per head-dim row).
template <int NT, int MT>
__device__ __forceinline__ void store_attn(const GemmArgs &p, const f32x4 (&acc)[NT][MT], int mw, int nw, int col,
                                           int grp) {
  const AttnOut &o = p.attn;
  const int c = o.H * o.Dh;
  int smp[MT], tok[MT];                                 // per row: sample b and token t
#pragma unroll
  for (int y = 0; y < MT; ++y) {
    const int m = mw + y * 16 + col;
    smp[y] = m / o.T;
    tok[y] = m - smp[y] * o.T;
  }
#pragma unroll
  for (int x = 0; x < NT; ++x) {
    const int n = nw + x * 16 + grp * 4;
    if (n >= p.N) continue;
    const int part = n / c, w = n - part * c, h = w / o.Dh, d = w - h * o.Dh;
    const float scale = part == 0 ? o.qscale : 1.0f;
    float bias[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.bias)
#pragma unroll
      for (int e = 0; e < 4; ++e) bias[e] = p.bias[n + e];
#pragma unroll
    for (int y = 0; y < MT; ++y) {
      if (mw + y * 16 + col >= p.M) continue;
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = bf16((acc[x][y][e] + bias[e]) * scale);
      const int64_t bh = int64_t(smp[y]) * o.H + h;
      if (part == 0) {
        *reinterpret_cast<bf16x4 *>(o.q + (bh * o.T + tok[y]) * o.Dp + d) = v;
      } else if (part == 1) {
        *reinterpret_cast<bf16x4 *>(o.k + (bh * o.Tpad + tok[y]) * o.Dp + d) = v;
      } else if (part == 2) {
        bf16 *dst = o.vt + (bh * o.Dp + d) * o.Tpad + vt_position(tok[y]);
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[int64_t(e) * o.Tpad] = v[e];
      } else {
        *reinterpret_cast<bf16x4 *>(o.gate + (int64_t(smp[y]) * o.T + tok[y]) * c + w) = v;
      }
    }
  }
}

// V^T tiles of an attention projection computed with swapped MFMA operands (acc[x][y][e] =
// C[mw + y*16 + grp*4 + e][nw + x*16 + col]): keys t0 .. t0+3 of one head-dim row sit at 4
// consecutive V^T positions (t0 % 4 == 0), one 8-byte store each.
template <int NT, int MT>
__device__ __forceinline__ void store_attn_vt(const GemmArgs &p, const f32x4 (&acc)[NT][MT], int mw, int nw, int col,
                                              int grp) {
  const AttnOut &o = p.attn;
  const int c = o.H * o.Dh;
  int smp[MT], pos[MT];
#pragma unroll
  for (int y = 0; y < MT; ++y) {
    const int t0 = mw + y * 16 + grp * 4;
    smp[y] = t0 / o.T;
    pos[y] = vt_position(t0 - smp[y] * o.T);
  }
#pragma unroll
  for (int x = 0; x < NT; ++x) {
    const int n = nw + x * 16 + col, w = n - 2 * c, h = w / o.Dh, d = w - h * o.Dh;
    const float bias = p.bias ? p.bias[n] : 0.f;
#pragma unroll
    for (int y = 0; y < MT; ++y) {
      if (mw + y * 16 + grp * 4 >= p.M) continue;   // M = B*T is a multiple of 4 here
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = bf16(acc[x][y][e] + bias);
      *reinterpret_cast<bf16x4 *>(o.vt + ((int64_t(smp[y]) * o.H + h) * o.Dp + d) * o.Tpad + pos[y]) = v;
    }
  }
}

template <class G, int N> __device__ __forceinline__ void wait_younger(int younger) {
  // Waits until at most `younger` k-steps of this wavefront's loads are in flight.
  if constexpr (N == 0) {
    wait_vmcnt<0>();
  } else {
    if (younger >= N) wait_vmcnt<N * G::PPW>();
    else wait_younger<G, N - 1>(younger);
  }
}

// ATTN: the attention-operand output (AttnOut, bf16, store epilogue) instead of C.
template <typename TO, bool GLU, class G, bool XCD = false, bool ATTN = false>
__global__ __launch_bounds__(256, G::WGS) void gemm_ring_kernel(GemmArgs p) {
  constexpr int BM = G::BM, BN = G::BN, TK = G::TK, SLOTS = G::SLOTS, CH = G::CH, NT = G::NT;
  constexpr int RPP = G::ROWS_PER_PIECE, PPW = G::PPW, WN = BN / 2, WM = G::WM, MT = G::MT;
  __shared__ __attribute__((aligned(16))) bf16 lds[SLOTS * G::SLOT_ELEMS];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
  // With XCD the grid is 1-D and workgroup i runs on XCD i % 8 (workgroups are dealt
  // round-robin to the 8 XCDs). The output's tiles are split into 8 / g row groups times g
  // column groups (g = xcd_split); XCD x takes rectangle x, row-major inside it, so each
  // XCD's L2 holds the A row blocks and B column tiles of one rectangle rather than a
  // scatter over all of them. Workgroups past a rectangle's edge exit at once.
  int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  if constexpr (XCD) {
    const int tn = (p.N + BN - 1) / BN, tm = (p.M + BM - 1) / BM;
    const int gn = p.xcd_split, gm = 8 / gn;
    const int cn = (tn + gn - 1) / gn, cm = (tm + gm - 1) / gm;
    const int xcd = int(blockIdx.x % 8), local = int(blockIdx.x / 8);
    const int n_lo = (xcd % gn) * cn, m_lo = (xcd / gn) * cm;
    const int w = min(cn, tn - n_lo), h = min(cm, tm - m_lo);
    if (w <= 0 || h <= 0 || local >= w * h) return;
    m0 = (m_lo + local / w) * BM;
    n0 = (n_lo + local % w) * BN;
  }
  const int64_t batch = blockIdx.z;
  const bf16 *A = static_cast<const bf16 *>(p.A) + batch * p.sA;
  const bf16 *B = static_cast<const bf16 *>(p.B) + batch * p.sB;

  // Piece q of a k-step covers rows RPP q .. of the [A rows; B rows] stage; lane -> row
  // RPP q + lane / CH, LDS slot lane % CH holding chunk (lane % CH) ^ sw(row).
  const bf16 *src[PPW];
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    const int q = wave + 4 * j;
    const int row = q * RPP + lane / CH;
    const int chunk = (lane % CH) ^ G::sw(row);
    if (row < BM) {
      const int m = m0 + row;
      src[j] = A + int64_t(m < p.M ? m : p.M - 1) * p.lda + chunk * 8;
    } else {
      const int n = n0 + row - BM;
      src[j] = B + int64_t(n < p.N ? n : p.N - 1) * p.ldb + chunk * 8;
    }
  }
  auto issue = [&](int step, int slot) {
#pragma unroll
    for (int j = 0; j < PPW; ++j) {
      const int q = wave + 4 * j;
      bf16 *dst = lds + slot * G::SLOT_ELEMS + q * RPP * TK;
      __builtin_amdgcn_global_load_lds((global_void *)(src[j] + step * TK), (lds_void *)dst, 16, 0, 0);
    }
  };

  // Fragment offset of (row base + col, k-substep ks, chunk 4 ks + grp) for a row base that
  // is a multiple of 16: the swizzle depends on col only.
  int frag[G::KS];
#pragma unroll
  for (int ks = 0; ks < G::KS; ++ks) frag[ks] = col * TK + ((4 * ks + grp) ^ G::sw(col)) * 8;

  f32x4 acc[NT][MT];   // [x][y]: rows n (A operand = B rows), cols m (B operand = A rows)
#pragma unroll
  for (int x = 0; x < NT; ++x)
#pragma unroll
    for (int y = 0; y < MT; ++y) acc[x][y] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int steps = p.K / TK;
#pragma unroll
  for (int s = 0; s < SLOTS - 1; ++s)
    if (s < steps) issue(s, s);
  // TR swaps the MFMA operands: acc[x][y][e] then holds C[m = .. + y*16 + grp*4 + e][n = ..
  // + x*16 + col], four consecutive rows of one column (the V^T tiles of an attention
  // projection, stored as 4 consecutive keys of one head-dim row).
  auto main_loop = [&](auto tr_c) {
    constexpr bool TR = decltype(tr_c)::value;
    for (int s = 0; s < steps; ++s) {
      // This wavefront's loads of step s have landed (the younger steps may still fly), then
      // every wavefront's have, and every wavefront is done with step s - 1.
      const int younger = steps - 1 - s;
      wait_younger<G, SLOTS - 2>(younger);
      ring_barrier();
      if (s + SLOTS - 1 < steps) issue(s + SLOTS - 1, (s + SLOTS - 1) % SLOTS);
      const bf16 *ta = lds + (s % SLOTS) * G::SLOT_ELEMS, *tb = ta + BM * TK;
#pragma unroll
      for (int ks = 0; ks < G::KS; ++ks) {
        bf16x8 fa[MT], fb[NT];
#pragma unroll
        for (int y = 0; y < MT; ++y) fa[y] = *reinterpret_cast<const bf16x8 *>(ta + (wm * WM + y * 16) * TK + frag[ks]);
#pragma unroll
        for (int x = 0; x < NT; ++x) {
          fb[x] = *reinterpret_cast<const bf16x8 *>(tb + (wn * WN + x * 16) * TK + frag[ks]);
#pragma unroll
          for (int y = 0; y < MT; ++y)
            acc[x][y] = TR ? mfma16(fa[y], fb[x], acc[x][y]) : mfma16(fb[x], fa[y], acc[x][y]);
        }
      }
    }
  };
  static_assert(!ATTN || (!GLU && std::is_same<TO, bf16>::value), "attention output: bf16 store only");
  constexpr bool kAttnOut = ATTN;
  bool vt_tile = false;
  if constexpr (kAttnOut) {
    // A workgroup whose columns all fall in the V part writes V^T in 8-byte key runs when
    // groups of 4 rows never straddle two samples (T % 4 == 0).
    const int c = p.attn.H * p.attn.Dh;
    vt_tile = p.attn.T % 4 == 0 && n0 >= 2 * c && n0 + BN <= 3 * c;
  }
  if (vt_tile) {
    if constexpr (kAttnOut) {
      main_loop(std::true_type{});
      store_attn_vt(p, acc, m0 + wm * WM, n0 + wn * WN, col, grp);
    }
    return;
  }
  main_loop(std::false_type{});

  // acc[x][y][e] = C[m = m0 + wm*WM + y*16 + col][n = n0 + wn*WN + x*16 + grp*4 + e]
  TO *C = static_cast<TO *>(p.C) + batch * p.sC;
  if constexpr (GLU) {
    // Packed GLU weight: 32-column groups = 16 gate columns then the 16 matching value
    // columns, so tiles (0, 1) and (2, 3) of a wavefront hold gate/value of the same features.
    static_assert(!GLU || NT % 2 == 0, "GLU pairs whole 32-column groups");
#pragma unroll
    for (int q = 0; q < NT / 2; ++q) {
      const int f = (n0 + wn * WN) / 2 + q * 16 + grp * 4;
#pragma unroll
      for (int y = 0; y < MT; ++y) {
        const int m = m0 + wm * WM + y * 16 + col;
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
  const int mw = m0 + wm * WM, nw = n0 + wn * WN;
  if constexpr (ATTN) {
    store_attn(p, acc, mw, nw, col, grp);
    return;
  }
  switch (p.epi) {
    case XFH_EPI_MUL_SIGMOID_AUX:
      store_tile<XFH_EPI_MUL_SIGMOID_AUX, TO, NT>(p, acc, batch, mw, nw, col, grp);
      break;
    case XFH_EPI_SIGMOID_MUL_AUX:
      store_tile<XFH_EPI_SIGMOID_MUL_AUX, TO, NT>(p, acc, batch, mw, nw, col, grp);
      break;
    case XFH_EPI_ACCUMULATE:
      store_tile<XFH_EPI_ACCUMULATE, TO, NT>(p, acc, batch, mw, nw, col, grp);
      break;
    case XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE:
      store_tile<XFH_EPI_MUL_SIGMOID_AUX_ACCUMULATE, TO, NT>(p, acc, batch, mw, nw, col, grp);
      break;
    default:
      store_tile<XFH_EPI_STORE, TO, NT>(p, acc, batch, mw, nw, col, grp);
  }
}

bool aligned(const void *ptr, int bytes) { return reinterpret_cast<uintptr_t>(ptr) % bytes == 0; }

}  // namespace

// Ring configurations (tile width, k-step, stages, workgroups per CU).
using RingMid = Ring<96, 64, 2, 2>;       // 3/4-width tiles: more workgroups for narrow outputs
using RingNarrow = Ring<64, 64, 3, 2>;    // N <= 64, or too few workgroups otherwise
using RingShallow = Ring<128, 32, 4, 2>;  // k % 64 != 0
using RingShallowNarrow = Ring<64, 32, 4, 2>;
using RingXWide = Ring<192, 64, 2, 2>;     // 1.5x-width tiles: one round where 96 needs two
using RingSkinny = Ring<64, 64, 2, 3>;     // k = 64 (one step) over many tiles: three workgroups per CU

template <class G>
int launch_ring(const GemmArgs &p, int64_t batch, int out_dtype, bool glu, hipStream_t s, KernelTimer &timer) {
  const int64_t tiles = ceil_div(p.N, G::BN) * ceil_div(p.M, G::BM);
  if (tiles > (int64_t(1) << 30)) return fail(XFH_EUNSUPPORTED, "gemm_ring: too many tiles");
  dim3 grid(unsigned(ceil_div(p.N, G::BN)), unsigned(ceil_div(p.M, G::BM)), unsigned(batch));
  if (p.xcd_split) {
    const int64_t gn = p.xcd_split, gm = 8 / gn;
    grid = dim3(unsigned(8 * ceil_div(ceil_div(p.N, G::BN), gn) * ceil_div(ceil_div(p.M, G::BM), gm)), 1,
                unsigned(batch));
  }
  if (glu) {
    if constexpr (G::NT % 2 == 0) {
      if (p.xcd_split) {
        if (out_dtype == XFH_BF16) timer.launch(gemm_ring_kernel<bf16, true, G, true>, dim3(grid), dim3(256), 0, p);
        else timer.launch(gemm_ring_kernel<float, true, G, true>, dim3(grid), dim3(256), 0, p);
      } else {
        if (out_dtype == XFH_BF16) timer.launch(gemm_ring_kernel<bf16, true, G>, dim3(grid), dim3(256), 0, p);
        else timer.launch(gemm_ring_kernel<float, true, G>, dim3(grid), dim3(256), 0, p);
      }
    } else {
      return fail(XFH_EUNSUPPORTED, "gemm_ring: GLU needs whole 32-column groups per wavefront");
    }
  } else if (p.attn.q) {
    if (out_dtype != XFH_BF16) return fail(XFH_EUNSUPPORTED, "gemm_ring: the attention layouts are bf16");
    if (p.xcd_split) timer.launch(gemm_ring_kernel<bf16, false, G, true, true>, dim3(grid), dim3(256), 0, p);
    else timer.launch(gemm_ring_kernel<bf16, false, G, false, true>, dim3(grid), dim3(256), 0, p);
  } else if (p.xcd_split) {
    if (out_dtype == XFH_BF16) timer.launch(gemm_ring_kernel<bf16, false, G, true>, dim3(grid), dim3(256), 0, p);
    else timer.launch(gemm_ring_kernel<float, false, G, true>, dim3(grid), dim3(256), 0, p);
  } else {
    if (out_dtype == XFH_BF16) timer.launch(gemm_ring_kernel<bf16, false, G>, dim3(grid), dim3(256), 0, p);
    else timer.launch(gemm_ring_kernel<float, false, G>, dim3(grid), dim3(256), 0, p);
  }
  return check_launch("gemm_ring");
}

enum class RingPick { Mid, Narrow, Shallow, ShallowNarrow, XWide, Skinny };

// Tile width: the 64-column tile (the only one with a 3-stage ring at two workgroups per
// CU) unless the grid then needs more rounds of workgroups than a wider tile would, rounds
// weighted by the tile's width (measured on the diffusion transformer's Linears: the
// 64-column tile is fastest whenever it fits in one round, the 96-column tile on
// 3840 x 2304 outputs; the 192-column tile wherever it needs one round fewer: the diffusion
// QKV Linear and GLU, 0.5% and 1.9% of a diffusion transformer). 64-deep k-steps when k
// allows. GLU pairs whole 32-column groups per wavefront, so it takes 64 or 192. A
// 128-column tile with 64-deep steps never wins this cost: a 128-column grid needs at
// least half the rounds of the 64-column one, so it is not built. A single 64-deep k-step
// over more than four rounds of tiles (the 64-channel pair widths' Linears over N^2 rows)
// runs three workgroups per CU with a 2-slot ring: each tile is one load, one step and its
// store, so more tiles in flight hide more of that latency (template block at N=768: its
// Linears 1309 -> 1221 us).
RingPick pick_ring(const GemmArgs &p, int64_t batch, bool glu, int cus) {
  const int64_t mt = ceil_div(p.M, 128) * batch, slots = 2 * int64_t(cus);
  auto rounds = [&](int bn) { return ceil_div(mt * ceil_div(p.N, bn), slots); };
  if (p.K == 64 && rounds(64) > 4) return RingPick::Skinny;
  if (p.K % 64 != 0) return (p.N <= 64 || rounds(64) <= 1) ? RingPick::ShallowNarrow : RingPick::Shallow;
  if (p.N <= 64 || rounds(64) <= 1) return RingPick::Narrow;
  RingPick best = RingPick::Narrow;
  int64_t cost = rounds(64) * 64;
  if (!glu && rounds(96) * 96 <= cost) {
    best = RingPick::Mid;
    cost = rounds(96) * 96;
  }
  if (p.N % 192 == 0 && rounds(192) * 192 <= cost) best = RingPick::XWide;
  return best;
}

bool gemm_ring_supported(const GemmArgs &p, int out_dtype) {
  const int ob = out_dtype == XFH_BF16 ? 2 : 4;
  if (p.pair_blk && (p.pair_blk % 4 || !aligned(p.C, 4 * ob) || p.sC % 4)) return false;
  const bool vec_out = p.ldc % 4 == 0 && p.sC % 4 == 0 && aligned(p.C, 4 * ob) &&
                       (!p.aux || (p.ldaux % 4 == 0 && p.sAux % 4 == 0 && aligned(p.aux, 4 * ob)));
  return p.K > 0 && p.K % 32 == 0 && p.aux_rows <= INT32_MAX && p.lda % 8 == 0 && p.ldb % 8 == 0 && p.sA % 8 == 0 &&
         p.sB % 8 == 0 && aligned(p.A, 16) && aligned(p.B, 16) && vec_out;
}

int gemm_ring(const GemmArgs &p, int64_t batch, int out_dtype, bool glu, hipStream_t s) {
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  KernelTimer timer("gemm_ring", s, 2.0 * double(p.M) * double(p.N) * double(p.K) * double(batch), true);
  const RingPick pick = pick_ring(p, batch, glu, cus);
  const int bn = pick == RingPick::XWide ? 192 : pick == RingPick::Shallow ? 128 : pick == RingPick::Mid ? 96 : 64;
  // Per-XCD row runs when row blocks span several tiles, the whole B operand fits comfortably
  // in one XCD's 4 MB L2 and the grid covers every CU (measured: 8% on 3840 x 768 outputs;
  // slower when B crowds the L2 or a row block is one tile).
  GemmArgs q = p;
  q.xcd_split = (!glu && p.K % 64 == 0 && int64_t(p.N) * p.K * 2 <= (int64_t(5) << 19) && p.N > bn &&
                 ceil_div(p.M, 128) * ceil_div(p.N, bn) >= cus) ? 1 : 0;
  // The configuration is observable through the kernel timer of that name.
  static const char *const names[6][2] = {{"gemm_ring.mid", "gemm_ring.mid+xcd"},
                                          {"gemm_ring.narrow", "gemm_ring.narrow+xcd"},
                                          {"gemm_ring.shallow", "gemm_ring.shallow+xcd"},
                                          {"gemm_ring.shallow_narrow", "gemm_ring.shallow_narrow+xcd"},
                                          {"gemm_ring.xwide", "gemm_ring.xwide+xcd"},
                                          {"gemm_ring.skinny", "gemm_ring.skinny+xcd"}};
  KernelTimer config_timer(names[int(pick)][q.xcd_split ? 1 : 0], s);
  switch (pick) {
    case RingPick::Mid: return launch_ring<RingMid>(q, batch, out_dtype, glu, s, timer);
    case RingPick::XWide: return launch_ring<RingXWide>(q, batch, out_dtype, glu, s, timer);
    case RingPick::Skinny: return launch_ring<RingSkinny>(q, batch, out_dtype, glu, s, timer);
    case RingPick::Narrow: return launch_ring<RingNarrow>(q, batch, out_dtype, glu, s, timer);
    case RingPick::Shallow: return launch_ring<RingShallow>(q, batch, out_dtype, glu, s, timer);
    default: return launch_ring<RingShallowNarrow>(q, batch, out_dtype, glu, s, timer);
  }
}

}  // namespace xfh
