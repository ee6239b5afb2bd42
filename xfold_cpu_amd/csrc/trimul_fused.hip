// Fused triangle-multiplication kernels (bf16 compute, c = 128), around the per-channel
// contraction (xfold/nn/triangle_multiplication.py:71-105):
//
//   trimul_project: LN_in(z) -> [projection | gate] (one GEMM over both weights' rows) ->
//       mask * proj * sigmoid(gate) -> channel 2k = a_k, 2k+1 = b_k -> written channel-major
//       in the contraction's operand layouts (left/right, see triangle.hip).
//   trimul_output: centre LN over the channel-major contraction result -> output_projection,
//       times sigmoid(gating_linear(LN_in(z))) (recomputed from z, which this kernel reads
//       anyway for the residual) -> z += update (or update stored).
//
// trimul_project is a row-panel kernel (panel.h, 128 pair positions per workgroup, so each
// channel's row of the operand layout is written 256 bytes at a time); trimul_output works
// on register-resident rows (rowstep.h).
#include <algorithm>

#include "common.h"
#include "kernels.h"
#include "panel.h"
#include "rowstep.h"

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
  // Weight row r of chunk j = r / 64 (64 rows): projection rows 32j..32j+15, gate rows
  // 32j..32j+15, projection rows 32j+16..32j+31, gate rows 32j+16..32j+31.
  auto wrow = [&](int r) -> const bf16 * {
    const int j = r >> 6, s4 = (r >> 4) & 3, i = r & 15;
    return ((s4 & 1) ? a.w_gate : a.w_proj) + (32 * j + (s4 >= 2 ? 16 : 0) + i) * K;
  };
  BStage st;
  const int nout = 4 * K;                          // projection + gate, 2c each
  fetch_rows(wrow, 0, st);
  __syncthreads();                                 // A tile consumed; reuse as B buffers
  stash_b(st, bbuf(0));
  __syncthreads();

  bf16 *left = a.left, *right = a.right;
  const int64_t plane = int64_t(n) * a.ld;
  const int chunks = nout / CHUNK;
  for (int j = 0; j < chunks; ++j) {
    if (j + 1 < chunks) fetch_rows(wrow, (j + 1) * CHUNK, st);
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

// trimul_output, one wavefront per 16 positions at a time (rowstep.h), weights resident in
// LDS, activations in registers, no barriers after the weights are in:
//   gate^T = Wg . LN_in(z)^T                  (K-layout z -> O-layout gate logits)
//   c      = contraction result, channel-major: 16-byte loads of 8 positions of a channel
//            are an MFMA A fragment, times an identity B (either k-half) they land in
//            O-layout (exact)
//   y      = bf16(LN_c(c))                    (statistics over the 4 lanes of a position)
//   u^T    = Wout . y^T                       (Wout in kperm order)
//   z     += bf16(u * sigmoid(gate))
template <typename TIN, typename TOUT>
__global__ __launch_bounds__(512, 1) void trimul_output_kernel(TriOutputArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 w_gate[rowstep::W_ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 w_out[rowstep::W_ELEMS];
  __shared__ __attribute__((aligned(16))) float lnw_in[K], lnb_in[K], lnw_c[K], lnb_c[K];
  rowstep::load_weight(a.w_gating, w_gate, false);
  rowstep::load_weight(a.w_out, w_out, true);
  rowstep::load_ln(a.ln_in_w, a.ln_in_b, lnw_in, lnb_in);
  rowstep::load_ln(a.ln_c_w, a.ln_c_b, lnw_c, lnb_c);
  __syncthreads();

  const int64_t npos = int64_t(a.n) * a.n;
  const int64_t steps = (npos + 15) / 16;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int64_t waves = int64_t(gridDim.x) * (blockDim.x >> 6);
  const TIN *z = static_cast<const TIN *>(a.pair);
  TOUT *out = static_cast<TOUT *>(a.out);
  constexpr bool kBf16 = sizeof(TIN) == 2 && sizeof(TOUT) == 2;
  const bool res_from_z = kBf16 && a.accumulate && a.pair == a.out;
  const bool res_load = a.accumulate && !res_from_z;
  const bool c_vec = (npos % 8) == 0;
  bf16x8 id[2];
  rowstep::identity_frags(id);

  struct Rows {
    rowstep::Raw4<TIN> z[8];                       // K-layout
    bf16x8 c[4];                                   // see fetch
    rowstep::Raw4<TOUT> res[8];                    // O-layout (only when not derived from z)
  };
  auto fetch = [&](int64_t st, Rows &rw) {
    const int64_t pos = st * 16 + r, pc = pos < npos ? pos : npos - 1;
    rowstep::load_k<TIN>(z + pc * K, rw.z);
    // c[q]: channel 16 q + r (g < 2) or 16 (q + 4) + r (g >= 2), positions 8 (g % 2) .. +7
    // of the step: k = 8 g + j of an A fragment whose k-halves hold tiles q and q + 4.
    const int64_t p0 = st * 16 + 8 * (g & 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bf16 *src = a.contracted + int64_t(16 * (q + 4 * (g >> 1)) + r) * npos + p0;
      bf16x8 v = {};
      if (c_vec && p0 + 8 <= npos) {
        v = *reinterpret_cast<const bf16x8 *>(src);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (p0 + j < npos) v[j] = src[j];
      }
      rw.c[q] = v;
    }
    if (res_load) rowstep::load_o<TOUT>(out + pc * K, rw.res);
  };

  int64_t st = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  Rows cur;
  if (st < steps) fetch(st, cur);
  for (; st < steps; st += waves) {
    Rows next;
    if (st + waves < steps) fetch(st + waves, next);
    // gate = sigmoid(Wg . LN_in(z))
    float sig[8][4];
    {
      bf16x8 x[4];
      float v[32];
      rowstep::k_to_float(cur.z, v);
      rowstep::ln_k(v, lnw_in, lnb_in, a.eps_in, x);
      f32x4 acc[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      rowstep::gemm_t(w_gate, x, acc);
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) sig[t][e] = sigmoidf_(acc[t][e]);
    }
    // y = LN_c(c), O-layout
    bf16x8 y[4];
    {
      f32x4 co[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        co[q] = mfma16(cur.c[q], id[0], f32x4{0.f, 0.f, 0.f, 0.f});
        co[q + 4] = mfma16(cur.c[q], id[1], f32x4{0.f, 0.f, 0.f, 0.f});
      }
      float v[32];
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * t + e] = co[t][e];
      float mean, rstd;
      rowstep::ln_stats(v, a.eps_c, mean, rstd);
      float yo[8][4];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float4 w = *reinterpret_cast<const float4 *>(lnw_c + 16 * t + 4 * g);
        const float4 b = *reinterpret_cast<const float4 *>(lnb_c + 16 * t + 4 * g);
        const float wv[4] = {w.x, w.y, w.z, w.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) yo[t][e] = (v[4 * t + e] - mean) * rstd * wv[e] + bv[e];
      }
      rowstep::o_to_operand(yo, y);
    }
    f32x4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    rowstep::gemm_t(w_out, y, acc);
    f32x4 res[8];
    if (res_from_z) {
      if constexpr (kBf16) {
        bf16x8 zk[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            zk[ks][e] = cur.z[2 * ks].v[e];
            zk[ks][4 + e] = cur.z[2 * ks + 1].v[e];
          }
        rowstep::k_to_o(id, zk, res);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) res[t][e] = res_load ? cur.res[t][e] : 0.f;
    }
    const int64_t pos = st * 16 + r;
    if (pos < npos) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = res[t][e] + static_cast<float>(bf16(acc[t][e] * sig[t][e]));
        rowstep::store4f<TOUT>(out + pos * K + 16 * t + 4 * g, o);
      }
    }
    cur = next;
  }
}

}  // namespace

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
  const int64_t steps = ceil_div(int64_t(a.n) * a.n, 16);
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const dim3 grid(unsigned(std::min<int64_t>(cus, ceil_div(steps, 8))));
  KernelTimer timer("trimul_output", s);
  if (pair_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    trimul_output_kernel<bf16, bf16><<<grid, 512, 0, s>>>(a);
  else if (pair_dtype == XFH_BF16 && out_dtype == XFH_F32)
    trimul_output_kernel<bf16, float><<<grid, 512, 0, s>>>(a);
  else if (pair_dtype == XFH_F32 && out_dtype == XFH_F32)
    trimul_output_kernel<float, float><<<grid, 512, 0, s>>>(a);
  else
    trimul_output_kernel<float, bf16><<<grid, 512, 0, s>>>(a);
  return check_launch("trimul_output");
}

}  // namespace xfh
