// Fused triangle-multiplication kernels (bf16 compute, c = 128), around the per-channel
// contraction (xfold/nn/triangle_multiplication.py:71-105):
//
//   trimul_project: LN_in(z) -> [projection | gate] (one GEMM over both weights' rows) ->
//       mask * proj * sigmoid(gate) -> channel 2k = a_k, 2k+1 = b_k -> written in the
//       contraction's blocked operand layout (left/right; kernels.h).
//   trimul_output: centre LN over the blocked contraction result -> output_projection,
//       times sigmoid(gating_linear(LN_in(z))) (recomputed from z, which this kernel reads
//       anyway for the residual) -> z += update (or update stored).
//
// Both work on register-resident rows (rowstep.h) with their weights resident in LDS.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "panel.h"
#include "rowstep.h"

namespace xfh {

namespace {

using namespace panel;

// trimul_project, one wavefront per unit of 16 RT positions (x, y0 .. y0 + 16 RT - 1) at a
// time (y0 a multiple of 16 RT, y up to ld: the pad columns n <= y < ld come out as zeros), the
// projection and gate weights resident in LDS (rowstep.h layout), the next unit's rows
// loaded while this one is computed, no barriers after the weights are in:
//   x      = bf16(LN_in(z))                    RT K-layout sets (row tiles rt < RT)
//   p, g   = x . Wproj^T, x . Wgate^T          rows = positions, 16 channels per tile
//   out    = p * sigmoid(g) * mask             channel 2k -> a_k, 2k + 1 -> b_k
// With RT = 2, row m of row tile rt is position y0 + 8 (m / 4) + 4 rt + m % 4, so that the
// lane that holds channel c of rows 4 g .. 4 g + 3 in both tiles has positions y0 + 8 g .. + 7
// of c: one 16-byte store into the blocked operand layout (kernels.h), where the 16 grid
// lines x of one row group and the 32 positions of a k-slice of all channels form one block.
// RT = 1 (row m = position y0 + m, 8-byte stores) halves the unit for grids too small to
// give every wavefront several 32-position units.
constexpr int PROJ = 2 * K;          // projection (and gate) output channels

template <typename TIN, int RT>
__global__ __launch_bounds__(512, 1) void trimul_project_kernel(TriProjectArgs a) {
  constexpr int UP = 16 * RT;                       // positions per unit
  // Position offset (in the unit) of row m of row tile rt, and of output element i < 4 RT
  // of a lane in channel-tile group g.
  auto row_y = [](int rt, int m) { return RT == 2 ? 8 * (m >> 2) + 4 * rt + (m & 3) : m; };
  __shared__ __attribute__((aligned(16))) bf16 w_proj[PROJ * K];
  __shared__ __attribute__((aligned(16))) bf16 w_gate[PROJ * K];
  __shared__ __attribute__((aligned(16))) float lnw[K], lnb[K];
  rowstep::WeightStage<PROJ, 512> sp, sg;
  rowstep::LnStage sl;
  sp.load([&](int row) { return a.w_proj + row * K; }, false);
  sg.load([&](int row) { return a.w_gate + row * K; }, false);
  sl.load(a.ln_w, a.ln_b);

  // Unit u = (grid line x = u % n, positions y0 = (u / n) UP ..): the wavefronts of a
  // workgroup take neighbouring grid lines of one k-slice, whose operand rows are
  // neighbours in the blocked layout.
  const int n = a.n, cpr = a.ld / UP;               // units per grid line
  const int units = n * cpr;                        // < 2^31 (n * ld fits in 32 bits)
  const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
  const int waves = int(gridDim.x) * int(blockDim.x >> 6);
  const TIN *z = static_cast<const TIN *>(a.pair);
  // Pair position of grid-line entry (x, y): (x, y) outgoing, (y, x) incoming.
  auto pos_of = [&](int x, int y) -> int64_t { return a.outgoing ? int64_t(x) * n + y : int64_t(y) * n + x; };

  struct Unit {
    rowstep::Raw4<TIN> z[RT][8];                    // K-layout rows of the row tiles
    float mrow[RT];                                 // mask of those rows (0 for y >= n)
  };
  auto fetch = [&](int u, Unit &w) {
    const int y0 = (u / n) * UP, x = u - (u / n) * n;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int y = y0 + row_y(rt, m);
      const int64_t pos = pos_of(x, y < n ? y : n - 1);
      rowstep::load_k<TIN>(z + pos * K, w.z[rt]);
      w.mrow[rt] = y >= n ? 0.f : a.mask ? load_any(a.mask, a.mask_dtype, pos) : 1.f;
    }
  };
  int u = int(blockIdx.x) * int(blockDim.x >> 6) + int(threadIdx.x >> 6);
  Unit cur;
  if (u < units) fetch(u, cur);                     // in flight while the weights are stored
  sp.store(w_proj);
  sg.store(w_gate);
  sl.store(lnw, lnb);
  __syncthreads();
  for (; u < units; u += waves) {
    Unit next;
    if (u + waves < units) fetch(u + waves, next);
    bf16x8 xa[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float v[32];
      rowstep::k_to_float(cur.z[rt], v);
      rowstep::ln_k(v, lnw, lnb, a.eps, xa[rt]);
    }
    // Mask of output rows 4 g + e of tile rt: held by A-row lane 4 g + e.
    float mk[4 * RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int e = 0; e < 4; ++e) mk[4 * rt + e] = __shfl(cur.mrow[rt], 4 * g + e, 64);
    const int y0 = (u / n) * UP, x = u - (u / n) * n;
    const int y_lane = y0 + 4 * RT * g;             // positions y_lane .. + 4 RT - 1
    // k-slice y_lane / 32 of row x of channel 0; channel ch adds 512 ch.
    const int64_t row_off = op_offset(n, K, 0, x, y_lane >> 5) + (y_lane & 31);
    const bool pad = y0 + UP > n;
#pragma unroll 1
    for (int t = 0; t < PROJ / 16; ++t) {
      f32x4 ap[RT], ag[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) ap[rt] = ag[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 wp = rowstep::weight_frag(w_proj, t, ks), wg = rowstep::weight_frag(w_gate, t, ks);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          ap[rt] = mfma16(xa[rt][ks], wp, ap[rt]);
          ag[rt] = mfma16(xa[rt][ks], wg, ag[rt]);
        }
      }
      using Out = std::conditional_t<RT == 2, bf16x8, bf16x4>;
      Out o;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[4 * rt + e] = bf16(ap[rt][e] * sigmoidf_(ag[rt][e]) * mk[4 * rt + e]);
      if (pad) {
#pragma unroll
        for (int e = 0; e < 4 * RT; ++e)
          if (y_lane + e >= n) o[e] = bf16(0.0f);
      }
      const int p = 16 * t + m;                     // projection channel
      const bool is_a = (p & 1) == 0;
      bf16 *dst = ((a.outgoing != 0) == is_a ? a.left : a.right) + (p >> 1) * 512 + row_off;
      *reinterpret_cast<Out *>(dst) = o;
    }
    cur = next;
  }
}

// trimul_output, one wavefront per 16 positions at a time (rowstep.h), weights resident in
// LDS, activations in registers, no barriers after the weights are in:
//   gate^T = Wg . LN_in(z)^T                  (K-layout z -> O-layout gate logits)
//   c      = contraction result, blocked (kernels.h): the 16 positions' channels are one
//            contiguous 4 KB block; 16-byte loads of 8 positions of a channel are an MFMA A
//            fragment, times an identity B (either k-half) they land in O-layout (exact)
//   y      = bf16(LN_c(c))                    (statistics over the 4 lanes of a position)
//   u^T    = Wout . y^T                       (Wout in kperm order)
//   z     += bf16(u * sigmoid(gate))
template <typename TIN, typename TOUT>
__global__ __launch_bounds__(512, 1) void trimul_output_kernel(TriOutputArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 w_gate[rowstep::W_ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 w_out[rowstep::W_ELEMS];
  __shared__ __attribute__((aligned(16))) float lnw_in[K], lnb_in[K], lnw_c[K], lnb_c[K];
  rowstep::WeightStage<K, 512> sg, so;
  rowstep::LnStage sl_in, sl_c;
  sg.load([&](int row) { return a.w_gating + row * K; }, false);
  so.load([&](int row) { return a.w_out + row * K; }, true);
  sl_in.load(a.ln_in_w, a.ln_in_b);
  sl_c.load(a.ln_c_w, a.ln_c_b);

  const int64_t npos = int64_t(a.n) * a.n;
  const int64_t steps = (npos + 15) / 16;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int64_t waves = int64_t(gridDim.x) * (blockDim.x >> 6);
  const TIN *z = static_cast<const TIN *>(a.pair);
  TOUT *out = static_cast<TOUT *>(a.out);
  constexpr bool kBf16 = sizeof(TIN) == 2 && sizeof(TOUT) == 2;
  const bool res_from_z = kBf16 && a.accumulate && a.pair == a.out;
  const bool res_load = a.accumulate && !res_from_z;
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
      const bf16 *src = a.contracted + res_offset(K, 16 * (q + 4 * (g >> 1)) + r, p0);
      bf16x8 v = {};
      if (p0 + 8 <= npos) {
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
  if (st < steps) fetch(st, cur);                   // in flight while the weights are stored
  sg.store(w_gate);
  so.store(w_out);
  sl_in.store(lnw_in, lnb_in);
  sl_c.store(lnw_c, lnb_c);
  __syncthreads();
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
  if (a.ld != contraction_ld(a.n)) return fail(XFH_EINVAL, "trimul_project: ld must be contraction_ld(n)");
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  // 32-position units unless that leaves fewer than four per wavefront (the last round of
  // units would then run on a fraction of the wavefronts).
  const int64_t units32 = int64_t(a.n) * (a.ld / 32);
  const bool wide = units32 >= int64_t(cus) * 8 * 4;
  const int64_t units = wide ? units32 : 2 * units32;
  const dim3 grid(unsigned(balanced_grid(units, 8, cus)));
  KernelTimer timer("trimul_project", s, 0.0, true);
  if (pair_dtype == XFH_BF16) {
    if (wide) timer.launch(trimul_project_kernel<bf16, 2>, dim3(grid), dim3(512), 0, a);
    else timer.launch(trimul_project_kernel<bf16, 1>, dim3(grid), dim3(512), 0, a);
  } else {
    if (wide) timer.launch(trimul_project_kernel<float, 2>, dim3(grid), dim3(512), 0, a);
    else timer.launch(trimul_project_kernel<float, 1>, dim3(grid), dim3(512), 0, a);
  }
  return check_launch("trimul_project");
}

int trimul_output(const TriOutputArgs &a, int pair_dtype, int out_dtype, hipStream_t s) {
  const int64_t steps = ceil_div(int64_t(a.n) * a.n, 16);
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const dim3 grid(unsigned(balanced_grid(steps, 8, cus)));
  KernelTimer timer("trimul_output", s, 0.0, true);
  if (pair_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    timer.launch(trimul_output_kernel<bf16, bf16>, dim3(grid), dim3(512), 0, a);
  else if (pair_dtype == XFH_BF16 && out_dtype == XFH_F32)
    timer.launch(trimul_output_kernel<bf16, float>, dim3(grid), dim3(512), 0, a);
  else if (pair_dtype == XFH_F32 && out_dtype == XFH_F32)
    timer.launch(trimul_output_kernel<float, float>, dim3(grid), dim3(512), 0, a);
  else
    timer.launch(trimul_output_kernel<float, bf16>, dim3(grid), dim3(512), 0, a);
  return check_launch("trimul_output");
}

}  // namespace xfh
