// Fused projection and output kernels around the triangle-attention core (bf16 compute,
// c = 128, 4 heads x 32), following GridSelfAttention.forward (xfold/nn/attention.py:80-105):
//
//   grid_project: LN(z) -> GEMMs over the q, k, v and bias weights (resident in LDS) -> q
//       scaled by d^-0.5 * log2(e), k (rows up to npad, zero beyond n), v^T (zero
//       beyond n, keys permuted in runs of 32), the fp32 pair bias (times log2(e)) and the
//       kept-key words, each written straight into the attention kernel's layout
//       (grid_attention.hip). The bias comes from the un-transposed pair in both directions.
//   grid_output: gate = sigmoid(LN(z) Wgating^T) (recomputed: z is read here anyway for
//       the residual) -> (gate * o) Wout^T -> z += update (or update stored).
#include <algorithm>

#include "common.h"
#include "kernels.h"
#include "panel.h"
#include "rowstep.h"

namespace xfh {

namespace {

using namespace panel;

constexpr int HD = 32;                 // head dim
constexpr int QKV_ROWS = 3 * K;        // q, k, v weight rows in LDS, then the bias rows

// grid_project, one wavefront per unit of 32 attention positions t0 .. t0 + 31 of one batch
// row b (t0 a multiple of 32, t up to npad so the pad rows and columns come out as zeros),
// the q, k, v and bias weight rows resident in LDS (rowstep.h layout), the next unit's rows
// loaded while this one is computed, no barriers after the weights are in. Row m of row tile
// rt is position t0 + 16 rt + m.
//   q, k:  out^T = W x^T with W's rows permuted inside each 32-channel head (tile 2s + p, row
//          r = channel 32 s + 8 (r / 4) + 4 p + r % 4), so the lane holding rows 4 g .. of
//          both tiles of head s has its channels 32 s + 8 g .. + 7: one 16-byte store;
//   v^T:   out = x W^T, whose lane (channel, g) holds keys 4 g + e (tile 0) and 16 + 4 g + e
//          (tile 1): exactly the 8 keys of positions t0 + 8 g .. + 7 of the permuted layout;
//   bias:  out = x W^T, 4 consecutive keys per lane (starting node) or one value per
//          (query t, key b) (ending node).
constexpr int W_ROWS = QKV_ROWS + 16;  // q, k, v, then one tile of bias rows (heads <= 16)

template <typename TIN>
__global__ __launch_bounds__(512, 1) void grid_project_kernel(GridProjectArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 w_lds[W_ROWS * K];
  __shared__ __attribute__((aligned(16))) float lnw[K], lnb[K];
  rowstep::WeightStage<W_ROWS, 512> sw;
  rowstep::LnStage sl;
  sw.load([&](int r) -> const bf16 * {
    const int blk = r / K, rr = r % K;              // q, k, v, bias
    if (blk < 2) {                                  // q, k: rows permuted inside each head
      const int t = rr / 16, e = rr % 16;
      return (blk == 0 ? a.wq : a.wk) + (32 * (t / 2) + 8 * (e / 4) + 4 * (t % 2) + (e % 4)) * K;
    }
    if (blk == 2) return a.wv + rr * K;
    return rr < a.heads ? a.wb + rr * K : nullptr;
  }, false);
  sl.load(a.ln_w, a.ln_b);

  const int n = a.n, H = a.heads, npad = a.npad, upr = npad / 32;
  const int units = n * upr;
  const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
  const int waves = int(gridDim.x) * int(blockDim.x >> 6);
  // The attention kernel's kept-key words: word w of row b has bit i set iff key 64 w + i < n
  // is kept (mask[b*n + key] != 0); one wavefront ballot per word.
  {
    const int nblk = npad / 64;
    for (int wd = int(blockIdx.x) * int(blockDim.x >> 6) + int(threadIdx.x >> 6); wd < n * nblk; wd += waves) {
      const int b = wd / nblk, key = (wd - b * nblk) * 64 + lane;
      const bool keep = key < n && (!a.mask || load_any(a.mask, a.mask_dtype, int64_t(b) * n + key) != 0.f);
      const uint64_t ballot = __ballot(keep);
      if (lane == 0) a.maskbits[wd] = ballot;
    }
  }
  const TIN *z = static_cast<const TIN *>(a.pair);
  // Pair row of attention position (b, t): b*n + t (starting node) or t*n + b (ending node).
  auto pos_of = [&](int b, int t) -> int64_t { return a.transpose ? int64_t(t) * n + b : int64_t(b) * n + t; };
  struct Unit {
    rowstep::Raw4<TIN> z[2][8];
  };
  auto fetch = [&](int u, Unit &w) {
    const int b = u / upr, t0 = (u - b * upr) * 32;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int t = t0 + 16 * rt + m;
      rowstep::load_k<TIN>(z + pos_of(b, t < n ? t : n - 1) * K, w.z[rt]);
    }
  };
  int u = int(blockIdx.x) * int(blockDim.x >> 6) + int(threadIdx.x >> 6);
  Unit cur;
  if (u < units) fetch(u, cur);                     // in flight while the weights are stored
  sw.store(w_lds);
  sl.store(lnw, lnb);
  __syncthreads();
  for (; u < units; u += waves) {
    Unit next;
    if (u + waves < units) fetch(u + waves, next);
    bf16x8 xa[2][4];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float v[32];
      rowstep::k_to_float(cur.z[rt], v);
      rowstep::ln_k(v, lnw, lnb, a.eps, xa[rt]);
    }
    const int b = u / upr, t0 = (u - b * upr) * 32;

    // q (rows < n) and k (rows < npad, zero from n on): [b][h][rows][32].
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const bf16 *wb = w_lds + blk * K * K;
      const float scale = blk == 0 ? a.qscale : 1.0f;
      const int rows = blk == 0 ? n : npad;
      bf16 *dst_base = blk == 0 ? a.q : a.k;
#pragma unroll 1
      for (int s = 0; s < H; ++s) {
        f32x4 acc[2][2];
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) acc[p][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const bf16x8 wf = rowstep::weight_frag(wb, 2 * s + p, ks);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) acc[p][rt] = mfma16(wf, xa[rt][ks], acc[p][rt]);
          }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int t = t0 + 16 * rt + m;
          if (t >= rows) continue;
          bf16x8 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = bf16(acc[0][rt][e] * scale);
            v[4 + e] = bf16(acc[1][rt][e] * scale);
          }
          if (t >= n) v = bf16x8{};
          *reinterpret_cast<bf16x8 *>(dst_base + ((int64_t(b) * H + s) * rows + t) * HD + 8 * g) = v;
        }
      }
    }

    // v^T: [b][h][d][npad], keys permuted in runs of 32 (zero from n on).
    {
      const bf16 *wv = w_lds + 2 * K * K;
#pragma unroll 1
      for (int tile = 0; tile < K / 16; ++tile) {
        f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8 wf = rowstep::weight_frag(wv, tile, ks);
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) acc[rt] = mfma16(xa[rt][ks], wf, acc[rt]);
        }
        const int c = tile * 16 + m, h = c / HD, d = c % HD;
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = t0 + 4 * g + e < n ? bf16(acc[0][e]) : bf16(0.0f);
          v[4 + e] = t0 + 16 + 4 * g + e < n ? bf16(acc[1][e]) : bf16(0.0f);
        }
        *reinterpret_cast<bf16x8 *>(a.vt + ((int64_t(b) * H + h) * HD + d) * npad + t0 + 8 * g) = v;
      }
    }

    // Bias, from the un-transposed pair: bias[h][i][j] for pair (i, j) = (b, t) starting node,
    // (t, b) ending node; the pad columns j in [n, npad) are zeros.
    {
      const bf16 *wbias = w_lds + QKV_ROWS * K;
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 wf = rowstep::weight_frag(wbias, 0, ks);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) acc[rt] = mfma16(xa[rt][ks], wf, acc[rt]);
      }
      if (m < H) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int tb = t0 + 16 * rt + 4 * g;        // keys / queries tb .. tb + 3
          if (!a.transpose) {
            float4 v;
            v.x = tb + 0 < n ? acc[rt][0] * kLog2e : 0.f;
            v.y = tb + 1 < n ? acc[rt][1] * kLog2e : 0.f;
            v.z = tb + 2 < n ? acc[rt][2] * kLog2e : 0.f;
            v.w = tb + 3 < n ? acc[rt][3] * kLog2e : 0.f;
            *reinterpret_cast<float4 *>(a.bias + (int64_t(m) * n + b) * npad + tb) = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int t = tb + e;
              if (t >= n) continue;
              float *row = a.bias + (int64_t(m) * n + t) * npad;
              row[b] = acc[rt][e] * kLog2e;
              if (b == n - 1)
                for (int j = n; j < npad; ++j) row[j] = 0.0f;
            }
          }
        }
      }
    }
    cur = next;
  }
}

// grid_output, one wavefront per 16 positions at a time (rowstep.h): the gating and
// output weights stay in LDS for the workgroup's lifetime, the activations never leave
// the registers, and there is no barrier after the weights are in.
//   gate^T = Wg . LN(z)^T              (K-layout z -> O-layout gate)
//   y      = bf16(sigmoid(gate) * o)   (o: attention output rows, K-layout loads moved to
//                                       O-layout by identity MFMAs)
//   u^T    = Wout . y^T                (y is the k operand as it stands, Wout in kperm order)
//   z     += bf16(u)                   (bf16 pair updated in place: the residual is the z
//                                       already loaded, moved to O-layout the same way)
template <typename TIN, typename TOUT>
__global__ __launch_bounds__(512, 1) void grid_output_kernel(GridOutputArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 w_gate[rowstep::W_ELEMS];
  __shared__ __attribute__((aligned(16))) bf16 w_out[rowstep::W_ELEMS];
  __shared__ __attribute__((aligned(16))) float lnw[K], lnb[K];
  rowstep::WeightStage<K, 512> sg, so;
  rowstep::LnStage sl;
  sg.load([&](int row) { return a.w_gating + row * K; }, false);
  so.load([&](int row) { return a.w_out + row * K; }, true);
  sl.load(a.ln_w, a.ln_b);

  const int64_t npos = int64_t(a.n) * a.n;
  const int64_t steps = (npos + 15) / 16;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int64_t waves = int64_t(gridDim.x) * (blockDim.x >> 6);
  const TIN *z = static_cast<const TIN *>(a.pair);
  TOUT *out = static_cast<TOUT *>(a.out);
  // In-place bf16 update: the residual is the z this kernel reads anyway.
  constexpr bool kBf16 = sizeof(TIN) == 2 && sizeof(TOUT) == 2;
  const bool res_from_z = kBf16 && a.accumulate && a.pair == a.out;
  const bool res_load = a.accumulate && !res_from_z;
  bf16x8 id[2];
  rowstep::identity_frags(id);

  struct Rows {
    rowstep::Raw4<TIN> z[8];                       // K-layout
    bf16x8 att[4];                                 // K-layout
    rowstep::Raw4<TOUT> res[8];                    // O-layout (only when not derived from z)
  };
  auto fetch = [&](int64_t st, Rows &rw) {
    const int64_t pos = st * 16 + r, pc = pos < npos ? pos : npos - 1;
    rowstep::load_k<TIN>(z + pc * K, rw.z);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) rw.att[ks] = *reinterpret_cast<const bf16x8 *>(a.attn + pc * K + 32 * ks + 8 * g);
    if (res_load) rowstep::load_o<TOUT>(out + pc * K, rw.res);
  };
  // Rows of the next step are loaded while this one is computed.
  int64_t st = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  Rows cur;
  if (st < steps) fetch(st, cur);                   // in flight while the weights are stored
  sg.store(w_gate);
  so.store(w_out);
  sl.store(lnw, lnb);
  __syncthreads();
  for (; st < steps; st += waves) {
    Rows next;
    if (st + waves < steps) fetch(st + waves, next);
    bf16x8 x[4];
    {
      float v[32];
      rowstep::k_to_float(cur.z, v);
      rowstep::ln_k(v, lnw, lnb, a.eps, x);
    }
    f32x4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    rowstep::gemm_t(w_gate, x, acc);
    f32x4 att[8];
    rowstep::k_to_o(id, cur.att, att);
    float y[8][4];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) y[t][e] = sigmoidf_(acc[t][e]) * att[t][e];
    rowstep::o_to_operand(y, x);
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    rowstep::gemm_t(w_out, x, acc);
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
        for (int e = 0; e < 4; ++e) o[e] = res[t][e] + static_cast<float>(bf16(acc[t][e]));  // bf16 update
        rowstep::store4f<TOUT>(out + pos * K + 16 * t + 4 * g, o);
      }
    }
    cur = next;
  }
}

}  // namespace

int grid_project(const GridProjectArgs &a, int pair_dtype, hipStream_t s) {
  if (a.npad % 64 != 0 || a.npad < a.n || a.heads > 16 || a.heads * HD != K)
    return fail(XFH_EINVAL, "grid_project: npad must be a multiple of 64 >= n, heads * 32 == 128");
  const int64_t units = int64_t(a.n) * (a.npad / 32);
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const dim3 grid(unsigned(balanced_grid(units, 8, cus)));
  KernelTimer timer("grid_project", s, 0.0, true);
  if (pair_dtype == XFH_BF16)
    timer.launch(grid_project_kernel<bf16>, dim3(grid), dim3(512), 0, a);
  else
    timer.launch(grid_project_kernel<float>, dim3(grid), dim3(512), 0, a);
  return check_launch("grid_project");
}

int grid_output(const GridOutputArgs &a, int pair_dtype, int out_dtype, hipStream_t s) {
  const int64_t steps = ceil_div(int64_t(a.n) * a.n, 16);
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const dim3 grid(unsigned(balanced_grid(steps, 8, cus)));
  KernelTimer timer("grid_output", s, 0.0, true);
  if (pair_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    timer.launch(grid_output_kernel<bf16, bf16>, dim3(grid), dim3(512), 0, a);
  else if (pair_dtype == XFH_BF16 && out_dtype == XFH_F32)
    timer.launch(grid_output_kernel<bf16, float>, dim3(grid), dim3(512), 0, a);
  else if (pair_dtype == XFH_F32 && out_dtype == XFH_F32)
    timer.launch(grid_output_kernel<float, float>, dim3(grid), dim3(512), 0, a);
  else
    timer.launch(grid_output_kernel<float, bf16>, dim3(grid), dim3(512), 0, a);
  return check_launch("grid_output");
}

}  // namespace xfh
