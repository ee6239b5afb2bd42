// Pair-logits attention biases straight from the pair tensor (bf16 compute, c = 128):
//   packed[h][i][j] = log2(e) * sum_k LN(z[i][j])[k] * W[h][k]   (j < n; 0 for n <= j < npad)
// in fp32, or the sum itself rounded to bf16 (the dtype of the reference's autocast Linear
// output; the attention kernel applies log2(e) after widening it),
// i.e. Linear(LayerNorm(pair)) rearranged 'i j h -> h i j' into the attention kernel's bias
// layout (grid_attention.hip: [H][Nq][Npad] fp32 times log2(e)), for
//   - PairformerBlock's single-track attention bias (xfold/nn/pairformer.py:103-106), and
//   - DiffusionTransformer's pair logits (xfold/nn/diffusion_transformer.py:258-271), all
//     super-blocks' projections stacked into one weight, so the pair is read once.
//
// One wavefront per unit of 32 pair positions (i, j0 .. j0 + 31) (j0 a multiple of 32, j up
// to npad so the pad columns come out as zeros), the projection weight resident in LDS
// (rowstep.h layout), the next unit's rows loaded while this one is computed, no barriers
// after the weight is in. Row m of row tile rt is position j0 + 16 rt + m, so out = x W^T
// leaves 4 consecutive keys of one head in a lane: one 16-byte store per head and tile.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "rowstep.h"

namespace xfh {

namespace {

constexpr int K = rowstep::C;          // pair channels
constexpr int MAX_HEADS = 384;         // LDS rows of the projection weight
constexpr float kLog2eF = 1.4426950408889634f;

template <typename TIN, typename TOUT>
__global__ __launch_bounds__(512, 1) void pair_bias_kernel(PairBiasArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 w_lds[MAX_HEADS * K];
  __shared__ __attribute__((aligned(16))) float lnw[K], lnb[K];
  const int tiles = (a.heads + 15) / 16;
  rowstep::WeightStage<MAX_HEADS, 512> sw;          // rows >= heads are zeros
  rowstep::LnStage sl;
  sw.load([&](int r) { return r < a.heads ? a.w + int64_t(r) * K : nullptr; }, false);
  sl.load(a.ln_w, a.ln_b);

  const int n = a.n, npad = a.npad, upr = npad / 32;
  const int units = n * upr;
  const int lane = threadIdx.x & 63, m = lane & 15, g = lane >> 4;
  const int waves = int(gridDim.x) * int(blockDim.x >> 6);
  const TIN *z = static_cast<const TIN *>(a.pair);
  struct Unit {
    rowstep::Raw4<TIN> z[2][8];
  };
  auto fetch = [&](int u, Unit &w) {
    const int i = u / upr, j0 = (u - i * upr) * 32;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int j = j0 + 16 * rt + m;
      rowstep::load_k<TIN>(z + (int64_t(i) * n + (j < n ? j : n - 1)) * K, w.z[rt]);
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
    const int i = u / upr, j0 = (u - i * upr) * 32;
#pragma unroll 1
    for (int t = 0; t < tiles; ++t) {
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 wf = rowstep::weight_frag(w_lds, t, ks);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) acc[rt] = mfma16(xa[rt][ks], wf, acc[rt]);
      }
      const int h = 16 * t + m;
      if (h >= a.heads) continue;
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int jb = j0 + 16 * rt + 4 * g;        // keys jb .. jb + 3
        const int64_t off = (int64_t(h) * n + i) * npad + jb;
        if constexpr (std::is_same<TOUT, float>::value) {
          float4 v;
          v.x = jb + 0 < n ? acc[rt][0] * kLog2eF : 0.f;
          v.y = jb + 1 < n ? acc[rt][1] * kLog2eF : 0.f;
          v.z = jb + 2 < n ? acc[rt][2] * kLog2eF : 0.f;
          v.w = jb + 3 < n ? acc[rt][3] * kLog2eF : 0.f;
          *reinterpret_cast<float4 *>(static_cast<float *>(a.packed) + off) = v;
        } else {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = bf16(jb + e < n ? acc[rt][e] : 0.f);
          *reinterpret_cast<bf16x4 *>(static_cast<bf16 *>(a.packed) + off) = v;
        }
      }
    }
    cur = next;
  }
}

}  // namespace

int pair_bias_max_heads() { return MAX_HEADS; }

int pair_bias(const PairBiasArgs &a, int pair_dtype, hipStream_t s) {
  if (a.heads <= 0 || a.heads > MAX_HEADS || a.npad % 64 != 0 || a.npad < a.n)
    return fail(XFH_EINVAL, "pair_attention_bias: 1..384 heads, npad a multiple of 64 >= n");
  const int64_t units = int64_t(a.n) * (a.npad / 32);
  if (units == 0) return XFH_OK;
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const dim3 grid(unsigned(balanced_grid(units, 8, cus)));
  KernelTimer timer("pair_bias", s, 0.0, true);
  if (pair_dtype == XFH_BF16) {
    if (a.packed_bf16) timer.launch(pair_bias_kernel<bf16, bf16>, dim3(grid), dim3(512), 0, a);
    else timer.launch(pair_bias_kernel<bf16, float>, dim3(grid), dim3(512), 0, a);
  } else {
    if (a.packed_bf16) timer.launch(pair_bias_kernel<float, bf16>, dim3(grid), dim3(512), 0, a);
    else timer.launch(pair_bias_kernel<float, float>, dim3(grid), dim3(512), 0, a);
  }
  return check_launch("pair_bias");
}

}  // namespace xfh
