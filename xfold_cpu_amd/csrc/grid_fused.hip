// Fused projection and output kernels around the triangle-attention core (bf16 compute,
// c = 128, 4 heads x 32), following GridSelfAttention.forward (xfold/nn/attention.py:80-105):
//
//   grid_project: LN(z) -> one GEMM over a packed [q | k | v | bias] weight -> q scaled by
//       d^-0.5 * log2(e), k (rows up to npad, zero beyond n), v^T (zero beyond n, keys
//       permuted in runs of 32) and the fp32 pair bias (times log2(e)),
//       each written straight into the attention kernel's layout (grid_attention.hip).
//       The bias comes from the un-transposed pair in both directions.
//   grid_output: gate = sigmoid(LN(z) Wgating^T) (recomputed: z is read here anyway for
//       the residual) -> (gate * o) Wout^T -> z += update (or update stored).
//   grid_prepare: the packed weight and the attention kernel's kept-key words, one launch.
#include <algorithm>

#include "common.h"
#include "kernels.h"
#include "panel.h"
#include "rowstep.h"

namespace xfh {

namespace {

using namespace panel;

constexpr int HD = 32;                 // head dim
constexpr int QKV_ROWS = 3 * K;        // packed weight: q, k, v rows, then a 64-row bias chunk
constexpr int PACKED_ROWS = QKV_ROWS + CHUNK;
constexpr int CPITCH = CHUNK + 8;      // staging pitch [row][col] (bf16)
constexpr int TPITCH = ROWS + 8;       // staging pitch [col][row] (bf16)
static_assert(CHUNK * TPITCH <= ROWS * CPITCH, "v^T staging must fit the q/k staging area");

template <typename TIN>
__global__ __launch_bounds__(256, 2) void grid_project_kernel(GridProjectArgs a) {
  __shared__ bf16 lds_a[A_ELEMS];                   // A tile, later two B buffers
  __shared__ bf16 stage[ROWS * CPITCH];             // [128][72] (q, k) or [64][136] (v^T)
  auto bbuf = [&](int i) -> bf16 * { return lds_a + (i & 1) * B_ELEMS; };

  const int n = a.n, H = a.heads;
  const int ppb = (n + ROWS - 1) / ROWS;            // panels per batch row
  const int b = blockIdx.x / ppb, t0 = (blockIdx.x % ppb) * ROWS;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
  const TIN *z = static_cast<const TIN *>(a.pair);
  // Pair row of attention position (b, t): b*n + t (starting node) or t*n + b (ending node).
  auto row_of = [&](int t) -> int64_t { return a.transpose ? int64_t(t) * n + b : int64_t(b) * n + t; };

  ln_panel<TIN>([&](int r) -> const TIN * { return (t0 + r < n) ? z + row_of(t0 + r) * K : nullptr; },
                a.ln_w, a.ln_b, a.eps, lds_a);
  __syncthreads();
  AFrags af;
  load_a_frags(lds_a, wm, af);
  BStage st;
  fetch_b(a.w_packed, 0, PACKED_ROWS, st);
  __syncthreads();
  stash_b(st, bbuf(0));
  __syncthreads();

  const int chunks = PACKED_ROWS / CHUNK;           // 2 q, 2 k, 2 v, 1 bias
  for (int j = 0; j < chunks; ++j) {
    if (j + 1 < chunks) fetch_b(a.w_packed, (j + 1) * CHUNK, PACKED_ROWS, st);
    f32x4 acc[4][2];
    zero(acc);
    mma_chunk(af, bbuf(j), wn, acc);
    const int kind = j / 2;                         // 0 q, 1 k, 2 v, 3 bias
    if (kind == 3) {
      // Bias: column h < H of this chunk; bias[h][i][j] for pair (i, j) = (b, t) or (t, b).
      // The pad columns j in [n, npad) are written as zeros (the attention kernel adds its
      // mask to them, so they must be finite): by the panels with t >= n when j = t, by the
      // panels of the last batch row when j = b.
      if (wn == 0 && col < H) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int t = t0 + wm * 64 + mt * 16 + grp * 4 + e;
            if (t >= n) {
              if (!a.transpose && t < a.npad) a.bias[(int64_t(col) * n + b) * a.npad + t] = 0.0f;
              continue;
            }
            const int64_t qi = a.transpose ? t : b, kj = a.transpose ? b : t;
            float *row = a.bias + (int64_t(col) * n + qi) * a.npad;
            row[kj] = acc[mt][0][e] * kLog2e;
            if (a.transpose && b == n - 1)
              for (int j = n; j < a.npad; ++j) row[j] = 0.0f;
          }
      }
    } else if (kind < 2) {
      // q or k: stage [row t][64 cols] then 16-byte rows of [b][h][t][32].
      const float scale = kind == 0 ? a.qscale : 1.0f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            stage[(wm * 64 + mt * 16 + grp * 4 + e) * CPITCH + wn * 32 + nt * 16 + col] =
                bf16(acc[mt][nt][e] * scale);
      __syncthreads();
      // q rows: [b][h][n][32]; k rows: [b][h][npad][32], zero for n <= t < npad (the
      // attention kernel loads whole 64-key blocks of k without bounds).
      bf16 *dst = kind == 0 ? a.q : a.k;
      const int rows = kind == 0 ? n : a.npad;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + i * 256;              // 128 rows x 8 chunks of 8
        const int r = idx >> 3, c = (idx & 7) * 8;
        const int t = t0 + r;
        if (t >= rows) continue;
        const int h = (j & 1) * 2 + c / HD;
        bf16x8 v = *reinterpret_cast<const bf16x8 *>(&stage[r * CPITCH + c]);
        if (t >= n) v = bf16x8{};
        *reinterpret_cast<bf16x8 *>(dst + ((int64_t(b) * H + h) * rows + t) * HD + (c % HD)) = v;
      }
    } else {
      // v: stage transposed [64 cols][128 rows] then [b][h][d][npad] rows, zero beyond n.
      // Inside every run of 32 keys, position 8g + j holds key 4g + j (j < 4) or
      // 16 + 4g + (j - 4) (j >= 4): the key order of the attention kernel's P^T fragment,
      // so that one 16-byte LDS read there yields a whole V^T fragment.
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = bf16(acc[mt][nt][e]);
          *reinterpret_cast<bf16x4 *>(&stage[(wn * 32 + nt * 16 + col) * TPITCH + wm * 64 + mt * 16 + grp * 4]) = v;
        }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + i * 256;              // 64 cols x 16 chunks of 8 rows
        const int c = idx >> 4, rc = (idx & 15) * 8;    // positions rc .. rc+7 of the panel
        const int t = t0 + rc;
        if (t >= a.npad) continue;
        const int h = (j & 1) * 2 + c / HD, d = c % HD;
        const int key0 = (rc & ~31) + ((rc & 31) >> 1);   // panel-relative: 4g, and 16 + 4g
        const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(&stage[c * TPITCH + key0]);
        const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(&stage[c * TPITCH + key0 + 16]);
        bf16x8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = t0 + key0 + e < n ? lo[e] : bf16(0.0f);
          v[4 + e] = t0 + key0 + 16 + e < n ? hi[e] : bf16(0.0f);
        }
        *reinterpret_cast<bf16x8 *>(a.vt + ((int64_t(b) * H + h) * HD + d) * a.npad + t) = v;
      }
    }
    if (j + 1 < chunks) stash_b(st, bbuf(j + 1));
    __syncthreads();
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
  rowstep::load_weight(a.w_gating, w_gate, false);
  rowstep::load_weight(a.w_out, w_out, true);
  rowstep::load_ln(a.ln_w, a.ln_b, lnw, lnb);
  __syncthreads();

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
  if (st < steps) fetch(st, cur);
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

// Blocks [0, pack_blocks): packed weight [3c + 64][c] (q, k, v, then the bias rows
// zero-padded to 64), one element per thread. The rest: one wavefront per 64-key word,
// lane i tests key w*64 + i and the ballot is the word.
__global__ void grid_prepare_kernel(const bf16 *__restrict__ wq, const bf16 *__restrict__ wk,
                                    const bf16 *__restrict__ wv, const bf16 *__restrict__ wb, int c,
                                    int heads, bf16 *__restrict__ packed, int64_t pack_blocks,
                                    const void *__restrict__ mask, int mask_dtype, int64_t n, int64_t nblk,
                                    uint64_t *__restrict__ bits) {
  if (blockIdx.x < pack_blocks) {
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= int64_t(PACKED_ROWS) * c) return;
    const int r = int(idx / c), k = int(idx % c);
    bf16 v = bf16(0.0f);
    if (r < c) v = wq[int64_t(r) * c + k];
    else if (r < 2 * c) v = wk[int64_t(r - c) * c + k];
    else if (r < 3 * c) v = wv[int64_t(r - 2 * c) * c + k];
    else if (r - 3 * c < heads) v = wb[int64_t(r - 3 * c) * c + k];
    packed[idx] = v;
    return;
  }
  const int64_t word = (int64_t(blockIdx.x) - pack_blocks) * 4 + (threadIdx.x >> 6);
  if (word >= n * nblk) return;
  const int64_t b = word / nblk, w = word % nblk;
  const int64_t k = w * 64 + (threadIdx.x & 63);
  const bool keep = k < n && (!mask || load_any(mask, mask_dtype, b * n + k) != 0.f);
  const uint64_t ballot = __ballot(keep);
  if ((threadIdx.x & 63) == 0) bits[word] = ballot;
}

}  // namespace

int64_t grid_packed_rows() { return PACKED_ROWS; }

int grid_prepare(const void *wq, const void *wk, const void *wv, const void *wb, int c, int heads,
                 void *packed, const void *mask, int mask_dtype, int64_t n, int64_t nblk,
                 uint64_t *bits, hipStream_t s) {
  const int64_t pack_blocks = ceil_div(int64_t(PACKED_ROWS) * c, 256);
  const int64_t word_blocks = ceil_div(n * nblk, 4);
  grid_prepare_kernel<<<dim3(pack_blocks + word_blocks), 256, 0, s>>>(
      (const bf16 *)wq, (const bf16 *)wk, (const bf16 *)wv, (const bf16 *)wb, c, heads, (bf16 *)packed,
      pack_blocks, mask, mask_dtype, n, nblk, bits);
  return check_launch("grid_prepare");
}

int grid_project(const GridProjectArgs &a, int pair_dtype, hipStream_t s) {
  const int64_t panels = int64_t(a.n) * ceil_div(a.n, ROWS);
  KernelTimer timer("grid_project", s);
  if (pair_dtype == XFH_BF16)
    grid_project_kernel<bf16><<<dim3(panels), 256, 0, s>>>(a);
  else
    grid_project_kernel<float><<<dim3(panels), 256, 0, s>>>(a);
  return check_launch("grid_project");
}

int grid_output(const GridOutputArgs &a, int pair_dtype, int out_dtype, hipStream_t s) {
  const int64_t steps = ceil_div(int64_t(a.n) * a.n, 16);
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const dim3 grid(unsigned(std::min<int64_t>(cus, ceil_div(steps, 8))));
  KernelTimer timer("grid_output", s);
  if (pair_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    grid_output_kernel<bf16, bf16><<<grid, 512, 0, s>>>(a);
  else if (pair_dtype == XFH_BF16 && out_dtype == XFH_F32)
    grid_output_kernel<bf16, float><<<grid, 512, 0, s>>>(a);
  else if (pair_dtype == XFH_F32 && out_dtype == XFH_F32)
    grid_output_kernel<float, float><<<grid, 512, 0, s>>>(a);
  else
    grid_output_kernel<float, bf16><<<grid, 512, 0, s>>>(a);
  return check_launch("grid_output");
}

}  // namespace xfh
