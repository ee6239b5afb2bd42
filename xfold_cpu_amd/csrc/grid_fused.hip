// Fused projection and output kernels around the triangle-attention core (bf16 compute,
// c = 128, 4 heads x 32), following GridSelfAttention.forward (xfold/nn/attention.py:80-105):
//
//   grid_project: LN(z) -> one GEMM over a packed [q | k | v | bias] weight -> q scaled by
//       d^-0.5 * log2(e), k, v^T (zero beyond n, keys permuted in runs of 32) and the fp32
//       pair bias (times log2(e)),
//       each written straight into the attention kernel's layout (grid_attention.hip).
//       The bias comes from the un-transposed pair in both directions.
//   grid_output: gate = sigmoid(LN(z) Wgating^T) (recomputed: z is read here anyway for
//       the residual) -> (gate * o) Wout^T -> z += update (or update stored).
//   grid_mask_words: per batch row, one 64-bit word of kept keys per 64 keys.
#include "common.h"
#include "kernels.h"
#include "panel.h"

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
      bf16 *dst = kind == 0 ? a.q : a.k;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + i * 256;              // 128 rows x 8 chunks of 8
        const int r = idx >> 3, c = (idx & 7) * 8;
        const int t = t0 + r;
        if (t >= n) continue;
        const int h = (j & 1) * 2 + c / HD;
        *reinterpret_cast<bf16x8 *>(dst + ((int64_t(b) * H + h) * n + t) * HD + (c % HD)) =
            *reinterpret_cast<const bf16x8 *>(&stage[r * CPITCH + c]);
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

template <typename TIN, typename TOUT>
__global__ __launch_bounds__(256, 2) void grid_output_kernel(GridOutputArgs a) {
  __shared__ bf16 lds_a[A_ELEMS];
  __shared__ bf16 lds_b[2 * B_ELEMS];
  auto bbuf = [&](int i) -> bf16 * { return lds_b + (i & 1) * B_ELEMS; };

  const int64_t plane = int64_t(a.n) * a.n;
  const int64_t pos0 = int64_t(blockIdx.x) * ROWS;
  const int valid = int(plane - pos0 < ROWS ? plane - pos0 : ROWS);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
  const TIN *z = static_cast<const TIN *>(a.pair);

  // 1) gate logits from LN(z), in registers.
  ln_panel<TIN>([&](int r) -> const TIN * { return r < valid ? z + (pos0 + r) * K : nullptr; },
                a.ln_w, a.ln_b, a.eps, lds_a);
  __syncthreads();
  AFrags af;
  load_a_frags(lds_a, wm, af);
  BStage st;
  fetch_b(a.w_gating, 0, K, st);
  stash_b(st, bbuf(0));
  fetch_b(a.w_gating, CHUNK, K, st);
  stash_b(st, bbuf(1));
  __syncthreads();
  f32x4 gate[2][4][2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    zero(gate[j]);
    mma_chunk(af, bbuf(j), wn, gate[j]);
  }
  __syncthreads();
  // 2) A tile <- o (attention output rows), then scaled in place by sigmoid(gate).
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid + i * 256;
    const int r = idx >> 4, c = (idx & 15) * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < valid) v = *reinterpret_cast<const uint4 *>(a.attn + (pos0 + r) * K + c);
    *reinterpret_cast<uint4 *>(&lds_a[r * PITCH + c]) = v;
  }
  fetch_b(a.w_out, 0, K, st);
  stash_b(st, bbuf(0));
  fetch_b(a.w_out, CHUNK, K, st);
  stash_b(st, bbuf(1));
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bf16 *p = &lds_a[(wm * 64 + mt * 16 + grp * 4 + e) * PITCH + j * CHUNK + wn * 32 + nt * 16 + col];
          *p = bf16(static_cast<float>(*p) * sigmoidf_(gate[j][mt][nt][e]));
        }
  __syncthreads();
  load_a_frags(lds_a, wm, af);
  __syncthreads();
  // 3) output projection -> staging (bf16 update) -> residual.
  bf16 *stage = lds_a;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    f32x4 acc[4][2];
    zero(acc);
    mma_chunk(af, bbuf(j), wn, acc);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          stage[(wm * 64 + mt * 16 + grp * 4 + e) * PITCH + j * CHUNK + wn * 32 + nt * 16 + col] =
              bf16(acc[mt][nt][e]);
  }
  __syncthreads();
  TOUT *out = static_cast<TOUT *>(a.out);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid + i * 256;
    const int r = idx >> 4, c = (idx & 15) * 8;
    if (r >= valid) continue;
    TOUT *dst = out + (pos0 + r) * K + c;
    float u[8], o[8];
    load8<bf16>(&stage[r * PITCH + c], u);
    if (a.accumulate) {
      load8<TOUT>(dst, o);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += u[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = u[e];
    }
    if constexpr (sizeof(TOUT) == 2) {
      bf16x8 w;
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = bf16(o[e]);
      *reinterpret_cast<bf16x8 *>(dst) = w;
    } else {
      reinterpret_cast<float4 *>(dst)[0] = make_float4(o[0], o[1], o[2], o[3]);
      reinterpret_cast<float4 *>(dst)[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
  }
}

// One wavefront per 64-key word: lane i tests key w*64 + i, the ballot is the word.
__global__ void grid_mask_words(const void *__restrict__ mask, int mask_dtype, int64_t n, int64_t nblk,
                                uint64_t *__restrict__ bits) {
  const int64_t word = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (word >= n * nblk) return;
  const int64_t b = word / nblk, w = word % nblk;
  const int64_t k = w * 64 + (threadIdx.x & 63);
  const bool keep = k < n && (!mask || load_any(mask, mask_dtype, b * n + k) != 0.f);
  const uint64_t ballot = __ballot(keep);
  if ((threadIdx.x & 63) == 0) bits[word] = ballot;
}

// Packed [3c + 64][c]: q, k, v weights, then the bias projection rows (zero-padded to 64).
__global__ void grid_pack_kernel(const bf16 *__restrict__ wq, const bf16 *__restrict__ wk,
                                 const bf16 *__restrict__ wv, const bf16 *__restrict__ wb, int c,
                                 int heads, bf16 *__restrict__ packed) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = int64_t(PACKED_ROWS) * c;
  if (idx >= total) return;
  const int r = int(idx / c), k = int(idx % c);
  bf16 v = bf16(0.0f);
  if (r < c) v = wq[int64_t(r) * c + k];
  else if (r < 2 * c) v = wk[int64_t(r - c) * c + k];
  else if (r < 3 * c) v = wv[int64_t(r - 2 * c) * c + k];
  else if (r - 3 * c < heads) v = wb[int64_t(r - 3 * c) * c + k];
  packed[idx] = v;
}

}  // namespace

int64_t grid_packed_rows() { return PACKED_ROWS; }

int grid_pack(const void *wq, const void *wk, const void *wv, const void *wb, int c, int heads,
              void *packed, hipStream_t s) {
  const int64_t total = int64_t(PACKED_ROWS) * c;
  grid_pack_kernel<<<dim3(ceil_div(total, 256)), 256, 0, s>>>((const bf16 *)wq, (const bf16 *)wk,
                                                               (const bf16 *)wv, (const bf16 *)wb, c, heads,
                                                               (bf16 *)packed);
  return check_launch("grid_pack");
}

int grid_mask(const void *mask, int mask_dtype, int64_t n, int64_t nblk, uint64_t *bits, hipStream_t s) {
  const int64_t words = n * nblk;
  grid_mask_words<<<dim3(ceil_div(words, 4)), 256, 0, s>>>(mask, mask_dtype, n, nblk, bits);
  return check_launch("grid_mask_words");
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
  const int64_t panels = ceil_div(int64_t(a.n) * a.n, ROWS);
  KernelTimer timer("grid_output", s);
  if (pair_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    grid_output_kernel<bf16, bf16><<<dim3(panels), 256, 0, s>>>(a);
  else if (pair_dtype == XFH_BF16 && out_dtype == XFH_F32)
    grid_output_kernel<bf16, float><<<dim3(panels), 256, 0, s>>>(a);
  else if (pair_dtype == XFH_F32 && out_dtype == XFH_F32)
    grid_output_kernel<float, float><<<dim3(panels), 256, 0, s>>>(a);
  else
    grid_output_kernel<float, bf16><<<dim3(panels), 256, 0, s>>>(a);
  return check_launch("grid_output");
}

}  // namespace xfh
