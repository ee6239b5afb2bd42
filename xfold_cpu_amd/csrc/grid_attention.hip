// Triangle (grid) attention core for bf16, head dim 32: the Pairformer's hot kernel.
//
// For batch row b (a row of the pair grid, or a column for the ending node), head h,
// query t and key s:  o[b,t,h,:] = softmax_s(q.k + bias[h,t,s], keys with mask[b,s]==0
// removed) @ v, which equals xfold/fastnn/attention.py:45-66 with its -1e9 fill whenever
// a row keeps at least one key (a masked key then gets probability exactly 0 in fp32);
// a row whose keys are all masked averages v uniformly over all keys, as -1e9 does.
//
// Operand layouts (written by the projection / repack kernels):
//   q   [B][H][N][32] bf16, pre-multiplied by d^-0.5 * log2(e)
//   k   [B][H][N][32] bf16
//   vt  [B][H][32][Npad] bf16 (keys contiguous, zero beyond N)
//   bias [H][N][Npad] fp32, pre-multiplied by log2(e)
//   maskbits [B][Npad/64] uint64: bit s%64 of word s/64 set iff key s < N is kept
//
// One workgroup = one head, 64 queries (4 wavefronts x 16) and R = 4 batch rows. Per key
// block of 64 the bias tile [16 q x 64 keys] is loaded once into registers and passed as
// the accumulator input of the Q.K^T MFMA for every row, so the bias add costs no VALU
// work and bias traffic is shared by R rows. The MFMA computes S^T = K Q^T (a lane holds
// four keys of one query), which is directly the B operand of O^T = V^T P^T; a constant
// ones row appended to V^T makes the same MFMA produce the softmax denominator. Key
// blocks with no kept key are skipped for that row. Workgroups are numbered so that one
// XCD walks the row groups of one head, keeping that head's bias in its L2.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int GD = 32;               // head dim
constexpr int GKB = 64;              // keys per block
constexpr int GR = 4;                // batch rows per workgroup
constexpr int KPITCH = GD + 8;       // LDS pitch of a K row (bf16)
constexpr int VPITCH = GKB + 8;      // LDS pitch of a V^T row (bf16)

__device__ __forceinline__ int64_t xcd_logical(int64_t physical, int64_t per_xcd) {
  return (physical % 8) * per_xcd + physical / 8;
}

__global__ __launch_bounds__(256, 2) void grid_attention_kernel(GridAttentionArgs a) {
  __shared__ bf16 ks[GR][GKB * KPITCH];
  __shared__ bf16 vts[GR][GD * VPITCH];

  const int qblocks = (a.N + 63) / 64;
  const int rgroups = (a.B + GR - 1) / GR;
  const int64_t total = int64_t(qblocks) * rgroups * a.H;
  const int64_t logical = xcd_logical(blockIdx.x, (total + 7) / 8);
  if (logical >= total) return;
  const int qblk = int(logical % qblocks);
  const int rg = int((logical / qblocks) % rgroups);
  const int h = int(logical / (int64_t(qblocks) * rgroups));

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int q = qblk * 64 + wave * 16 + col;
  const int qc = q < a.N ? q : a.N - 1;
  const int64_t HN = int64_t(a.H) * a.N;

  // Per-row state. Rows beyond B are inert (their loads are zero and stores skipped).
  bf16x8 qf[GR];
  f32x4 o[GR][3];
  float m[GR];
  bool all_masked[GR];
#pragma unroll
  for (int r = 0; r < GR; ++r) {
    const int b = rg * GR + r;
    bf16x8 z = {};
    qf[r] = z;
    if (b < a.B && q < a.N)
      qf[r] = *reinterpret_cast<const bf16x8 *>(a.q + ((int64_t(b) * a.H + h) * a.N + q) * GD + grp * 8);
#pragma unroll
    for (int t = 0; t < 3; ++t) o[r][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[r] = -INFINITY;
    uint64_t any = 0;
    if (b < a.B)
      for (int w = 0; w < a.Nblk; ++w) any |= a.maskbits[int64_t(b) * a.Nblk + w];
    all_masked[r] = (b < a.B) && any == 0;
  }
  // A operand of the denominator MFMA: V^T row 32 = ones, rows 33..47 = zeros.
  bf16x8 ones_frag;
#pragma unroll
  for (int s = 0; s < 8; ++s) ones_frag[s] = col == 0 ? bf16(1.0f) : bf16(0.0f);

  // Register prefetch of one key block: per row 4 KB of K and 4 KB of V^T, i.e. one
  // 16-byte chunk of each per thread.
  uint4 pk[GR], pv[GR];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int r = 0; r < GR; ++r) {
      const int b = rg * GR + r;
      const int key = kb * GKB + (tid >> 2), kc = (tid & 3) * 8;
      pk[r] = make_uint4(0, 0, 0, 0);
      pv[r] = make_uint4(0, 0, 0, 0);
      if (b < a.B) {
        if (key < a.N)
          pk[r] = *reinterpret_cast<const uint4 *>(a.k + ((int64_t(b) * a.H + h) * a.N + key) * GD + kc);
        const int d = tid >> 3, vc = (tid & 7) * 8;
        pv[r] = *reinterpret_cast<const uint4 *>(a.vt + ((int64_t(b) * a.H + h) * GD + d) * a.Npad +
                                                 int64_t(kb) * GKB + vc);
      }
    }
  };
  fetch(0);
  const float *bias_row = a.bias + (int64_t(h) * a.N + qc) * a.Npad;

  for (int kb = 0; kb < a.Nblk; ++kb) {
    __syncthreads();
#pragma unroll
    for (int r = 0; r < GR; ++r) {
      *reinterpret_cast<uint4 *>(&ks[r][(tid >> 2) * KPITCH + (tid & 3) * 8]) = pk[r];
      *reinterpret_cast<uint4 *>(&vts[r][(tid >> 3) * VPITCH + (tid & 7) * 8]) = pv[r];
    }
    __syncthreads();
    if (kb + 1 < a.Nblk) fetch(kb + 1);

    f32x4 bias[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
      bias[kt] = *reinterpret_cast<const f32x4 *>(bias_row + kb * GKB + kt * 16 + grp * 4);
    const int valid_keys = a.N - kb * GKB;   // keys of this block that exist
    const uint64_t exist = valid_keys >= 64 ? ~0ull : ((1ull << valid_keys) - 1);

#pragma unroll
    for (int r = 0; r < GR; ++r) {
      const int b = rg * GR + r;
      if (b >= a.B) break;
      uint64_t word = all_masked[r] ? exist : a.maskbits[int64_t(b) * a.Nblk + kb];
      if (word == 0) continue;
      float sv[16];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        f32x4 acc = bias[kt];
        if (all_masked[r]) {
          acc = f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
          const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(&ks[r][(kt * 16 + col) * KPITCH + grp * 8]);
          acc = mfma16(kf, qf[r], acc);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) sv[kt * 4 + e] = acc[e];
      }
      if (word != ~0ull) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const uint32_t nib = uint32_t(word >> (kt * 16 + grp * 4)) & 0xFu;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (!((nib >> e) & 1u)) sv[kt * 4 + e] = -INFINITY;
        }
      }
      float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
#pragma unroll
      for (int i = 4; i < 16; i += 4) mx = fmaxf(mx, fmaxf(fmaxf(sv[i], sv[i + 1]), fmaxf(sv[i + 2], sv[i + 3])));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m[r], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[r] - m_new);
      m[r] = m_new;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int t = 0; t < 3; ++t) o[r][t] *= alpha;
      }
      bf16x8 pf[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pf[c][e] = bf16(__builtin_amdgcn_exp2f(sv[(2 * c) * 4 + e] - m_new));
          pf[c][4 + e] = bf16(__builtin_amdgcn_exp2f(sv[(2 * c + 1) * 4 + e] - m_new));
        }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const bf16 *row = &vts[r][(t * 16 + col) * VPITCH + c * 32 + grp * 4];
          bf16x8 vf;
          const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(row);
          const bf16x4 hi = *reinterpret_cast<const bf16x4 *>(row + 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            vf[e] = lo[e];
            vf[4 + e] = hi[e];
          }
          o[r][t] = mfma16(vf, pf[c], o[r][t]);
        }
        o[r][2] = mfma16(ones_frag, pf[c], o[r][2]);
      }
    }
  }

#pragma unroll
  for (int r = 0; r < GR; ++r) {
    const int b = rg * GR + r;
    const float l = __shfl(o[r][2][0], col, 64);     // denominator sits in lane `col`, grp 0
    if (b >= a.B || q >= a.N) continue;
    const float inv = 1.0f / l;
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

// ---------------------------------------------------------------- operand repacking
// From the projection GEMM outputs (pair-row major) to the kernel's operand layouts.
// Pair row of (batch row b, position t): b*n + t (starting node) or t*n + b (ending node).

__global__ void grid_repack_qk(const bf16 *__restrict__ qkv, int64_t n, int heads, int transpose,
                               float qscale, bf16 *__restrict__ qh, bf16 *__restrict__ kh) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = n * heads * n * 4;
  if (idx >= total) return;
  const int ch = int(idx & 3);
  const int64_t t = (idx >> 2) % n;
  const int64_t bh = (idx >> 2) / n;
  const int h = int(bh % heads);
  const int64_t b = bh / heads;
  const int64_t c = int64_t(heads) * GD;
  const int64_t row = transpose ? t * n + b : b * n + t;
  const bf16 *src = qkv + row * 3 * c + h * GD + ch * 8;
  bf16x8 qv = *reinterpret_cast<const bf16x8 *>(src);
  bf16x8 kv = *reinterpret_cast<const bf16x8 *>(src + c);
#pragma unroll
  for (int e = 0; e < 8; ++e) qv[e] = bf16(static_cast<float>(qv[e]) * qscale);
  const int64_t dst = ((b * heads + h) * n + t) * GD + ch * 8;
  *reinterpret_cast<bf16x8 *>(qh + dst) = qv;
  *reinterpret_cast<bf16x8 *>(kh + dst) = kv;
}

__global__ void grid_repack_vt(const bf16 *__restrict__ qkv, int64_t n, int64_t npad, int heads,
                               int transpose, bf16 *__restrict__ vt) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = n * heads * GD * npad;
  if (idx >= total) return;
  const int64_t t = idx % npad;
  const int64_t rest = idx / npad;
  const int d = int(rest % GD);
  const int64_t bh = rest / GD;
  const int h = int(bh % heads);
  const int64_t b = bh / heads;
  const int64_t c = int64_t(heads) * GD;
  bf16 v = bf16(0.0f);
  if (t < n) {
    const int64_t row = transpose ? t * n + b : b * n + t;
    v = qkv[row * 3 * c + 2 * c + h * GD + d];
  }
  vt[idx] = v;
}

__global__ void grid_repack_bias(const bf16 *__restrict__ lin, int64_t n, int64_t npad, int heads,
                                 float *__restrict__ bias) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = int64_t(heads) * n * npad;
  if (idx >= total) return;
  const int64_t k = idx % npad;
  const int64_t qh = idx / npad;
  const int64_t q = qh % n;
  const int h = int(qh / n);
  bias[idx] = k < n ? static_cast<float>(lin[(q * n + k) * heads + h]) * kLog2e : 0.0f;
}

__global__ void grid_mask_bits(const void *__restrict__ mask, int mask_dtype, int64_t n, int64_t nblk,
                               uint64_t *__restrict__ bits) {
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= n * nblk) return;
  const int64_t b = idx / nblk, w = idx % nblk;
  uint64_t word = 0;
  for (int i = 0; i < 64; ++i) {
    const int64_t k = w * 64 + i;
    if (k < n && (!mask || load_any(mask, mask_dtype, b * n + k) != 0.f)) word |= (1ull << i);
  }
  bits[idx] = word;
}

}  // namespace

int64_t grid_attention_pad(int64_t n) { return align_up(n, GKB); }

int grid_attention_prepare(const void *qkv, const void *bias_lin, const void *mask, int mask_dtype,
                           int64_t n, int heads, int transpose, float scale, void *qh, void *kh,
                           void *vt, float *bias, uint64_t *maskbits, hipStream_t s) {
  const int64_t npad = grid_attention_pad(n), nblk = npad / GKB;
  const int64_t c = int64_t(heads) * GD;
  (void)c;
  int64_t total = n * heads * n * 4;
  grid_repack_qk<<<dim3(ceil_div(total, 256)), 256, 0, s>>>((const bf16 *)qkv, n, heads, transpose,
                                                             scale * kLog2e, (bf16 *)qh, (bf16 *)kh);
  XFH_TRY(check_launch("grid_repack_qk"));
  total = n * heads * GD * npad;
  grid_repack_vt<<<dim3(ceil_div(total, 256)), 256, 0, s>>>((const bf16 *)qkv, n, npad, heads, transpose,
                                                             (bf16 *)vt);
  XFH_TRY(check_launch("grid_repack_vt"));
  total = int64_t(heads) * n * npad;
  grid_repack_bias<<<dim3(ceil_div(total, 256)), 256, 0, s>>>((const bf16 *)bias_lin, n, npad, heads, bias);
  XFH_TRY(check_launch("grid_repack_bias"));
  grid_mask_bits<<<dim3(ceil_div(n * nblk, 256)), 256, 0, s>>>(mask, mask_dtype, n, nblk, maskbits);
  return check_launch("grid_mask_bits");
}

int grid_attention(const GridAttentionArgs &a, hipStream_t s) {
  if (a.B == 0 || a.N == 0) return XFH_OK;
  const int64_t qblocks = ceil_div(a.N, 64), rgroups = ceil_div(a.B, GR);
  const int64_t total = qblocks * rgroups * a.H;
  const int64_t grid = ceil_div(total, 8) * 8;
  if (grid > (int64_t(1) << 31) - 1) return fail(XFH_EUNSUPPORTED, "grid_attention: problem too large");
  KernelTimer timer("grid_attention", s);
  grid_attention_kernel<<<dim3(grid), 256, 0, s>>>(a);
  return check_launch("grid_attention");
}

}  // namespace xfh
