// dot_product_attention (xfold/fastnn/attention.py:45-66) on the triangle-attention kernel
// (grid_attention.hip): one preparation launch turns the caller's strided q, k, v, bias and
// mask into that kernel's layouts, then the kernel runs at head dim 16, 32 or 64.
//
// Preparation (one launch; each part takes its own range of workgroups):
//   0  q  [B][H][Nq][D]   = q * scale * log2(e), zero for d >= Dqk
//   1  k  [B][H][Npad][D] = k, zero for keys >= N or d >= Dqk
//   2  vt [B][H][D][Npad] = v^T, zero for keys >= N or d >= Dv; inside each run of 32 keys
//      position 8g + j holds key 4g + j (j < 4) or 16 + 4g + j - 4 (j >= 4)
//   3  bias [H][Nq][Npad] fp32 = bias * log2(e) (batch-shared), zero for keys >= N (part 5:
//      the same from a bf16 view whose heads are innermost)
//   4  mask words [Bm][Npad/64]: bit s of row b set iff key s < N is kept (Bm = B when the
//      mask depends on the batch entry, else 1)
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr float kLog2eF = 1.4426950408889634f;

struct MhaPrep {
  AttentionArgs a;
  int D;                      // padded head dim
  int64_t npad, nblk, mask_rows;
  bf16 *q, *k, *vt;
  float *bias;
  uint64_t *words;
  bool vec_qk;               // q and k rows hold whole 16-byte chunks (D, strides % 8, aligned)
  // One launch runs every part: blocks [start[j], start[j + 1]) run part id[j].
  int nparts;
  int id[5];
  int64_t start[6];
};

template <typename T> __device__ __forceinline__ float ld(const void *p, int64_t i) {
  return static_cast<float>(static_cast<const T *>(p)[i]);
}

__global__ void mha_prepare_kernel(MhaPrep p) {
  const AttentionArgs &a = p.a;
  int j = 0;
  while (j + 1 < p.nparts && int64_t(blockIdx.x) >= p.start[j + 1]) ++j;
  const int part = p.id[j];
  const int64_t idx = (int64_t(blockIdx.x) - p.start[j]) * blockDim.x + threadIdx.x;
  const int D = p.D, dc = D / 8;            // 8-element chunks per row
  switch (part) {
    case 0: {                               // q: thread = (b, h, n, chunk)
      const int64_t total = a.B * a.H * a.Q * dc;
      if (idx >= total) return;
      const int c = int(idx % dc);
      const int64_t row = idx / dc, n = row % a.Q, bh = row / a.Q, h = bh % a.H, b = bh / a.H;
      const bf16 *src = static_cast<const bf16 *>(a.q) + b * a.qs[0] + h * a.qs[1] + n * a.qs[2];
      const float s = a.scale * kLog2eF;
      bf16x8 v;
      if (p.vec_qk) {                               // one 16-byte load per chunk
        bf16x8 x = {};
        if (c * 8 < a.D) x = *reinterpret_cast<const bf16x8 *>(src + c * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = bf16(static_cast<float>(x[e]) * s);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = c * 8 + e;
          v[e] = bf16(d < a.D ? static_cast<float>(src[d]) * s : 0.f);
        }
      }
      *reinterpret_cast<bf16x8 *>(p.q + row * D + c * 8) = v;
      return;
    }
    case 1: {                               // k: thread = (b, h, key, chunk)
      const int64_t total = a.B * a.H * p.npad * dc;
      if (idx >= total) return;
      const int c = int(idx % dc);
      const int64_t row = idx / dc, key = row % p.npad, bh = row / p.npad, h = bh % a.H, b = bh / a.H;
      const bf16 *src = static_cast<const bf16 *>(a.k) + b * a.ks[0] + h * a.ks[1] + key * a.ks[2];
      bf16x8 v = {};
      if (p.vec_qk) {
        if (key < a.K && c * 8 < a.D) v = *reinterpret_cast<const bf16x8 *>(src + c * 8);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = c * 8 + e;
          v[e] = (key < a.K && d < a.D) ? src[d] : bf16(0.f);
        }
      }
      *reinterpret_cast<bf16x8 *>(p.k + row * D + c * 8) = v;
      return;
    }
    case 2: {                               // v^T: thread = (b, h, 8-position group, d), d fastest
      const int64_t groups = p.npad / 8;
      const int64_t total = a.B * a.H * groups * D;
      if (idx >= total) return;
      const int d = int(idx % D);
      const int64_t rest = idx / D, grp = rest % groups, bh = rest / groups, h = bh % a.H, b = bh / a.H;
      const bf16 *src = static_cast<const bf16 *>(a.v) + b * a.vs[0] + h * a.vs[1] + d;
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t pos = grp * 8 + e, run = pos & ~int64_t(31);
        const int w = int(pos & 31), g = w >> 3, j = w & 7;
        const int64_t key = run + (j < 4 ? 4 * g + j : 16 + 4 * g + j - 4);
        v[e] = (key < a.K && d < a.Dv) ? src[key * a.vs[2]] : bf16(0.f);
      }
      *reinterpret_cast<bf16x8 *>(p.vt + (bh * D + d) * p.npad + grp * 8) = v;
      return;
    }
    case 3: {                               // bias, key-minor view: thread = (h, q, 4 keys)
      const int64_t quads = p.npad / 4;
      const int64_t total = a.H * a.Q * quads;
      if (idx >= total) return;
      const int64_t kq = idx % quads, row = idx / quads, n = row % a.Q, h = row / a.Q;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t key = kq * 4 + e;
        float x = 0.f;
        if (key < a.K && a.bias) {
          const int64_t off = h * a.bs[1] + n * a.bs[2] + key * a.bs[3];
          x = (a.bias_dtype == XFH_F32 ? ld<float>(a.bias, off) : ld<bf16>(a.bias, off)) * kLog2eF;
        }
        v[e] = x;
      }
      *reinterpret_cast<float4 *>(p.bias + row * p.npad + kq * 4) = make_float4(v[0], v[1], v[2], v[3]);
      return;
    }
    case 5: {                               // bias, bf16 head-minor view (heads contiguous, H % 8
                                            // == 0, 16-byte aligned): thread = (q, key)
      const int64_t total = a.Q * p.npad;
      if (idx >= total) return;
      const int64_t key = idx % p.npad, n = idx / p.npad;
      const bf16 *src = static_cast<const bf16 *>(a.bias) + n * a.bs[2] + key * a.bs[3];
      float *dst = p.bias + n * p.npad + key;
      for (int64_t h0 = 0; h0 < a.H; h0 += 8) {
        bf16x8 v = {};
        if (key < a.K) v = *reinterpret_cast<const bf16x8 *>(src + h0);
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[(h0 + e) * a.Q * p.npad] = static_cast<float>(v[e]) * kLog2eF;
      }
      return;
    }
    default: {                              // mask words: one wavefront per word
      const int64_t word = idx >> 6;
      if (word >= p.mask_rows * p.nblk) return;
      const int64_t b = word / p.nblk, w = word % p.nblk;
      const int64_t key = w * 64 + (threadIdx.x & 63);
      const bool keep = key < a.K && (!a.mask || load_any(a.mask, a.mask_dtype, b * a.ms[0] + key * a.ms[3]) != 0.f);
      const uint64_t ballot = __ballot(keep);
      if ((threadIdx.x & 63) == 0) p.words[word] = ballot;
      return;
    }
  }
}

int padded_dim(int64_t d) { return d <= 16 ? 16 : d <= 32 ? 32 : d <= 64 ? 64 : 0; }

struct MhaPlan {
  int D;
  int64_t npad, nblk, mask_rows;
  int64_t q_bytes, k_bytes, v_bytes, bias_bytes, word_bytes;
  int64_t total() const { return q_bytes + k_bytes + v_bytes + bias_bytes + word_bytes + 5 * 256; }
};

MhaPlan plan(int64_t B, int64_t H, int64_t Q, int64_t K, int64_t D, int64_t Dv, bool mask_per_row) {
  MhaPlan p;
  p.D = padded_dim(D > Dv ? D : Dv);
  p.npad = align_up(K, 64);
  p.nblk = p.npad / 64;
  p.mask_rows = mask_per_row ? B : 1;
  p.q_bytes = B * H * Q * p.D * 2;
  p.k_bytes = B * H * p.npad * p.D * 2;
  p.v_bytes = B * H * p.D * p.npad * 2;
  p.bias_bytes = H * Q * p.npad * 4;
  p.word_bytes = p.mask_rows * p.nblk * 8;
  return p;
}

}  // namespace

int64_t mha_workspace_size(const AttentionArgs &a) {
  if (padded_dim(a.D > a.Dv ? a.D : a.Dv) == 0) return 0;
  return plan(a.B, a.H, a.Q, a.K, a.D, a.Dv, true).total();
}

bool mha_supported(const AttentionArgs &a, int dtype) {
  return dtype == XFH_BF16 && a.out_dtype == XFH_BF16 && padded_dim(a.D > a.Dv ? a.D : a.Dv) != 0 &&
         a.K > 0 && align_up(a.K, 64) <= grid_attention_max_n() &&
         (!a.bias || a.bias_dtype == XFH_BIAS_PACKED || a.bias_dtype == XFH_BIAS_PACKED_BF16 || a.B == 1 ||
          a.bs[0] == 0) &&  // batch-shared bias
         // mask per (batch entry, key); a size-1 head or query dimension has no stride to speak of
         (!a.mask || ((a.ms[1] == 0 || a.H == 1) && (a.ms[2] == 0 || a.Q == 1))) &&
         a.os[1] % 4 == 0 && a.os[2] % 4 == 0 && a.os[0] % 4 == 0 &&
         reinterpret_cast<uintptr_t>(a.o) % 8 == 0;
}

int mha(const AttentionArgs &a, void *workspace, int64_t workspace_bytes, hipStream_t s) {
  const bool per_row = a.mask && a.B > 1 && a.ms[0] != 0;
  const MhaPlan pl = plan(a.B, a.H, a.Q, a.K, a.D, a.Dv, per_row);
  if (!workspace || pl.total() > workspace_bytes)
    return fail(XFH_EWORKSPACE, "dot_product_attention: workspace too small (need " +
                                    std::to_string(pl.total()) + " bytes)");
  Carver cv(workspace, workspace_bytes);
  MhaPrep p;
  p.a = a;
  p.D = pl.D;
  p.npad = pl.npad;
  p.nblk = pl.nblk;
  p.mask_rows = pl.mask_rows;
  p.q = static_cast<bf16 *>(cv.take(pl.q_bytes));
  p.k = static_cast<bf16 *>(cv.take(pl.k_bytes));
  p.vt = static_cast<bf16 *>(cv.take(pl.v_bytes));
  p.bias = static_cast<float *>(cv.take(pl.bias_bytes));
  p.words = static_cast<uint64_t *>(cv.take(pl.word_bytes));
  p.vec_qk = a.D % 8 == 0 && a.qs[0] % 8 == 0 && a.qs[1] % 8 == 0 && a.qs[2] % 8 == 0 && a.ks[0] % 8 == 0 &&
             a.ks[1] % 8 == 0 && a.ks[2] % 8 == 0 && reinterpret_cast<uintptr_t>(a.q) % 16 == 0 &&
             reinterpret_cast<uintptr_t>(a.k) % 16 == 0;
  const int dc = pl.D / 8;
  const int64_t work[5] = {a.B * a.H * a.Q * dc, a.B * a.H * pl.npad * dc, a.B * a.H * (pl.npad / 8) * pl.D,
                           a.H * a.Q * (pl.npad / 4), pl.mask_rows * pl.nblk * 64};
  // Bias views with the heads innermost (the diffusion transformer's rearranged pair logits)
  // are read a whole head vector per thread.
  const bool head_minor = a.bias && a.bias_dtype == XFH_BF16 && a.bs[1] == 1 && a.H % 8 == 0 &&
                          a.bs[2] % 8 == 0 && a.bs[3] % 8 == 0 &&
                          reinterpret_cast<uintptr_t>(a.bias) % 16 == 0;
  const bool packed = a.bias && (a.bias_dtype == XFH_BIAS_PACKED || a.bias_dtype == XFH_BIAS_PACKED_BF16);
  p.nparts = 0;
  p.start[0] = 0;
  for (int part = 0; part < 5; ++part) {
    if (part == 3 && packed) continue;             // already in the kernel's layout
    const int64_t n_work = part == 3 && head_minor ? a.Q * pl.npad : work[part];
    const int64_t blocks = ceil_div(n_work, 256);
    if (blocks == 0) continue;
    p.id[p.nparts] = part == 3 && head_minor ? 5 : part;
    p.start[p.nparts + 1] = p.start[p.nparts] + blocks;
    ++p.nparts;
  }
  if (p.start[p.nparts] > (int64_t(1) << 31) - 1) return fail(XFH_EUNSUPPORTED, "dot_product_attention: problem too large");
  if (p.nparts > 0) mha_prepare_kernel<<<dim3(unsigned(p.start[p.nparts])), 256, 0, s>>>(p);
  XFH_TRY(check_launch("mha_prepare"));

  GridAttentionArgs ga;
  ga.q = p.q; ga.k = p.k; ga.vt = p.vt; ga.maskbits = p.words;
  ga.bias = packed ? a.bias : p.bias;
  ga.bias_bf16 = packed && a.bias_dtype == XFH_BIAS_PACKED_BF16;
  ga.out = static_cast<bf16 *>(a.o);
  ga.osb = a.os[0]; ga.ost = a.os[2]; ga.ohs = a.os[1];
  ga.mbs = per_row ? pl.nblk : 0;
  ga.B = int(a.B); ga.H = int(a.H); ga.Nq = int(a.Q); ga.N = int(a.K);
  ga.Npad = int(pl.npad); ga.Nblk = int(pl.nblk); ga.Dv = int(a.Dv);
  return mha_attention(ga, pl.D, s);
}

// ---- self-attention on operands projected straight into the kernel's layouts

namespace {

// words[b][w]: one wavefront per word, lane j = key 64 w + j.
__global__ void mask_words_kernel(const void *__restrict__ mask, int dtype, int64_t stride, int64_t rows,
                                  int64_t T, int64_t nblk, uint64_t *__restrict__ words) {
  const int64_t word = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (word >= rows * nblk) return;
  const int64_t b = word / nblk, key = (word % nblk) * 64 + (threadIdx.x & 63);
  const bool keep = key < T && (!mask || load_any(mask, dtype, b * stride + key) != 0.f);
  const uint64_t ballot = __ballot(keep);
  if ((threadIdx.x & 63) == 0) words[word] = ballot;
}

}  // namespace

int attention_operands_dims(int64_t T, int64_t Dh, int *dp, int64_t *tpad) {
  if (Dh <= 0 || Dh % 4 || padded_dim(Dh) == 0) return fail(XFH_EUNSUPPORTED, "attention operands: head dim must be a multiple of 4, at most 64");
  if (T <= 0 || align_up(T, 64) > grid_attention_max_n())
    return fail(XFH_EUNSUPPORTED, "attention operands: token count outside (0, xfh_attention_max_keys()]");
  *dp = padded_dim(Dh);
  *tpad = align_up(T, 64);
  return XFH_OK;
}

int attention_mask_words(const void *mask, int dtype, int64_t stride, int64_t rows, int64_t T, uint64_t *words,
                         hipStream_t s) {
  const int64_t nblk = ceil_div(T, 64), blocks = ceil_div(rows * nblk * 64, 256);
  if (blocks == 0) return XFH_OK;
  if (blocks > (int64_t(1) << 31) - 1) return fail(XFH_EUNSUPPORTED, "attention_mask_words: problem too large");
  mask_words_kernel<<<dim3(unsigned(blocks)), 256, 0, s>>>(mask, dtype, stride, rows, T, nblk, words);
  return check_launch("attention_mask_words");
}

int attention_operands(const bf16 *q, const bf16 *k, const bf16 *vt, const uint64_t *words, bool words_shared,
                       const void *bias, bool bias_bf16, const bf16 *gate, bf16 *out, int64_t B, int64_t T,
                       int64_t H, int64_t Dh, hipStream_t s) {
  int dp = 0;
  int64_t tpad = 0;
  XFH_TRY(attention_operands_dims(T, Dh, &dp, &tpad));
  GridAttentionArgs ga;
  ga.q = q; ga.k = k; ga.vt = vt; ga.maskbits = words; ga.bias = bias; ga.bias_bf16 = bias_bf16; ga.gate = gate;
  ga.out = out;
  ga.osb = T * H * Dh; ga.ost = H * Dh; ga.ohs = Dh;
  ga.mbs = words_shared ? 0 : tpad / 64;
  ga.B = int(B); ga.H = int(H); ga.Nq = int(T); ga.N = int(T);
  ga.Npad = int(tpad); ga.Nblk = int(tpad / 64); ga.Dv = int(Dh);
  return mha_attention(ga, dp, s);
}

namespace {

// Bias packing: thread = (q, key) over keys < npad, reading all G*H heads of a bf16 view whose
// heads are innermost (g stride H, h stride 1) 8 at a time.
__global__ void bias_pack_head_minor_kernel(const bf16 *__restrict__ src, int64_t sq, int64_t sk, int gh,
                                            int64_t Q, int64_t K, int64_t npad, float *__restrict__ dst) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= Q * npad) return;
  const int64_t key = idx % npad, q = idx / npad;
  const bf16 *row = src + q * sq + key * sk;
  float *out = dst + q * npad + key;
  const int64_t plane = Q * npad;
  for (int c = 0; c < gh; c += 8) {
    bf16x8 v = {};
    if (key < K) v = *reinterpret_cast<const bf16x8 *>(row + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[(c + e) * plane] = static_cast<float>(v[e]) * kLog2eF;
  }
}

// Any strides: thread = (g*H + h, q, 4 keys).
__global__ void bias_pack_kernel(const void *__restrict__ src, int dtype, int64_t H, int64_t sg, int64_t sh,
                                 int64_t sq, int64_t sk, int64_t GH, int64_t Q, int64_t K, int64_t npad,
                                 float *__restrict__ dst) {
  const int64_t quads = npad / 4;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= GH * Q * quads) return;
  const int64_t kq = idx % quads, row = idx / quads, q = row % Q, gh = row / Q;
  const int64_t base = (gh / H) * sg + (gh % H) * sh + q * sq;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t key = kq * 4 + e;
    const int64_t off = base + key * sk;
    v[e] = key < K ? (dtype == XFH_F32 ? ld<float>(src, off) : ld<bf16>(src, off)) * kLog2eF : 0.f;
  }
  *reinterpret_cast<float4 *>(dst + row * npad + kq * 4) = make_float4(v[0], v[1], v[2], v[3]);
}

}  // namespace

int attention_bias_pack(const void *bias, int dtype, const int64_t *shape, const int64_t *strides, void *packed,
                        hipStream_t s) {
  const int64_t G = shape[0], H = shape[1], Q = shape[2], K = shape[3];
  const int64_t npad = align_up(K, 64), GH = G * H;
  if (GH * Q * npad == 0) return XFH_OK;
  const bool head_minor = dtype == XFH_BF16 && strides[1] == 1 && strides[0] == H && GH % 8 == 0 &&
                          strides[2] % 8 == 0 && strides[3] % 8 == 0 &&
                          reinterpret_cast<uintptr_t>(bias) % 16 == 0;
  if (head_minor) {
    const int64_t blocks = ceil_div(Q * npad, 256);
    if (blocks > (int64_t(1) << 31) - 1) return fail(XFH_EUNSUPPORTED, "attention_bias_pack: problem too large");
    bias_pack_head_minor_kernel<<<dim3(unsigned(blocks)), 256, 0, s>>>(
        static_cast<const bf16 *>(bias), strides[2], strides[3], int(GH), Q, K, npad, static_cast<float *>(packed));
  } else {
    const int64_t blocks = ceil_div(GH * Q * (npad / 4), 256);
    if (blocks > (int64_t(1) << 31) - 1) return fail(XFH_EUNSUPPORTED, "attention_bias_pack: problem too large");
    bias_pack_kernel<<<dim3(unsigned(blocks)), 256, 0, s>>>(bias, dtype, H, strides[0], strides[1], strides[2],
                                                             strides[3], GH, Q, K, npad, static_cast<float *>(packed));
  }
  return check_launch("attention_bias_pack");
}

namespace {

// Operands of the grid attention at widths off the fast path, from the row-major projection
// rows [q | k | v] (row stride ld, c = H dh columns each): workgroup = (batch row b, 64
// tokens). The tile's rows are read whole (16-byte pieces) into LDS; q (times scale), k and
// v^T (the kernel's key order) are written as runs of the kernel's layouts at head dim D,
// zero beyond dh and for tokens >= T. Row (b, t) of the projection is pair row b n + t, or
// t n + b for the ending node (transpose).
constexpr int kRepackTokens = 64;
__global__ __launch_bounds__(256) void qkv_repack_kernel(const bf16 *__restrict__ qkv, int64_t ld, int T, int Tpad,
                                                         int H, int dh, int D, int transpose, float scale,
                                                         bf16 *__restrict__ q, bf16 *__restrict__ k,
                                                         bf16 *__restrict__ vt) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int c = H * dh, width = 3 * c, lw = width + 8;        // LDS row: 16 bytes of padding
  bf16 *tile = reinterpret_cast<bf16 *>(smem);
  const int b = blockIdx.y, t0 = blockIdx.x * kRepackTokens, tid = threadIdx.x;
  const int chunks = width / 8;
  for (int i = tid; i < kRepackTokens * chunks; i += 256) {
    const int t = i / chunks, ch = i - t * chunks, tok = t0 + t;
    bf16x8 v = {};
    if (tok < T) {
      const int64_t row = transpose ? int64_t(tok) * T + b : int64_t(b) * T + tok;
      v = *reinterpret_cast<const bf16x8 *>(qkv + row * ld + ch * 8);
    }
    *reinterpret_cast<bf16x8 *>(tile + t * lw + ch * 8) = v;
  }
  __syncthreads();
  const int dc = D / 8;
  // q and k: thread = (head, token, 8-dim chunk)
  for (int i = tid; i < H * kRepackTokens * dc; i += 256) {
    const int ch = i % dc, rest = i / dc, t = rest % kRepackTokens, h = rest / kRepackTokens, tok = t0 + t;
    bf16x8 vq, vk;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = ch * 8 + e;
      const bool in = d < dh && tok < T;
      vq[e] = bf16(in ? static_cast<float>(tile[t * lw + h * dh + d]) * scale : 0.f);
      vk[e] = in ? tile[t * lw + c + h * dh + d] : bf16(0.f);
    }
    const int64_t bh = int64_t(b) * H + h;
    if (tok < T) *reinterpret_cast<bf16x8 *>(q + (bh * T + tok) * D + ch * 8) = vq;
    *reinterpret_cast<bf16x8 *>(k + (bh * Tpad + tok) * D + ch * 8) = vk;
  }
  // v^T: thread = (head, dim, 8-position group); position p of a run of 32 holds key
  // 4g + j (p = 8g + j, j < 4) or 16 + 4g + j - 4 (j >= 4).
  for (int i = tid; i < H * D * (kRepackTokens / 8); i += 256) {
    const int g8 = i % (kRepackTokens / 8), rest = i / (kRepackTokens / 8), d = rest % D, h = rest / D;
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int pos = g8 * 8 + e, run = pos & ~31, w = pos & 31, g = w >> 3, j = w & 7;
      const int key = run + (j < 4 ? 4 * g + j : 16 + 4 * g + j - 4);
      v[e] = (d < dh && t0 + key < T) ? tile[key * lw + 2 * c + h * dh + d] : bf16(0.f);
    }
    *reinterpret_cast<bf16x8 *>(vt + ((int64_t(b) * H + h) * D + d) * Tpad + t0 + g8 * 8) = v;
  }
}

}  // namespace

int qkv_repack(const bf16 *qkv, int64_t ld, int64_t B, int64_t T, int64_t H, int64_t dh, int transpose, float scale,
               bf16 *q, bf16 *k, bf16 *vt, hipStream_t s) {
  const int D = padded_dim(dh);
  const int64_t c = H * dh, tpad = align_up(T, 64), lds = kRepackTokens * (3 * c + 8) * 2;
  if (D == 0 || c % 8 || ld % 8 || ld < 3 * c || lds > 65536 || B > 65535 || tpad > grid_attention_max_n() ||
      reinterpret_cast<uintptr_t>(qkv) % 16 || (transpose && B != T))
    return fail(XFH_EUNSUPPORTED, "qkv_repack: unsupported shape");
  if (B * T == 0) return XFH_OK;
  const dim3 grid(unsigned(tpad / kRepackTokens), unsigned(B));
  qkv_repack_kernel<<<grid, 256, size_t(lds), s>>>(qkv, ld, int(T), int(tpad), int(H), int(dh), D, transpose, scale,
                                                   q, k, vt);
  return check_launch("qkv_repack");
}

}  // namespace xfh
