// Flash-style scaled dot-product attention with additive bias and key mask.
//
// Semantics (xfold/fastnn/attention.py:45-66): logits = (q * scale) k^T + bias; a masked
// logit is replaced by exactly -1e9 (so a fully masked row averages v uniformly over all
// keys); softmax over keys; @ v. The logits never exist in memory: each workgroup owns 64
// queries of one (batch, head), walks the keys in blocks of 64 and keeps a running max and
// sum (online softmax, base-2: log2(e) is folded into the q.k scale, the bias and the -1e9
// fill).
//
// MFMA formulation (16x16 tiles): the kernel computes S^T = K Q^T so that after the MFMA a
// lane holds four keys of ONE query (column l%16). That is exactly the B-operand layout of
// the next product O^T = V^T P^T, up to a fixed permutation of the 32 keys of a k-step,
// which the V^T fragment read reproduces. V is stored transposed in LDS for that read.
#include "common.h"
#include "kernels.h"

namespace xfh {

namespace {

constexpr int QB = 64;    // queries per workgroup (16 per wavefront)
constexpr int KB = 64;    // keys per block

template <typename T> struct AttnSmemPitch { static constexpr int kPad = 16 / sizeof(T); };

template <typename T, typename TO, int DP, int DVT>
__global__ __launch_bounds__(256) void attention_kernel(AttentionArgs a) {
  constexpr int kPad = AttnSmemPitch<T>::kPad;
  constexpr int KP = DP + kPad;          // K tile pitch
  constexpr int VP = KB + kPad;          // V^T tile pitch
  __shared__ T ks[KB * KP];
  __shared__ T vt[DVT * 16 * VP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.z, h = blockIdx.y;
  const int64_t q0 = int64_t(blockIdx.x) * QB + wave * 16;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t query = q0 + col;
  const bool qvalid = query < a.Q;

  const T *qp = static_cast<const T *>(a.q) + b * a.qs[0] + h * a.qs[1];
  const T *kp = static_cast<const T *>(a.k) + b * a.ks[0] + h * a.ks[1];
  const T *vp = static_cast<const T *>(a.v) + b * a.vs[0] + h * a.vs[1];

  // Q^T fragments (B operand): lane supplies d = step*32 + 8*grp + s of its query, as
  // stored (the scale goes onto the fp32 products, so q is not rounded a second time).
  typename Frag<T>::type qf[DP / 32];
  const float qscale = a.scale * kLog2e;
#pragma unroll
  for (int st = 0; st < DP / 32; ++st) {
    T tmp[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int64_t d = st * 32 + grp * 8 + s;
      tmp[s] = (qvalid && d < a.D) ? qp[query * a.qs[2] + d] : T(0);
    }
    __builtin_memcpy(&qf[st], tmp, sizeof(tmp));
  }

  const char *biasb = static_cast<const char *>(a.bias);
  const uint8_t *maskb = static_cast<const uint8_t *>(a.mask);

  float m_run = -INFINITY;
  float l_part = 0.f;
  f32x4 o[DVT];
#pragma unroll
  for (int t = 0; t < DVT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const float masked_logit = -1e9f * kLog2e;
  for (int64_t kb0 = 0; kb0 < a.K; kb0 += KB) {
    __syncthreads();
    // Cooperative load of K [KB x DP] and V^T [DVT*16 x KB], zero outside the tensors.
    for (int idx = tid; idx < KB * DP; idx += 256) {
      const int r = idx / DP, d = idx % DP;
      const int64_t key = kb0 + r;
      ks[r * KP + d] = (key < a.K && d < a.D) ? kp[key * a.ks[2] + d] : T(0);
    }
    for (int idx = tid; idx < KB * DVT * 16; idx += 256) {
      const int r = idx / (DVT * 16), d = idx % (DVT * 16);
      const int64_t key = kb0 + r;
      vt[d * VP + r] = (key < a.K && d < a.Dv) ? vp[key * a.vs[2] + d] : T(0);
    }
    __syncthreads();

    // S^T for 4 tiles of 16 keys: lane holds keys kt*16 + 4*grp + e of query `col`.
    float sv[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < DP / 32; ++st) {
        typename Frag<T>::type kf;
        const T *src = &ks[(kt * 16 + col) * KP + st * 32 + grp * 8];
        __builtin_memcpy(&kf, src, sizeof(kf));
        acc = mfma16(kf, qf[st], acc);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[kt][e] = acc[e] * qscale;
    }

    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t key = kb0 + kt * 16 + grp * 4 + e;
        float v = sv[kt][e];
        if (key >= a.K) {
          v = -INFINITY;
        } else if (qvalid) {
          if (a.bias) {
            const int64_t off = b * a.bs[0] + h * a.bs[1] + query * a.bs[2] + key * a.bs[3];
            const float bv = a.bias_dtype == XFH_F32
                                 ? reinterpret_cast<const float *>(biasb)[off]
                                 : static_cast<float>(reinterpret_cast<const bf16 *>(biasb)[off]);
            v += bv * kLog2e;
          }
          if (maskb) {
            const int64_t off = b * a.ms[0] + h * a.ms[1] + query * a.ms[2] + key * a.ms[3];
            if (load_any(maskb, a.mask_dtype, off) == 0.f) v = masked_logit;
          }
        }
        sv[kt][e] = v;
        bmax = fmaxf(bmax, v);
      }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float m_new = fmaxf(m_run, bmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    m_run = m_new;
    l_part *= alpha;
#pragma unroll
    for (int t = 0; t < DVT; ++t) o[t] *= alpha;

    float pv[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[kt][e] = exp2f(sv[kt][e] - m_use);
        l_part += pv[kt][e];
      }

    // O^T += V^T P^T over two 32-key steps; slot s<4 -> key 4*grp+s of the even tile,
    // slot s>=4 -> key 4*grp+s-4 of the odd tile (same permutation on both operands).
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      T ptmp[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ptmp[e] = from_f32<T>(pv[2 * c][e]);
        ptmp[4 + e] = from_f32<T>(pv[2 * c + 1][e]);
      }
      typename Frag<T>::type pf;
      __builtin_memcpy(&pf, ptmp, sizeof(ptmp));
#pragma unroll
      for (int t = 0; t < DVT; ++t) {
        T vtmp[8];
        const T *row = &vt[(t * 16 + col) * VP + c * 32 + grp * 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vtmp[e] = row[e];
          vtmp[4 + e] = row[16 + e];
        }
        typename Frag<T>::type vf;
        __builtin_memcpy(&vf, vtmp, sizeof(vtmp));
        o[t] = mfma16(vf, pf, o[t]);
      }
    }
  }

  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!qvalid) return;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;   // no keys at all -> zeros
  TO *op = static_cast<TO *>(a.o) + b * a.os[0] + h * a.os[1] + query * a.os[2];
#pragma unroll
  for (int t = 0; t < DVT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t d = t * 16 + grp * 4 + e;
      if (d < a.Dv) op[d] = from_f32<TO>(o[t][e] * inv);
    }
}

template <typename T, typename TO, int DP>
int launch_dv(const AttentionArgs &a, hipStream_t s) {
  dim3 grid(ceil_div(a.Q, QB), a.H, a.B);
  const int dvt = int(ceil_div(a.Dv, 16));
  switch (dvt) {
    case 1: attention_kernel<T, TO, DP, 1><<<grid, 256, 0, s>>>(a); break;
    case 2: attention_kernel<T, TO, DP, 2><<<grid, 256, 0, s>>>(a); break;
    case 3: attention_kernel<T, TO, DP, 3><<<grid, 256, 0, s>>>(a); break;
    case 4: attention_kernel<T, TO, DP, 4><<<grid, 256, 0, s>>>(a); break;
    default: return fail(XFH_EUNSUPPORTED, "attention: value head dim must be <= 64");
  }
  return check_launch("attention");
}

template <typename T, typename TO>
int launch_typed(const AttentionArgs &a, hipStream_t s) {
  if (a.D <= 32) return launch_dv<T, TO, 32>(a, s);
  if (a.D <= 64) return launch_dv<T, TO, 64>(a, s);
  return fail(XFH_EUNSUPPORTED, "attention: head dim must be <= 64");
}

}  // namespace

int attention(const AttentionArgs &a, int dtype, hipStream_t s) {
  if (a.B == 0 || a.H == 0 || a.Q == 0 || a.Dv == 0) return XFH_OK;
  if (a.H > 65535 || a.B > 65535) return fail(XFH_EUNSUPPORTED, "attention: B and H must be <= 65535");
  if (dtype == XFH_BF16 && a.out_dtype == XFH_BF16) return launch_typed<bf16, bf16>(a, s);
  if (dtype == XFH_BF16 && a.out_dtype == XFH_F32) return launch_typed<bf16, float>(a, s);
  if (dtype == XFH_F32 && a.out_dtype == XFH_F32) return launch_typed<float, float>(a, s);
  return fail(XFH_EUNSUPPORTED, "attention: dtypes must be bf16->bf16, bf16->f32 or f32->f32");
}

}  // namespace xfh
