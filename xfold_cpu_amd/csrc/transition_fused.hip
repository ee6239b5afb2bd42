// Fused pair transition (bf16 compute, c = 128, hidden 4c = 512), xfold/nn/primitives.py:33-37:
// LN(x) -> GLU(x Wg, x Wv) = silu(x Wg) * (x Wv) -> transition2 -> x += update.
//
// Persistent kernel, two independent workgroups of 4 wavefronts per CU, each wavefront
// owning up to 2 sets of 16 positions per step with everything in registers (rowstep.h
// layouts):
//   - a set's LayerNorm output is the K-layout B operand of transition1;
//   - the weights stream through a 3-slot LDS ring in chunks of 32 hidden features
//     (64 packed transition1 rows, 16 KB, plus the matching 128 x 32 block of transition2,
//     8 KB) filled by direct global -> LDS loads two chunks ahead, one barrier per chunk;
//   - transition1 rows are permuted on the way in so that the gate and value tiles of a
//     chunk land as lane g holding hidden features 8 g .. 8 g + 7: silu(gate) * value is
//     then directly the K-layout operand of transition2, whose fp32 out^T accumulators
//     persist across the 16 chunks. The hidden activations never leave the registers.
// Within a chunk the SiLU depends on transition1's MFMAs and transition2's on the SiLU, so
// a wavefront does not overlap them itself, and it issues at most one 1 KB LDS read every
// ~28 cycles; the second workgroup of the CU (own barriers, so not phase-locked to the
// first) fills the SIMDs while one waits on LDS, its chunk or a SiLU -> MFMA dependency.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "kernels.h"
#include "rowstep.h"

namespace xfh {

namespace {

using namespace rowstep;

constexpr int HID = 4 * C;                   // hidden features (512)
constexpr int CH = 32;                       // hidden features per chunk
constexpr int NCHUNK = HID / CH;             // 16
constexpr int W1_STAGE = 64 * C;             // 4 tiles of 16 packed rows x 128 (bf16)
constexpr int W2_STAGE = C * CH;             // 128 outputs x 32 hidden (bf16)
constexpr int SLOT = W1_STAGE + W2_STAGE;    // 24 KB
constexpr int SLOTS = 3;
constexpr int WAVES = 4;
constexpr int SEGS = SLOT / 512;             // 1 KB direct-load segments per chunk (24)
constexpr int SEG_PER_WAVE = SEGS / WAVES;   // 6
constexpr int SETS = 2;                      // 16-position sets per wavefront per step
constexpr int STEP_SETS = SETS * WAVES;      // 8
constexpr int WG_PER_CU = 2;                 // independent workgroups per CU
static_assert(SEGS % WAVES == 0, "segments spread evenly");
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

// Waits until at most N of this thread's vector memory operations are outstanding.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 16-byte direct global -> LDS load per lane from a uniform base and a 32-bit byte offset.
__device__ __forceinline__ void dma16(const void *base, uint32_t off, bf16 *lds) {
  __builtin_amdgcn_global_load_lds((global_void *)(static_cast<const char *>(base) + off), (lds_void *)lds, 16, 0, 0);
}

__device__ __forceinline__ float silu_mul(float gate, float value) {
  return gate * value * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gate * -1.4426950408889634f));
}

// A position's K-layout channels (32 ks + 8 g + j) as loaded.
template <typename T> struct RawK;
template <> struct RawK<bf16> {
  bf16x8 v[4];
  __device__ __forceinline__ void load(const bf16 *row, int g) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) v[ks] = *reinterpret_cast<const bf16x8 *>(row + 32 * ks + 8 * g);
  }
  __device__ __forceinline__ void to_float(float (&f)[32]) const {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) f[8 * ks + j] = static_cast<float>(v[ks][j]);
  }
};
template <> struct RawK<float> {
  float4 v[8];
  __device__ __forceinline__ void load(const float *row, int g) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      v[2 * ks] = *reinterpret_cast<const float4 *>(row + 32 * ks + 8 * g);
      v[2 * ks + 1] = *reinterpret_cast<const float4 *>(row + 32 * ks + 8 * g + 4);
    }
  }
  __device__ __forceinline__ void to_float(float (&f)[32]) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      f[4 * i] = v[i].x; f[4 * i + 1] = v[i].y; f[4 * i + 2] = v[i].z; f[4 * i + 3] = v[i].w;
    }
  }
};

// RES_INIT (bf16 in place, accumulating: the pair stack's residual update): the
// accumulators start from x itself, so the epilogue is a plain store of x + update.
// PB (with RES_INIT): the epilogue also writes the attention bias of the stored pair values
// (pair_bias.hip's arithmetic in the same order: the bf16 values moved to K-layout by lane
// swaps, LayerNorm, x . W^T over the 16-head tile, times log2(e)), so the pair is not read
// again for it (xfold/nn/pairformer.py:100-106).
template <typename TIN, typename TOUT, bool RES_INIT, bool PB>
__global__ __launch_bounds__(WAVES * 64, WG_PER_CU) void transition_kernel(TransitionArgs a, TransitionBias pb,
                                                                           int64_t total_sets) {
  __shared__ __attribute__((aligned(16))) bf16 ring[SLOTS * SLOT];
  __shared__ float lnw[C], lnb[C];
  __shared__ __attribute__((aligned(16))) bf16 w_pb[PB ? 16 * C : 8];
  __shared__ __attribute__((aligned(16))) float lnw_pb[PB ? C : 4], lnb_pb[PB ? C : 4];
  static_assert(!PB || RES_INIT, "the bias epilogue follows the in-place pair update");

  // Contiguous range of 16-position sets for this workgroup.
  const int64_t set_begin = total_sets * blockIdx.x / gridDim.x;
  const int64_t set_end = total_sets * (blockIdx.x + 1) / gridDim.x;
  const int steps = int((set_end - set_begin + STEP_SETS - 1) / STEP_SETS);
  const int total_chunks = steps * NCHUNK;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pos = lane & 15, g = lane >> 4;
  const TIN *x = static_cast<const TIN *>(a.x);
  TOUT *out = static_cast<TOUT *>(a.out);
  const int64_t rows = a.rows;
  constexpr bool res_init = RES_INIT;
  static_assert(!RES_INIT || (std::is_same<TIN, bf16>::value && std::is_same<TOUT, bf16>::value), "in-place residual needs bf16");

  // Direct-load sources of this lane's segments (seg = wave + WAVES j), chunk 0; chunk c adds
  // 64 c packed rows (transition1) or 32 c columns (transition2).
  //   seg < 16: stage rows 4 seg + lane / 16 of the transition1 stage, slot lane % 16 holding
  //     chunk slot ^ (row & 15). Stage tile 0/1 = gate, 2/3 = value; row r of tile 0/2 is
  //     hidden feature 8 (r / 4) + r % 4 of the chunk, of tile 1/3 that + 4.
  //   seg >= 16: transition2 rows 16 (seg - 16) + lane / 4 (64 B each), slot lane % 4
  //     holding chunk slot ^ ((row >> 2) & 3).
  uint32_t src_off[SEG_PER_WAVE];                    // bytes
#pragma unroll
  for (int j = 0; j < SEG_PER_WAVE; ++j) {
    const int seg = wave + WAVES * j;
    if (seg < 16) {
      const int n = 4 * seg + (lane >> 4), slot = lane & 15, chunk = slot ^ (n & 15);
      const int tile = n >> 4, r = n & 15;
      const int f = 8 * (r >> 2) + 4 * (tile & 1) + (r & 3);        // hidden feature in the chunk
      const int packed = 32 * (f >> 4) + (tile < 2 ? 0 : 16) + (f & 15);
      src_off[j] = uint32_t(packed * C + chunk * 8) * 2;
    } else {
      const int n = 16 * (seg - 16) + (lane >> 2), slot = lane & 3, chunk = slot ^ ((n >> 2) & 3);
      src_off[j] = uint32_t(n * HID + chunk * 8) * 2;
    }
  }
  // Workgroups walk the hidden chunks in rotated orders (the sum over them has no order
  // to keep): the 32 CUs of an XCD (blocks b, b + 8, ...) then read 16 different chunks
  // at any moment instead of all hitting the L2 channels of one.
  const int rot = (blockIdx.x / 8) % NCHUNK;
  auto issue = [&](int gc) {
    const int c = (gc + rot) % NCHUNK;
    bf16 *slot = ring + (gc % SLOTS) * SLOT;
    const bf16 *w1c = a.w1 + c * 64 * C, *w2c = a.w2 + c * CH;
#pragma unroll
    for (int j = 0; j < SEG_PER_WAVE; ++j) {
      const int seg = wave + WAVES * j;
      dma16(seg < 16 ? w1c : w2c, src_off[j], slot + seg * 512);
    }
  };
  LnStage sl, sl_pb;
  WeightStage<16, WAVES * 64> sw_pb;
  sl.load(a.ln_w, a.ln_b);
  if constexpr (PB) {
    sl_pb.load(pb.ln_w, pb.ln_b);
    sw_pb.load([&](int r) -> const bf16 * { return r < pb.heads ? pb.w + r * C : nullptr; }, false);
  }
  if (total_chunks > 0) issue(0);
  if (total_chunks > 1) issue(1);
  sl.store(lnw, lnb);                                // (its loads are older than the chunks')
  if constexpr (PB) {
    sl_pb.store(lnw_pb, lnb_pb);
    sw_pb.store(w_pb);
  }
  __syncthreads();                                   // LayerNorm parameters (and bias weight)

  // The bias of the set whose first position is p0, from its updated values acc (every lane
  // takes part: the lane swaps and the LayerNorm's sums cross lanes).
  auto bias_epilogue = [&](const f32x4 (&acc)[8], int64_t p0) {
    if constexpr (PB) {
      bf16x8 zk[4];
      float v[32];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const float lo[4] = {acc[2 * ks][0], acc[2 * ks][1], acc[2 * ks][2], acc[2 * ks][3]};
        const float hi[4] = {acc[2 * ks + 1][0], acc[2 * ks + 1][1], acc[2 * ks + 1][2], acc[2 * ks + 1][3]};
        zk[ks] = pack_tiles(lo, hi);                 // the bf16 values the pair holds
        o_to_k_step(zk[ks]);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[8 * ks + j] = static_cast<float>(zk[ks][j]);
      }
      bf16x8 xa[4];
      ln_k(v, lnw_pb, lnb_pb, pb.eps, xa);
      f32x4 r = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) r = mfma16(xa[ks], weight_frag(w_pb, 0, ks), r);
      // lane: head `pos`, positions p0 + 4 g .. + 3
      const int h = pos;
      const int n = pb.n;
      if (h < pb.heads) {
        constexpr float kLog2e = 1.4426950408889634f;
        const int64_t q = p0 + 4 * g;
        if (n % 4 == 0 && q + 3 < rows) {
          const int64_t i = q / n, j = q - i * n;
          *reinterpret_cast<float4 *>(pb.packed + (int64_t(h) * n + i) * pb.npad + j) =
              make_float4(r[0] * kLog2e, r[1] * kLog2e, r[2] * kLog2e, r[3] * kLog2e);
          if (j + 4 == n)
            for (int jj = n; jj < pb.npad; ++jj) pb.packed[(int64_t(h) * n + i) * pb.npad + jj] = 0.f;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (q + e >= rows) continue;
            const int64_t i = (q + e) / n, j = (q + e) - i * n;
            float *row = pb.packed + (int64_t(h) * n + i) * pb.npad;
            row[j] = r[e] * kLog2e;
            if (j + 1 == n)
              for (int jj = n; jj < pb.npad; ++jj) row[jj] = 0.f;
          }
        }
      }
    }
  };

  int gc = 0;                                        // chunks consumed so far

  // One step of NS sets (positions (base + WAVES i) * 16 + pos): every set is computed
  // unconditionally so that the sets' MFMA and VALU chains interleave.
  auto run_step = [&](int64_t base, auto ns_c) {
    constexpr int NS = decltype(ns_c)::value;    // 0: this wavefront only keeps pace
    constexpr int NA = NS > 0 ? NS : 1;
    bf16x8 xop[NA][4];
    f32x4 acc[NA][8];
    if constexpr (NS > 0) {
      bf16x8 id[2];
      identity_frags(id);
      RawK<TIN> raw[NA];
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int64_t p = (base + WAVES * i) * 16 + pos;
        raw[i].load(x + (p < rows ? p : rows - 1) * C, g);
      }
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        float v[32];
        raw[i].to_float(v);
        ln_k(v, lnw, lnb, a.eps, xop[i]);
        if constexpr (res_init) {
          k_to_o(id, raw[i].v, acc[i]);
          continue;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }

    for (int c = 0; c < NCHUNK; ++c, ++gc) {
      // This wavefront's loads of chunk gc have landed (those of gc + 1 may still fly),
      // then every wavefront's have, and every wavefront is done with chunk gc - 1.
      if (gc + 1 >= total_chunks) wait_vmcnt<0>();
      else wait_vmcnt<SEG_PER_WAVE>();
      ring_barrier();
      if (gc + 2 < total_chunks) issue(gc + 2);
      if constexpr (NS == 0) continue;
      const bf16 *w1s = ring + (gc % SLOTS) * SLOT, *w2s = w1s + W1_STAGE;
      // transition1: tiles 0/1 = gate, 2/3 = value, all sets side by side. The fragments
      // of k-step ks + 1 (and, during the last one, transition2's) load while the
      // MFMAs of k-step ks run.
      f32x4 h1[NA][4];
#pragma unroll
      for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) h1[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
      bf16x8 w1f[2][4], w2f[8];
#pragma unroll
      for (int t = 0; t < 4; ++t) w1f[0][t] = weight_frag(w1s, t, 0);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        // Issue order is pinned (sched_barrier): without it the register-pressure
        // scheduler sinks each read next to its first use and the wavefront waits on it.
        if (ks < 3) {
#pragma unroll
          for (int t = 0; t < 4; ++t) w1f[(ks + 1) & 1][t] = weight_frag(w1s, t, ks + 1);
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int n = 16 * t + pos;
            w2f[t] = *reinterpret_cast<const bf16x8 *>(w2s + n * CH + ((g ^ ((n >> 2) & 3)) * 8));
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < NS; ++i) h1[i][t] = mfma16(w1f[ks & 1][t], xop[i][ks], h1[i][t]);
        __builtin_amdgcn_sched_barrier(0);
      }
      // lane g: hidden 8 g + e from tiles 0 (gate) / 2 (value), 8 g + 4 + e from 1 / 3
      bf16x8 hop[NA];
#pragma unroll
      for (int i = 0; i < NS; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hop[i][e] = bf16(silu_mul(h1[i][0][e], h1[i][2][e]));
          hop[i][4 + e] = bf16(silu_mul(h1[i][1][e], h1[i][3][e]));
        }
      // transition2 block of this chunk's 32 hidden features
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int i = 0; i < NS; ++i) acc[i][t] = mfma16(w2f[t], hop[i], acc[i][t]);
    }

    // lane: position pos, channels 16 t + 4 g + e. In place: acc = x + update (one
    // rounding); otherwise the update is rounded to bf16 (the reference's transition2
    // output) and added to out when accumulating.
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int64_t p = (base + WAVES * i) * 16 + pos;
      TOUT *dst = out + p * C + 4 * g;
      if constexpr (res_init) {
        if (p < rows) {
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const float o[4] = {acc[i][t][0], acc[i][t][1], acc[i][t][2], acc[i][t][3]};
            store4f<TOUT>(dst + 16 * t, o);
          }
        }
        bias_epilogue(acc[i], (base + WAVES * i) * 16);
        continue;
      }
      if (p >= rows) continue;
      Raw4<TOUT> old[8];
      if (a.accumulate) {
#pragma unroll
        for (int t = 0; t < 8; ++t) old[t].load(dst + 16 * t);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = static_cast<float>(bf16(acc[i][t][e]));
          if (a.accumulate) o[e] += old[t][e];
        }
        store4f<TOUT>(dst + 16 * t, o);
      }
    }
  };

  for (int step = 0; step < steps; ++step) {
    // Sets of this wavefront: base + WAVES i for i < nsets (interleaved over the wavefronts,
    // so a short last step still gives every wavefront a share).
    const int64_t base = set_begin + int64_t(step) * STEP_SETS + wave;
    const int64_t left = set_end - base;
    const int nsets = left <= 0 ? 0 : int(std::min<int64_t>(SETS, (left + WAVES - 1) / WAVES));
    static_assert(SETS == 2, "one instantiation per set count");
    switch (nsets) {
      case 2: run_step(base, std::integral_constant<int, 2>{}); break;
      case 1: run_step(base, std::integral_constant<int, 1>{}); break;
      default: run_step(base, std::integral_constant<int, 0>{}); break;
    }
  }
}

}  // namespace

int transition_fused(const TransitionArgs &a, int x_dtype, int out_dtype, hipStream_t s) {
  if (a.rows == 0) return XFH_OK;
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const int64_t sets = ceil_div(a.rows, int64_t(16));
  const int grid = int(std::min<int64_t>(int64_t(cus) * WG_PER_CU, sets));
  KernelTimer timer("transition", s, 0.0, true);
  const bool in_place = a.accumulate && a.out == a.x;
  const TransitionBias none{};
  if (x_dtype == XFH_BF16 && out_dtype == XFH_BF16 && in_place)
    timer.launch(transition_kernel<bf16, bf16, true, false>, dim3(grid), dim3(WAVES * 64), 0, a, none, sets);
  else if (x_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    timer.launch(transition_kernel<bf16, bf16, false, false>, dim3(grid), dim3(WAVES * 64), 0, a, none, sets);
  else if (x_dtype == XFH_BF16 && out_dtype == XFH_F32)
    timer.launch(transition_kernel<bf16, float, false, false>, dim3(grid), dim3(WAVES * 64), 0, a, none, sets);
  else if (x_dtype == XFH_F32 && out_dtype == XFH_F32)
    timer.launch(transition_kernel<float, float, false, false>, dim3(grid), dim3(WAVES * 64), 0, a, none, sets);
  else
    timer.launch(transition_kernel<float, bf16, false, false>, dim3(grid), dim3(WAVES * 64), 0, a, none, sets);
  return check_launch("transition");
}

int transition_pair_bias(const TransitionArgs &a, const TransitionBias &b, hipStream_t s) {
  if (!a.accumulate || a.out != a.x || b.heads < 1 || b.heads > 16 || int64_t(b.n) * b.n != a.rows ||
      b.npad % 64 != 0 || b.npad < b.n)
    return fail(XFH_EINVAL, "transition_pair_bias: an in-place pair update, n * n rows, 1..16 heads, "
                            "npad a multiple of 64 >= n");
  if (a.rows == 0) return XFH_OK;
  int cus = 0;
  XFH_TRY(device_cu_count(&cus));
  const int64_t sets = ceil_div(a.rows, int64_t(16));
  const int grid = int(std::min<int64_t>(int64_t(cus) * WG_PER_CU, sets));
  KernelTimer timer("transition", s, 0.0, true);
  timer.launch(transition_kernel<bf16, bf16, true, true>, dim3(grid), dim3(WAVES * 64), 0, a, b, sets);
  return check_launch("transition_pair_bias");
}

}  // namespace xfh
