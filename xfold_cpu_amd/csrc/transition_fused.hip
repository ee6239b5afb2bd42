// Fused pair transition (bf16 compute, c = 128, hidden 4c = 512), xfold/nn/primitives.py:33-37:
// LN(x) -> GLU(x Wg, x Wv) = silu(x Wg) * (x Wv) -> transition2 -> x += update.
//
// Row panel of 128 rows (panel.h). The packed transition1 weight streams through two LDS
// buffers in chunks of 64 packed rows (32 hidden features: 16 gate + 16 value rows per
// wavefront column), the GLU result goes to a [128 rows x 128 features] LDS tile, and after
// every 4 chunks the tile is multiplied by the matching 128-column block of transition2
// (staged in the same two buffers, one 64-output half each) into fp32 accumulators that
// persist across the 4 feature blocks. The hidden activations never reach HBM.
#include "common.h"
#include "kernels.h"
#include "panel.h"

namespace xfh {

namespace {

using namespace panel;

constexpr int HID = 4 * K;             // hidden features (512)
constexpr int W1_ROWS = 2 * HID;       // packed GLU rows (1024)
constexpr int FB = 128;                // features per block

// Stage rows [row0, row0+64) x cols [col0, col0+128) of a row-major matrix with leading dim ld.
__device__ __forceinline__ void fetch_block(const bf16 *W, int row0, int ld, int col0, BStage &st) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + i * 256;
    const int r = idx >> 4, c = (idx & 15) * 8;
    st.v[i] = *reinterpret_cast<const uint4 *>(W + int64_t(row0 + r) * ld + col0 + c);
  }
}

template <typename TIN, typename TOUT>
__global__ __launch_bounds__(256, 2) void transition_kernel(TransitionArgs a) {
  __shared__ bf16 lds_a[A_ELEMS];                  // LN tile, then the hidden tile
  __shared__ bf16 lds_b[2 * B_ELEMS];              // W1 chunks / W2 halves
  auto bbuf = [&](int i) -> bf16 * { return lds_b + (i & 1) * B_ELEMS; };

  const int64_t row0 = int64_t(blockIdx.x) * ROWS;
  const int valid = int(a.rows - row0 < ROWS ? a.rows - row0 : ROWS);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1, col = lane & 15, grp = lane >> 4;
  const TIN *x = static_cast<const TIN *>(a.x);

  ln_panel<TIN>([&](int r) -> const TIN * { return r < valid ? x + (row0 + r) * K : nullptr; },
                a.ln_w, a.ln_b, a.eps, lds_a);
  __syncthreads();
  AFrags af;
  load_a_frags(lds_a, wm, af);
  BStage st1, st2;
  fetch_b(a.w1, 0, W1_ROWS, st1);
  stash_b(st1, bbuf(0));
  __syncthreads();                                 // A tile consumed; bbuf(0) ready

  f32x4 out[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) out[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16 *htile = lds_a;                             // [128 rows][PITCH], 128 features

  for (int fb = 0; fb < HID / FB; ++fb) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = fb * 4 + jj;
      if (jj < 3) fetch_b(a.w1, (j + 1) * CHUNK, W1_ROWS, st1);
      else fetch_block(a.w2, 0, HID, fb * FB, st1);          // W2 half 0 for this block
      if (jj == 2) fetch_block(a.w2, CHUNK, HID, fb * FB, st2);  // W2 half 1
      f32x4 acc[4][2];
      zero(acc);
      mma_chunk(af, bbuf(j), wn, acc);
      // features fb*128 + jj*32 + wn*16 + col: gate = tile 0, value = tile 1
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          htile[(wm * 64 + mt * 16 + grp * 4 + e) * PITCH + jj * 32 + wn * 16 + col] =
              bf16(siluf_(acc[mt][0][e]) * acc[mt][1][e]);
      stash_b(st1, bbuf(j + 1));
      __syncthreads();
    }
    // bbuf(0) holds W2 half 0; bbuf(1) is free: W2 half 1 goes there.
    stash_b(st2, bbuf(1));
    if (fb + 1 < HID / FB) fetch_b(a.w1, (fb + 1) * 4 * CHUNK, W1_ROWS, st1);
    __syncthreads();
    const bf16 *w2h = bbuf(wn);                    // this wavefront's 64 output columns
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      bf16x8 ha[4], wb[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        ha[mt] = *reinterpret_cast<const bf16x8 *>(htile + (wm * 64 + mt * 16 + col) * PITCH + ks * 32 + grp * 8);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        wb[nt] = *reinterpret_cast<const bf16x8 *>(w2h + (nt * 16 + col) * PITCH + ks * 32 + grp * 8);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) out[mt][nt] = mfma16(ha[mt], wb[nt], out[mt][nt]);
    }
    __syncthreads();
    if (fb + 1 < HID / FB) {
      stash_b(st1, bbuf(0));
      __syncthreads();
    }
  }

  // update (bf16, as the reference's transition2 output) -> residual
  bf16 *stage = lds_a;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        stage[(wm * 64 + mt * 16 + grp * 4 + e) * PITCH + wn * 64 + nt * 16 + col] = bf16(out[mt][nt][e]);
  __syncthreads();
  TOUT *dst_base = static_cast<TOUT *>(a.out);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int idx = tid + i * 256;
    const int r = idx >> 4, c = (idx & 15) * 8;
    if (r >= valid) continue;
    TOUT *dst = dst_base + (row0 + r) * K + c;
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

}  // namespace

int transition_fused(const TransitionArgs &a, int x_dtype, int out_dtype, hipStream_t s) {
  if (a.rows == 0) return XFH_OK;
  const int64_t panels = ceil_div(a.rows, ROWS);
  KernelTimer timer("transition", s);
  if (x_dtype == XFH_BF16 && out_dtype == XFH_BF16)
    transition_kernel<bf16, bf16><<<dim3(panels), 256, 0, s>>>(a);
  else if (x_dtype == XFH_BF16 && out_dtype == XFH_F32)
    transition_kernel<bf16, float><<<dim3(panels), 256, 0, s>>>(a);
  else if (x_dtype == XFH_F32 && out_dtype == XFH_F32)
    transition_kernel<float, float><<<dim3(panels), 256, 0, s>>>(a);
  else
    transition_kernel<float, bf16><<<dim3(panels), 256, 0, s>>>(a);
  return check_launch("transition");
}

}  // namespace xfh
