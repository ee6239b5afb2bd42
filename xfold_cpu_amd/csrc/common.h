// Shared device/host helpers for the xfold HIP library (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/xfold_hip.h"

namespace xfh {

typedef __bf16 bf16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- error reporting (host)
void set_error(const std::string &message);
int fail(int code, const std::string &message);
int check_launch(const char *what);

#define XFH_REQUIRE(cond, msg)                                   \
  do {                                                           \
    if (!(cond)) return ::xfh::fail(XFH_EINVAL, (msg));          \
  } while (0)

#define XFH_TRY(expr)                                            \
  do {                                                           \
    int _status = (expr);                                        \
    if (_status != XFH_OK) return _status;                       \
  } while (0)

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Opt-in per-kernel timing (xfh_set_kernel_timing): when enabled, a KernelTimer brackets a
// launch with HIP events recorded on the launch stream.
// `work` (algorithmic FLOPs or bytes of the launch) is summed with the durations, so a
// kernel launched on several shapes has one aggregate rate. A launch made through
// `launch()` is timed by its own dispatch (hipExtLaunchKernelGGL updates the two events
// with the kernel's start and end), so the interval excludes the event packets around it;
// otherwise the timer brackets whatever was enqueued in its scope with recorded events.
class KernelTimer {
 public:
  // dispatch = true: the scope holds one launch made through launch() (nothing is recorded
  // before it).
  KernelTimer(const char *name, hipStream_t stream, double work = 0.0, bool dispatch = false);
  ~KernelTimer();
  template <class K, class... Args>
  void launch(K kernel, dim3 grid, dim3 block, uint32_t shared, Args... args) {
    if (enabled_ && dispatch_events()) {
      hipExtLaunchKernelGGL(kernel, grid, block, shared, stream_, static_cast<hipEvent_t>(start_),
                            static_cast<hipEvent_t>(stop_), 0, args...);
      return;
    }
    kernel<<<grid, block, shared, stream_>>>(args...);
  }
 private:
  bool dispatch_events();                 // the dispatch's own start/stop pair
  const char *name_;
  hipStream_t stream_;
  double work_;
  bool enabled_ = false;
  void *start_ = nullptr, *stop_ = nullptr;
};
// Compute units of the current device (cached per device).
int device_cu_count(int *cus);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t align_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }
// Workgroups for a persistent kernel whose `per_wg` wavefronts take `units` work units
// round-robin, at most one workgroup per CU: as few as give every wavefront the same number
// of rounds as `cus` workgroups would (N=384 pair kernels: 192 or 231 instead of 256, 3% of
// a block, with the weights each workgroup stages into LDS fetched fewer times).
inline int64_t balanced_grid(int64_t units, int64_t per_wg, int cus) {
  if (units <= 0) return 0;
  return ceil_div(units, per_wg * ceil_div(units, per_wg * int64_t(cus)));
}

// Bump allocator over a caller-provided workspace; 256-byte aligned slices.
struct Carver {
  char *base;
  int64_t used = 0, cap;
  Carver(void *b, int64_t c) : base(static_cast<char *>(b)), cap(c) {}
  void *take(int64_t bytes) {
    used = align_up(used, 256);
    void *p = base ? base + used : nullptr;
    used += bytes;
    return p;
  }
};

// ---------------------------------------------------------------- device helpers
template <typename T> __device__ __forceinline__ float to_f32(T v) { return static_cast<float>(v); }
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }

template <typename T> __device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }

// sigmoid / SiLU with the hardware reciprocal (1 ulp) instead of an IEEE division.
// Workgroup barrier for rings of direct global->LDS loads: waits for this wavefront's LDS
// operations only, then s_barrier. __syncthreads() also waits vmcnt(0), i.e. for every
// direct load in flight, including those of the steps still ahead of the one about to be
// read; the rings already wait, per wavefront, exactly for the loads of that step. The asm
// has a memory clobber, so no LDS access moves across it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// DPP lane exchange inside a 16-lane row (no LDS traffic).
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over each row of 16 lanes: xor 1, xor 2 (quad permutes), then half-row and row mirrors.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);   // row_half_mirror
  v += dpp_f32<0x140>(v);   // row_mirror
  return v;
}

// Reads element `i` of a tensor whose dtype is only known at run time (masks, biases).
__device__ __forceinline__ float load_any(const void *p, int dtype, int64_t i) {
  if (dtype == XFH_F32) return reinterpret_cast<const float *>(p)[i];
  if (dtype == XFH_BF16) return static_cast<float>(reinterpret_cast<const bf16 *>(p)[i]);
  return reinterpret_cast<const uint8_t *>(p)[i] ? 1.0f : 0.0f;
}

template <typename T> __device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Sum across groups of `width` consecutive lanes (width a power of two <= 64).
template <int width> __device__ __forceinline__ float group_sum(float v) {
  if constexpr (width >= 16) {
    v = row16_sum(v);
#pragma unroll
    for (int o = 16; o < width; o <<= 1) v += __shfl_xor(v, o, kWave);
    return v;
  } else {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
  }
}

// MFMA wrappers. Both keep the 16x16 output layout: lane l holds column l%16 and rows
// 4*(l/16) + {0,1,2,3}. For bf16 a lane supplies 8 consecutive k of its row (k-group
// l/16). For fp32 the 16x16x4 instruction takes one k per lane; eight of them consume
// the same 8-element fragment, slot s of k-group g carrying k = 8g + s. Both operands
// use the same permutation, so the dot product over the 32-wide k-step is unchanged.
__device__ __forceinline__ f32x4 mfma16(const bf16x8 &a, const bf16x8 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
struct f32x8 { float v[8]; };
__device__ __forceinline__ f32x4 mfma16(const f32x8 &a, const f32x8 &b, f32x4 c) {
#pragma unroll
  for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[s], b.v[s], c, 0, 0, 0);
  return c;
}

template <typename T> struct Frag;
template <> struct Frag<bf16> { typedef bf16x8 type; };
template <> struct Frag<float> { typedef f32x8 type; };

}  // namespace xfh
