// xfh_triangle_multiplication_noalloc: the triangle multiplication entry point for callers
// that cannot allocate device memory (code under HIP graph capture, serving loops that
// forbid allocation). Its scratch (the contraction's operands and result, or the
// general path's intermediates) lives in one file-scope device array instead of a
// caller-provided workspace; every other argument and the result are those of
// xfh_triangle_multiplication, whose kernels it runs.
//
// Each device holds its own copy of `scratch` from the library's load until the process
// ends. Calls on one device share it and overlapping calls (concurrent streams, host
// threads) race on it; calls ordered on one stream do not. The kernels write every byte
// of scratch they later read (operand pad columns included), so nothing is cleared
// between calls and the contents a call leaves behind never reach the next one's result.
#include <mutex>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"

static constexpr int64_t kScratchBytes = XFH_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// Device address of `scratch` on the current device, looked up once per device. The host
// name `scratch` is only a handle for this lookup, never a device address.
int scratch_address(void **out) {
  static std::mutex mu;
  static std::vector<void *> addresses;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return xfh::fail(XFH_EHIP, std::string("hipGetDevice: ") + hipGetErrorString(err));
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= int(addresses.size())) addresses.resize(dev + 1, nullptr);
  if (!addresses[dev]) {
    void *ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return xfh::fail(XFH_EHIP, std::string("triangle_multiplication_noalloc: hipGetSymbolAddress: ") +
                                     hipGetErrorString(err));
    addresses[dev] = ptr;
  }
  *out = addresses[dev];
  return XFH_OK;
}

}  // namespace

extern "C" int xfh_triangle_multiplication_noalloc(
    const void *pair, int pair_dtype, const void *mask, int mask_dtype, int64_t n, int64_t c, int outgoing,
    const float *left_w, const float *left_b, float left_eps, const void *proj_w, const void *gate_w,
    const float *center_w, const float *center_b, float center_eps, const void *out_w,
    const void *gating_w, int dtype, void *out, int out_dtype, int accumulate, void *stream) {
  const int64_t need = xfh_triangle_multiplication_workspace_size(n, c, dtype);
  if (need < 0) return xfh::fail(XFH_EINVAL, "triangle_multiplication_noalloc: bad size or dtype");
  if (need > kScratchBytes)
    return xfh::fail(XFH_EUNSUPPORTED,
                     "triangle_multiplication_noalloc: n = " + std::to_string(n) + ", c = " + std::to_string(c) +
                         " needs " + std::to_string(need) + " bytes of scratch; the no-alloc entry point has " +
                         std::to_string(kScratchBytes) + " (use xfh_triangle_multiplication with a workspace)");
  void *ws = nullptr;
  XFH_TRY(scratch_address(&ws));
  return xfh_triangle_multiplication(pair, pair_dtype, mask, mask_dtype, n, c, outgoing, left_w, left_b, left_eps,
                                     proj_w, gate_w, center_w, center_b, center_eps, out_w, gating_w, dtype, out,
                                     out_dtype, accumulate, ws, kScratchBytes, stream);
}
