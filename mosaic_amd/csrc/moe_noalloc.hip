// A16 routed MoE layer without a caller workspace: the scratch the layer's
// kernels use (routing ids/weights, expert sort, tile list, z, down partials)
// lives in a file-scope device array instead, so a caller that cannot allocate
// device memory (code under graph capture, a serving loop, a harness that
// forbids allocation) can run the layer.
//
// Each GPU the library runs on holds its own copy of `scratch` until the
// process ends.  Every call on one GPU shares that copy and leaves the last
// call's contents in it; calls that overlap on one GPU (two streams, or two
// host threads) race.  Nothing in the layer reads scratch before writing it,
// so no clearing is needed between calls.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/mosaic_amd.h"
#include "common.h"

namespace {

constexpr size_t kScratchBytes = size_t(8) << 20;  // covers M <= 16 at hidden 7168, inter 2048, 256 experts, top-8
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct DeviceScratch {
  std::once_flag once;
  hipError_t status = hipSuccess;
  void* ptr = nullptr;
};
DeviceScratch g_scratch[kMaxDevices];

// The device address of this device's `scratch`, looked up once per device
// with that device current.  In host code the array's name is only a
// host-side stand-in, never a device address.
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    mosaic::set_last_error("moe_a16_forward_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  MOSAIC_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "moe_a16_forward_noalloc: device %d >= %d", dev, kMaxDevices);
  DeviceScratch& d = g_scratch[dev];
  std::call_once(d.once, [&d]() {
    void* p = nullptr;
    d.status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (d.status == hipSuccess) d.ptr = p;
  });
  if (d.status != hipSuccess || d.ptr == nullptr) {
    const hipError_t f = d.status != hipSuccess ? d.status : hipErrorInvalidSymbol;
    mosaic::set_last_error("moe_a16_forward_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                           hipGetErrorString(f));
    return (int)f;
  }
  *out = d.ptr;
  return mosaic::kOk;
}

}  // namespace

extern "C" size_t mosaic_moe_a16_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int mosaic_moe_a16_forward_noalloc(const uint16_t* x, const float* logits, int32_t* ids, float* weights,
                                              const uint8_t* gu_packed, const uint8_t* gu_scale,
                                              const uint8_t* d_packed, const uint8_t* d_scale,
                                              const uint8_t* sh_gu_packed, const uint8_t* sh_gu_scale,
                                              const uint8_t* sh_d_packed, const uint8_t* sh_d_scale, uint16_t* y,
                                              int64_t m, int64_t hidden, int64_t inter, int64_t n_experts,
                                              int64_t top_k, int score_func, int renorm, float route_scale,
                                              const float* route_bias, float swiglu_limit, void* stream) {
  MOSAIC_CHECK_ARG(m >= 1 && hidden > 0 && inter > 0 && n_experts > 0 && top_k > 0,
                   "moe_a16_forward_noalloc: bad shape");
  const size_t need = mosaic_moe_a16_workspace_bytes(m, hidden, inter, n_experts, top_k, sh_gu_packed != nullptr);
  MOSAIC_CHECK_ARG(need <= kScratchBytes,
                   "moe_a16_forward_noalloc: this shape needs %zu scratch bytes, more than the %zu-byte static "
                   "scratch (use mosaic_moe_a16_forward with a workspace)",
                   need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc != mosaic::kOk) return rc;
  return mosaic_moe_a16_forward(x, logits, ids, weights, gu_packed, gu_scale, d_packed, d_scale, sh_gu_packed,
                                sh_gu_scale, sh_d_packed, sh_d_scale, y, m, hidden, inter, n_experts, top_k, score_func,
                                renorm, route_scale, route_bias, swiglu_limit, ws, kScratchBytes, nullptr, stream);
}
