// Allocation-free backward: ca_bwd_f32 with its workspace in a static device
// array instead of a caller-allocated buffer, for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// The array lives in this translation unit only, so only processes that call
// this entry point have its code object (and the array) loaded on a device.
// Each device holds its own copy at its own address: the address is looked up
// with hipGetSymbolAddress once per device, with that device current, and
// only that address (never the array's name, which in host code is a
// host-side stand-in) is handed to the kernels.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "../../include/continuum_attention_amd.h"
#include "ca_kernels.h"

namespace {

constexpr size_t kScratchBytes = size_t(CA_NOALLOC_SCRATCH_MB) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's copy of `scratch` (nullptr and an error text on failure).
void* device_scratch(int* rc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *rc = ca::set_error(CA_ERR_HIP, "ca_bwd_f32_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = ca::set_error(CA_ERR_UNSUPPORTED, "ca_bwd_f32_noalloc: device %d beyond %d", dev, kMaxDevices);
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *rc = ca::set_error(CA_ERR_HIP, "ca_bwd_f32_noalloc: hipGetSymbolAddress(scratch): %s",
                          hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace

extern "C" int ca_bwd_f32_noalloc(const float* q, const float* k, const float* v,
                                  const float* log_gain, const float* out, const float* stats,
                                  const float* dout, float* dq, float* dk, float* dv,
                                  float* dlog_gain, int B, int H, int T, int D, void* stream) {
  const int rc0 = ca::check_shape(B, H, T, D);
  if (rc0) return rc0;
  // the backward runs in passes over query-group ranges (of every slice, or
  // of sets of heads) sized to the array; a shape whose single 128-query
  // group of one slice needs more is refused
  if (!ca::bwd_fits(B, H, T, D, kScratchBytes))
    return ca::set_error(CA_ERR_WORKSPACE,
                         "ca_bwd_f32_noalloc: one 128-query pass of this shape needs more than the "
                         "static %zu bytes of scratch (B=%d H=%d T=%d D=%d); use ca_bwd_f32 with "
                         "a workspace", kScratchBytes, B, H, T, D);
  // Every kernel of the backward writes each scratch element before it reads
  // it, so nothing needs clearing between calls.
  int rc = CA_OK;
  void* ws = device_scratch(&rc);
  if (!ws) return rc;
  return ca_bwd_f32(q, k, v, log_gain, out, stats, dout, dq, dk, dv, dlog_gain, ws, kScratchBytes,
                    B, H, T, D, stream);
}
