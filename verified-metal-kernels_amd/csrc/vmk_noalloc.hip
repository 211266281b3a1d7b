// The allocation-free spec entry point (vmk_spec_verify_noalloc) and its static scratch.  No counterpart in the
// reference: it is for callers that cannot allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc).  This file holds no kernel: the scratch is its code object's only device
// content, so the HIP runtime loads it onto a device, and allocates the scratch there, when the first call on that
// device looks the scratch up, not when the library's other kernels load.
//
// vmk_spec_verify without a workspace argument.  The partials go to `scratch`, a file-scope device array that every
// GPU the entry point has run on holds until the process ends.  Host code never passes the array's name to a kernel
// (on the host it is only a stand-in for the symbol): the device address comes from hipGetSymbolAddress, looked up
// once per device with that device current, and kept per device.  Every call on one GPU uses that GPU's one array,
// so calls that overlap on a GPU (two streams, two host threads) race; the array keeps the last call's partials, and
// no part of it must start at zero (every partial the combine reads is written first).
#include "vmk_internal.h"

#include <mutex>

namespace vmk {
constexpr size_t kScratchBytes = (size_t)32 << 20;   // fp16 partials of every bench shape (C4: 16.5 MiB)
constexpr int kScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static void* g_scratch_ptr[kScratchDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the device that `stream` belongs to (the current device for the null stream),
// looked up on the first call on that device with that device made current, and kept per device; 0 on success.
static int scratch_address(hipStream_t stream, void** ptr) {
  int dev = -1;
  if (stream) {
    VMK_CHECK_HIP(hipStreamGetDevice(stream, &dev));
  } else {
    VMK_CHECK_HIP(hipGetDevice(&dev));
  }
  VMK_CHECK(dev >= 0 && dev < kScratchDevices, "device index beyond the per-device scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    VMK_CHECK_HIP(hipGetDevice(&cur));
    if (cur != dev) VMK_CHECK_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) VMK_CHECK_HIP(hipSetDevice(cur));
    VMK_CHECK_HIP(e);
    VMK_CHECK(p != nullptr && ((uintptr_t)p & 255u) == 0, "scratch symbol address missing or misaligned");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return 0;
}
}  // namespace vmk

extern "C" size_t vmk_spec_noalloc_max_bytes(void) { return vmk::kScratchBytes; }

extern "C" int vmk_spec_verify_noalloc(const void* q, const void* k, const void* v, const void* mask_words, void* out,
                                       int64_t B, int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L,
                                       int64_t W, void* stream) {
  using namespace vmk;
  // Every check comes before the first HIP call: a rejected call touches no device.
  size_t need = 0;
  if (int rc = spec_noalloc_need(q, k, v, mask_words, out, B, kd, Hq, Hkv, D, L, W, &need)) return rc;
  if (need > kScratchBytes) {
    set_error("vmk_spec_verify_noalloc: this shape needs %zu bytes of partials, more than the %zu bytes of static "
              "scratch; call vmk_spec_verify with a workspace instead", need, kScratchBytes);
    return 1;
  }
  void* partials = nullptr;
  if (int rc = scratch_address((hipStream_t)stream, &partials)) return rc;
  return spec_noalloc_launch(q, k, v, mask_words, out, B, kd, Hq, Hkv, L, W, partials, (hipStream_t)stream);
}
