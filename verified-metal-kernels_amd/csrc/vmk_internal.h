// Host-side helpers of the C-ABI entry points: argument checks and the last-error string.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <algorithm>

namespace vmk {
void set_error(const char* fmt, ...);

// Kernel ids of the measurement hook (vmk_profile_next).
enum KernelId {
  kKSpecPartial = 0, kKSpecCombine = 1, kKPrefixPartial = 2, kKPrefixCombine = 3,
  kKDsaIndexer = 4, kKDsaSelect = 5, kKDsaAttn = 6, kKDsaCombine = 7, kKDsaSelectScan = 8,
  kKDsaProjectQ = 9, kKDsaSingle = 10,
};
void prof_before(int kernel_id, hipStream_t s);
void prof_after(int kernel_id, hipStream_t s);

// Every workspace starts with a head of kWsHead bytes that must be zero before the first call and that every call
// leaves zero again (histograms and counters that kernels accumulate into); data regions follow it.
// Layout of the head: [0, 2 MiB) histograms, [2 MiB, 4 MiB) counters.
constexpr size_t kWsHead = (size_t)4 << 20;
constexpr size_t kWsCounters = (size_t)2 << 20;
// The spec half of the allocation-free entry point (vmk_spec.hip): argument checks and the bytes of partials a shape
// needs (no HIP call), then the launches with the partials at `partials`.
int spec_noalloc_need(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                      int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W, size_t* need);
int spec_noalloc_launch(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                        int64_t kd, int64_t Hq, int64_t Hkv, int64_t L, int64_t W, void* partials, hipStream_t s);
// Compute units of the target GPU (MI355X): plans size their grids to one dispatch round of one workgroup per CU.
constexpr int kDeviceCUs = 256;
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline void* align_up(void* p, size_t a) { return (void*)(((uintptr_t)p + a - 1) & ~(uintptr_t)(a - 1)); }
}  // namespace vmk

// Returns 1 from the entry point with a message when a host-side precondition fails (nothing is launched).
#define VMK_CHECK(cond, msg)                                                   \
  do {                                                                         \
    if (!(cond)) {                                                             \
      ::vmk::set_error("%s: %s", __func__, msg);                               \
      return 1;                                                                \
    }                                                                          \
  } while (0)

// Returns 2 with the HIP error string when a launch or runtime call fails.
#define VMK_CHECK_HIP(expr)                                                    \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      ::vmk::set_error("%s: %s (%s)", __func__, hipGetErrorString(e_), #expr); \
      return 2;                                                                \
    }                                                                          \
  } while (0)
