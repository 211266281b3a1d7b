// Library-wide C-ABI: version and last-error reporting.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include "vmk_internal.h"

namespace vmk {
static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
}  // namespace vmk

extern "C" const char* vmk_last_error(void) { return vmk::g_err; }

// Measurement hook: the next launch of kernel `kernel_id` (vmk::KernelId) on this host thread is bracketed by
// hipEventRecord(before) / hipEventRecord(after) on the stream it is launched on; the request is then cleared.
namespace vmk {
static thread_local hipEvent_t g_prof_before = nullptr, g_prof_after = nullptr;
static thread_local int g_prof_kernel = -1;

void prof_before(int kernel_id, hipStream_t s) {
  if (g_prof_kernel == kernel_id && g_prof_before) (void)hipEventRecord(g_prof_before, s);
}

void prof_after(int kernel_id, hipStream_t s) {
  if (g_prof_kernel == kernel_id && g_prof_after) {
    (void)hipEventRecord(g_prof_after, s);
    g_prof_kernel = -1;
    g_prof_before = g_prof_after = nullptr;
  }
}
}  // namespace vmk

extern "C" int vmk_profile_next(void* before, void* after, int kernel_id) {
  vmk::g_prof_before = (hipEvent_t)before;
  vmk::g_prof_after = (hipEvent_t)after;
  vmk::g_prof_kernel = kernel_id;
  return 0;
}

extern "C" int vmk_version(void) { return 1; }

// Architecture check: 0 when the current device is gfx950, 1 otherwise (message in vmk_last_error).
extern "C" int vmk_check_device(void) {
  int dev = 0;
  VMK_CHECK_HIP(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  VMK_CHECK_HIP(hipGetDeviceProperties(&prop, dev));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    vmk::set_error("vmk_check_device: libvmk is built for gfx950, device %d is %s", dev, prop.gcnArchName);
    return 1;
  }
  return 0;
}

// Lane-layout check of the 32x32x16 fp16 MFMA used by every attention kernel: one wave, D = A . B with
// A, B given per lane (64 lanes x 8 halfs each) and D returned per lane (64 lanes x 16 floats).
#include "vmk_common.h"
__global__ __launch_bounds__(64) void debug_mfma32_kernel(const vmk::half8* a, const vmk::half8* b, float* d) {
  const int l = threadIdx.x;
  vmk::floatx16 acc = vmk::floatx16{};
  acc = vmk::mfma32(a[l], b[l], acc);
  for (int i = 0; i < 16; ++i) d[l * 16 + i] = acc[i];
}

extern "C" int vmk_debug_mfma32(const void* a, const void* b, void* d, void* stream) {
  VMK_CHECK(a && b && d, "null pointer argument");
  hipLaunchKernelGGL(debug_mfma32_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (const vmk::half8*)a,
                     (const vmk::half8*)b, (float*)d);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

// Stage dump of the attention wave pipeline for one full 32-key tile (test hook): q (32 x 128), k/v (32 x 128)
// fp16 -> s (64 lanes x 16, raw S^T), vt (128 x 36 halfs, the LDS tile), o (64 lanes x 64, O^T after one tile,
// unnormalised), ml (64 lanes x 2).
#include "attn_core.h"
__global__ __launch_bounds__(64) void debug_tile_kernel(const vmk::f16* q, const vmk::f16* k, const vmk::f16* v,
                                                        float* s_out, vmk::f16* vt_out, float* o_out, float* ml,
                                                        float sl2) {
  using namespace vmk;
  __shared__ __attribute__((aligned(16))) f16 vt[kVTileHalfs];
  const int lane = threadIdx.x, r = lane & 31, g = lane >> 5, dc = lane & 15, kg = lane >> 4;
  half8 qb[8];
  load_qt(qb, q + r * 128, g, true);
  u32x4 kr[8], vr[8];
  load_k(kr, k + r * 128, g);
  load_v(vr, [&](int j) -> const f16* { return v + (kg * 8 + j) * 128; }, [](int) { return true; }, dc);
  store_vt(vt, vr, dc, kg);
  floatx16 s = qk_tile(kr, qb);
  for (int i = 0; i < 16; ++i) s_out[lane * 16 + i] = s[i];
  for (int i = 0; i < 16; ++i) s[i] *= sl2;
  RowState st;
  row_state_init(st);
  half8 pb[2];
  softmax_update(st, s, 1.f, pb);
  pv_tile(st, vt, pb, lane);
  for (int dt = 0; dt < 4; ++dt)
    for (int i = 0; i < 16; ++i) o_out[lane * 64 + dt * 16 + i] = st.o[dt][i];
  ml[lane * 2] = st.m;
  ml[lane * 2 + 1] = st.l;
  __syncthreads();
  for (int i = lane; i < kVTileHalfs; i += 64) vt_out[i] = vt[i];
}

extern "C" int vmk_debug_tile(const void* q, const void* k, const void* v, void* s, void* vt, void* o, void* ml,
                              float sl2, void* stream) {
  hipLaunchKernelGGL(debug_tile_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (const vmk::f16*)q,
                     (const vmk::f16*)k, (const vmk::f16*)v, (float*)s, (vmk::f16*)vt, (float*)o, (float*)ml, sl2);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}
