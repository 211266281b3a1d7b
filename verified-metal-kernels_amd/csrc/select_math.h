// Bin arithmetic of the DSA top-2048 select, compiled for the device (the select kernels) and for the host
// (vmk_debug_select_threshold, which replays it on a histogram from a CPU test).  Every index it returns lies inside
// the histogram it was given, whatever the counts hold: an empty histogram, or fine counts that disagree with the
// coarse ones, give a valid (if meaningless) bin rather than an address outside the histogram.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vmk {

constexpr int kSelBins = 8192;   // fine histogram: fkey >> 19
constexpr int kSelCBins = 256;   // coarse histogram: fkey >> 24, 32 fine bins each

struct Threshold {
  uint32_t bin;   // bin holding the need-th largest element
  uint32_t rest;  // need minus the elements in higher bins
};

// One thread's share of the threshold search over hist[lo, lo + per), with `above` elements in the bins above lo +
// per - 1 (an exclusive scan from the top over the threads' ranges).  Sets *t and returns true when the need-th
// largest element lies in this range; at most one thread of a consistent scan returns true.
__host__ __device__ inline bool threshold_in_range(const uint32_t* hist, int lo, int per, uint32_t above,
                                                   uint32_t need, Threshold* t) {
  uint32_t acc = above;
  for (int i = per - 1; i >= 0; --i) {
    const uint32_t c = hist[lo + i];
    if (acc < need && acc + c >= need) {
      t->bin = (uint32_t)(lo + i);
      t->rest = need - acc;
      return true;
    }
    acc += c;
  }
  return false;
}

// First bin of thread `tid`'s range when nt threads share nbins bins, highest bins first (thread 0 owns the top).
__host__ __device__ inline int threshold_range_lo(int tid, int nt, int per) { return (nt - 1 - tid) * per; }

// The coarse bin a fine lookup may use: a coarse result out of range (possible only from inconsistent counts) is
// clamped to the last coarse bin, so the 32 fine bins read are inside the fine histogram.
__host__ __device__ inline uint32_t coarse_bin_clamped(uint32_t coarse) {
  return coarse < (uint32_t)kSelCBins ? coarse : (uint32_t)kSelCBins - 1;
}

// Fine bin 31 - lane of a coarse bin holds the rest-th element of that coarse bin when the inclusive count from the
// top (`incl`, fine bins 31 .. 31 - lane) reaches rest and the exclusive one does not.
__host__ __device__ inline bool fine_hit(uint32_t incl, uint32_t v, uint32_t rest) {
  return incl >= rest && incl - v < rest;
}

__host__ __device__ inline uint32_t fine_bin(uint32_t coarse, int lane) {
  return coarse_bin_clamped(coarse) * 32 + 31 - (uint32_t)lane;
}

}  // namespace vmk
