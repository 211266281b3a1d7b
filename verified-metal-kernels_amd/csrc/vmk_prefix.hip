// Shared-prefix decode on gfx950 (cascade attention).
//
// Replaces the reference's shpfx_main (prefix and suffix block roles) and shpfx_combine Metal kernels
// (kernels/prefix_opus55_v8.py:28-108, 109-208, 211-261) behind the kernel(q, kp, vp, ks, vs) contract of
// ops/prefix.py:1-4, plus optional ragged suffix lengths.
//
// Launch 1 (prefix_rows_kernel): items (KV head h, row block of 32*NW of the N*G rows, prefix chunk) stream the chunk
//   once through an LDS ring shared by NW waves of 32 rows each, so the prefix is read from HBM once per row block
//   instead of once per request.
// Launch 2 (prefix_partial_kernel): items (request n, KV head h, suffix chunk) attend the G rows of request n to its
//   own suffix rows.  When a suffix is one chunk, the item also merges the finished prefix partials of its rows and
//   writes the output.
// Launch 3 (prefix_combine_kernel, only when a suffix spans several chunks or there is no prefix): per output row,
//   the log-sum-exp merge of its prefix and suffix partials.
// With at most 128 rows per KV head, launches 1 and 2 are one grid (prefix_mixed_kernel; with at most 32 rows and
// more items than CUs, its prefix items are single-wave units packed 2 or 4 per workgroup).  Its whole-suffix items
// wait for their KV head's prefix partials and merge them in the same launch when G <= 4 and there are at most 32
// prefix chunks (mfuse below); otherwise prefix_merge_kernel does the whole-suffix merges.
#include "attn_core.h"
#include "vmk_internal.h"

namespace vmk {

struct PrefixArgs {
  const f16* q;            // (N, Hq, 128)
  const f16* kp;           // (Hkv, P, 128); paged: the K page pool (num_pages, Hkv, ps, 128)
  const f16* vp;           // paged: the V page pool
  const f16* ks;           // (N, Hkv, S, 128); paged: unused
  const f16* vs;
  const int* prefix_pages; // paged: (P / ps,) page ids of the shared prefix
  const int* suffix_pages; // paged: (N, max_sp) page ids of each request's suffix (S = max_sp * ps)
  int ps, max_sp, num_pages;
  const int* slens;        // (N,) or null
  f16* out;                // (N, Hq, 128)
  void* po_p;              // prefix partials [h][rb][split][32*WRp][128], normalised O of type part_t
  float* pml_p;
  void* po_s;              // suffix partials [n][h][split][32][128]
  float* pml_s;
  int N, Hq, Hkv, G, P, S;
  int WRp, nrb_p, nsplit_p, chunk_p;   // prefix plan
  int nsplit_s, chunk_s;                    // suffix plan (WR = 1, WK = 4)
  int n_prefix_items;
  int2* order;             // (N,) (request, suffix length) by decreasing length (written by the prefix launch), or null
  int fuse;                // 1: suffix items are whole suffixes and merge the (finished) prefix partials themselves
  int merge;               // 1: whole-suffix partials are merged with the prefix partials by prefix_merge_kernel
  int units;               // mixed launch, N*G <= 32: prefix units (one wave each) per workgroup; 0: row blocks
  int mfuse;               // 1: mixed launch whose whole-suffix items wait for their KV head's prefix partials and
                           //    merge them themselves (no merge launch)
  uint32_t* sync;          // mfuse: the sticky timeout flag, then per KV head the prefix arrivals and the finished
                           //        suffix items (workspace head, zero between calls)
  int sfx_delay;           // mixed launch: s_sleep(16) rounds before a suffix item's walk (0: none)
  float sl2;
};

// The in-kernel merge of a mixed launch (mfuse).  Prefix producers store their partials with agent-coherent stores
// and, once every wave's stores have completed (the workgroup barrier waits for them), add 1 to their KV head's
// arrival counter.  A whole-suffix item keeps its partial in LDS, waits until the arrivals of its head reach the
// head's producer count (nrb_p * nsplit_p), then fetches the prefix rows with agent-coherent loads and merges them
// with the functions the fused suffix items of the two-launch path use, on the same values, so the output bits are
// those of the merge launch.  The last suffix item of a head returns both of its counters to zero.  The wait is
// safe from deadlock: the producers never wait and come first in the grid, so each XCD dispatches them before any
// suffix item.  It is still bounded: after kPrefixSpinLimit polls the item sets the sticky flag and writes NaN rows,
// and every later mixed launch on that workspace sees the flag and writes NaN rows at once, until its head is zeroed.
// Layout, in the counter part of the workspace head (clear of the DSA histograms and barrier lines): the flag, then
// 128 bytes per KV head (arrivals, then 64 bytes on, finished suffix items).
constexpr size_t kPrefixSync = kWsCounters + ((size_t)3 << 19);
constexpr int kPrefixSyncHeads = (int)((((size_t)1 << 19) - 256) / 128);
constexpr uint32_t kPrefixSpinLimit = 1u << 20;
__device__ __forceinline__ uint32_t* pfx_arrivals(const PrefixArgs& a, int h) { return a.sync + 64 + 32 * h; }
__device__ __forceinline__ uint32_t* pfx_finished(const PrefixArgs& a, int h) { return a.sync + 64 + 32 * h + 16; }
__device__ __forceinline__ uint32_t ld_coherent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool pfx_poisoned(const PrefixArgs& a) { return ld_coherent(a.sync) != 0; }

// A prefix producer of KV head h has stored its partial: every wave of the workgroup (kWave: only the calling wave,
// a unit) waits until its stores have completed, then one lane counts the arrival.
template <bool kWave>
__device__ __forceinline__ void pfx_arrive(const PrefixArgs& a, int h) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (!kWave) __syncthreads();
  if ((kWave ? (threadIdx.x & 63) : threadIdx.x) == 0)
    __hip_atomic_fetch_add(pfx_arrivals(a, h), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0 of a suffix item: waits for the prefix partials of KV head h; false when it gave up or the flag is set
// (poisoned: the flag as read when the item started).
__device__ __forceinline__ bool pfx_wait(const PrefixArgs& a, int h, bool poisoned) {
  if (poisoned) return false;
  const uint32_t need = (uint32_t)(a.nrb_p * a.nsplit_p);
  for (uint32_t spin = 0;; ++spin) {
    if (ld_coherent(pfx_arrivals(a, h)) >= need) return true;
    if ((spin & 31) == 31 && pfx_poisoned(a)) return false;
    if (spin >= kPrefixSpinLimit) {
      __hip_atomic_fetch_or(a.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

struct RangeSrc {
  const f16* kbase;
  const f16* vbase;
  int kend;
  float scale;
  static constexpr bool kStrided = false;   // rows 256 bytes apart
  __device__ const f16* ktile(int key0) const { return kbase + (size_t)key0 * 128; }
  __device__ const f16* vtile(int key0) const { return vbase + (size_t)key0 * 128; }
  __device__ void mask(floatx16& s, int key0, int g) const {
    if (key0 + kTile <= kend) return;                      // whole tile inside (same for the whole wave)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key = key0 + 8 * blk + 4 * g + c;
        s[4 * blk + c] = key < kend ? s[4 * blk + c] : kNegInf;
      }
  }
};

template <bool kNHD>
__device__ __forceinline__ PagedSrc<kNHD> paged_src(const PrefixArgs& a, const int* table, int ntable, int h,
                                                    int kbeg, int kend) {
  return paged_src<kNHD>(a.kp, a.vp, a.ps, a.Hkv, a.num_pages, a.sl2, table, ntable, h, kbeg, kend);
}

// Suffix length of request n, clamped to [0, S] so that a bad length can never read past its own rows.
__device__ __forceinline__ int suffix_len(const PrefixArgs& a, int n) {
  return a.slens ? min(max(a.slens[n], 0), a.S) : a.S;
}

// LDS offset of a fused suffix item's partial: past attend_wg's cross-wave merge slots; its (m, l) pairs follow 16 KB
// further (room for 32 rows of 128 floats).
constexpr int kFuseOff = kAttnSlotsEnd;
constexpr int kFuseMlOff = kFuseOff + 32 * 128 * 4;
static_assert(kFuseMlOff + 64 * 4 <= kAttnSmemBytes, "fused partial must fit in the stage memory");

template <class PT> __device__ __forceinline__ const PT* prefix_po(const PrefixArgs& a) {
  return reinterpret_cast<const PT*>(a.po_p);
}

// Final output of request n's G rows of KV head h: log-sum-exp merge of the suffix partial (lpo: normalised rows of
// 128, lpml (m, l) pairs) with the prefix partials of those rows, each weighted exp2(m - M) * l.  One wave per row, two head-dims per lane.
// Lane s holds the (m, l) of prefix partial b0 + s; the O rows are fetched 16 partials at a time with independent
// loads (one memory round trip per 16), weighted with the lane-broadcast weights.
template <class E>
__device__ void merge_prefix_rows(const PrefixArgs& a, const part_t<E>* lpo, const float* lpml, int n, int h) {
  typedef part_t<E> PT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int np = a.P > 0 ? a.nsplit_p : 0;
  const int rows_p = 32 * a.WRp;
  for (int gg = wave; gg < a.G; gg += 4) {
    const int prow = n * a.G + gg, rb = prow / rows_p, rl = prow % rows_p;
    const size_t pbase = ((size_t)h * a.nrb_p + rb) * a.nsplit_p * rows_p + rl;   // partial s at pbase + s*rows_p
    const float ms = lpml[2 * gg], ls = lpml[2 * gg + 1];
    float M = ms;
    for (int s0 = lane; s0 < np; s0 += 64) M = fmaxf(M, a.pml_p[(pbase + (size_t)s0 * rows_p) * 2]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    const float Mu = (M == kNegInf) ? 0.f : M;
    const float ws = fast_exp2(ms - Mu) * ls;              // weights exp2(m - M) * l of the normalised partials
    float den = 0.f;                                       // this lane's share of the prefix denominators
    float2 num = load_part2(lpo + gg * 128 + 2 * lane);
    num.x *= ws;
    num.y *= ws;
    for (int b0 = 0; b0 < np; b0 += 64) {
      float w = 0.f;
      if (b0 + lane < np) {
        const float2 ml = *reinterpret_cast<const float2*>(a.pml_p + (pbase + (size_t)(b0 + lane) * rows_p) * 2);
        w = fast_exp2(ml.x - Mu) * ml.y;
        den += w;
      }
      const int nb = min(64, np - b0);
      for (int j0 = 0; j0 < nb; j0 += 16) {
        float2 v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int j = b0 + min(j0 + k, nb - 1);          // clamped: in bounds; weight 0 past nb
          v[k] = load_part2(prefix_po<PT>(a) + (pbase + (size_t)j * rows_p) * 128 + 2 * lane);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const float wb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), (j0 + k) & 63));
          const float wj = j0 + k < nb ? wb : 0.f;
          num.x += wj * v[k].x;
          num.y += wj * v[k].y;
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
    den += ws;
    E* out = reinterpret_cast<E*>(a.out) + ((size_t)n * a.Hq + h * a.G + gg) * 128 + 2 * lane;
    out[0] = (E)(num.x / den);
    out[1] = (E)(num.y / den);
  }
}

// Prefix partials of one output row held in registers: lane s has (m, l) of split s, and v[j] the lane's two
// head-dims of split j's O row.  Fetched before a fused suffix item's walk (the prefix launch has finished), so the
// final merge needs no memory round trip.
constexpr int kPrefetchSplits = 32;
struct PrefixRow {
  float2 ml;
  float2 v[kPrefetchSplits];
};

template <class PT, bool kCoherent = false>
__device__ __forceinline__ void prefetch_prefix_row(const PrefixArgs& a, PrefixRow& pr, int n, int h, int gg,
                                                    int lane) {
  const int np = a.nsplit_p, rows_p = 32 * a.WRp;
  const int prow = n * a.G + gg, rb = prow / rows_p, rl = prow % rows_p;
  const size_t pbase = ((size_t)h * a.nrb_p + rb) * a.nsplit_p * rows_p + rl;
  const float* mlp = a.pml_p + (pbase + (size_t)min(lane, np - 1) * rows_p) * 2;
  pr.ml = kCoherent ? load_part2_coherent(mlp) : *reinterpret_cast<const float2*>(mlp);
#pragma unroll
  for (int j = 0; j < kPrefetchSplits; ++j) {
    const PT* vp = prefix_po<PT>(a) + (pbase + (size_t)min(j, np - 1) * rows_p) * 128 + 2 * lane;
    pr.v[j] = kCoherent ? load_part2_coherent(vp) : load_part2(vp);
  }
}

// Final output of row gg of request n, KV head h, from the suffix partial in LDS and the prefetched prefix row.
template <class E>
__device__ __forceinline__ void merge_prefetched_row(const PrefixArgs& a, const PrefixRow& pr, const part_t<E>* lpo,
                                                     const float* lpml, int n, int h, int gg, int lane) {
  const int np = a.nsplit_p;
  const float ms = lpml[2 * gg], ls = lpml[2 * gg + 1];
  const float M = wave_max(lane < np ? fmaxf(ms, pr.ml.x) : ms);
  const float Mu = (M == kNegInf) ? 0.f : M;
  const float ws = fast_exp2(ms - Mu) * ls;                // weights exp2(m - M) * l of the normalised partials
  const float w = lane < np ? fast_exp2(pr.ml.x - Mu) * pr.ml.y : 0.f;
  float den = w;
  float2 num = load_part2(lpo + gg * 128 + 2 * lane);
  num.x *= ws;
  num.y *= ws;
#pragma unroll
  for (int j = 0; j < kPrefetchSplits; ++j) {
    const float wj = j < np ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j)) : 0.f;
    num.x += wj * pr.v[j].x;
    num.y += wj * pr.v[j].y;
  }
  den = wave_sum(den) + ws;
  E* out = reinterpret_cast<E*>(a.out) + ((size_t)n * a.Hq + h * a.G + gg) * 128 + 2 * lane;
  out[0] = (E)(num.x / den);
  out[1] = (E)(num.y / den);
}

// Row gg of request n, KV head h, as NaN (the mixed launch's merge gave up: the workspace's flag is set).
template <class E>
__device__ __forceinline__ void pfx_nan_row(const PrefixArgs& a, int n, int h, int gg, int lane) {
  E* out = reinterpret_cast<E*>(a.out) + ((size_t)n * a.Hq + h * a.G + gg) * 128 + 2 * lane;
  out[0] = (E)__builtin_nanf("");
  out[1] = (E)__builtin_nanf("");
}

// A suffix item of KV head h is done with its head's counters; the last of the head's N items clears them.
__device__ __forceinline__ void pfx_finish(const PrefixArgs& a, int h) {
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(pfx_finished(a, h), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (uint32_t)(a.N * a.nsplit_s) - 1) {
      __hip_atomic_store(pfx_arrivals(a, h), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(pfx_finished(a, h), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The walk and merge of a suffix item over key source src (keys [kbeg, src.kend)).
template <class V, class Src>
__device__ __forceinline__ void suffix_walk(const PrefixArgs& a, char* smem, const Src& src, int n, int h, int nh,
                                            int split, int kbeg) {
  const int ntiles = max(0, (src.kend - kbeg + kTile - 1) / kTile);
  auto qrow = [&](int r) { return a.q + ((size_t)n * a.Hq + h * a.G + r) * 128; };
  typedef part_t<elem_t<V>> PT;
  if (!a.fuse && !a.mfuse) {
    const size_t pi = (size_t)nh * a.nsplit_s + split;
    attend_wg<1, 4, 2, V>(smem, src, qrow, a.G, kbeg, ntiles, reinterpret_cast<PT*>(a.po_s) + pi * 32 * 128,
                          a.pml_s + pi * 32 * 2);
    return;
  }
  // Whole suffix: keep the partial in LDS (past the merge slots) and merge it with the prefix partials here.
  PT* lpo = reinterpret_cast<PT*>(smem + kFuseOff);
  float* lpml = reinterpret_cast<float*>(smem + kFuseMlOff);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (a.mfuse) {                                            // mixed launch: the prefix partials arrive meanwhile
    __shared__ int ready;
    const bool poisoned = threadIdx.x == 0 && pfx_poisoned(a);   // read now, used after the walk
    attend_wg<1, 4, 2, V>(smem, src, qrow, a.G, kbeg, ntiles, lpo, lpml);
    if (threadIdx.x == 0) ready = pfx_wait(a, h, poisoned);
    __syncthreads();                                        // the partial in LDS, and the wait's outcome
    if (wave < a.G) {
      if (ready) {
        PrefixRow pr;
        prefetch_prefix_row<PT, true>(a, pr, n, h, wave, lane);
        merge_prefetched_row<elem_t<V>>(a, pr, lpo, lpml, n, h, wave, lane);
      } else {
        pfx_nan_row<elem_t<V>>(a, n, h, wave, lane);
      }
    }
    pfx_finish(a, h);
    return;
  }
  if (a.G <= 4 && a.nsplit_p <= kPrefetchSplits) {          // wave w finishes row w
    PrefixRow pr;
    if (wave < a.G) prefetch_prefix_row<PT>(a, pr, n, h, wave, lane);
    attend_wg<1, 4, 2, V>(smem, src, qrow, a.G, kbeg, ntiles, lpo, lpml);
    __syncthreads();
    if (wave < a.G) merge_prefetched_row<elem_t<V>>(a, pr, lpo, lpml, n, h, wave, lane);
  } else {
    attend_wg<1, 4, 2, V>(smem, src, qrow, a.G, kbeg, ntiles, lpo, lpml);
    __syncthreads();
    merge_prefix_rows<elem_t<V>>(a, lpo, lpml, n, h);
  }
}

// The kernels' key source, a template argument: contiguous caches, or a page pool in the HND or NHD layout.
constexpr int kContig = 0, kPagedHND = 1, kPagedNHD = 2;

// Suffix item `sitem` (request, KV head, suffix chunk) of 4 waves.  Fused: the prefix partials are finished (an
// earlier launch) and the item writes its rows' outputs; otherwise it writes its partial to po_s / pml_s.
template <int kPaged, class V>
__device__ __forceinline__ void suffix_item(const PrefixArgs& a, char* smem, int sitem) {
  const int split = sitem % a.nsplit_s;
  int nh = sitem / a.nsplit_s, sn = 0;
  if (a.order) {                                        // long suffixes are dispatched first
    const int2 o = a.order[nh / a.Hkv];
    nh = o.x * a.Hkv + nh % a.Hkv;
    sn = o.y;
  }
  const int n = nh / a.Hkv, h = nh % a.Hkv;
  const int kbeg = split * a.chunk_s;
  if (!a.order) sn = suffix_len(a, n);
  if (kbeg >= sn && !a.fuse && !a.merge && !a.mfuse) return;   // whole workgroup: nothing of this suffix is here
  // A mixed launch's suffix items start their loads after the prefix items' first tiles have been requested, when
  // they have the slack (the prefix items are the launch's critical path).
  for (int i = 0; i < a.sfx_delay; ++i) __builtin_amdgcn_s_sleep(16);
  const int kend = min(sn, kbeg + a.chunk_s);
  if constexpr (kPaged != kContig) {
    const int* table = a.suffix_pages + (size_t)n * a.max_sp;
    suffix_walk<V>(a, smem, paged_src<kPaged == kPagedNHD>(a, table, a.max_sp, h, kbeg, kend), n, h, nh, split, kbeg);
  } else {
    RangeSrc src;
    src.scale = a.sl2;
    const size_t off = ((size_t)n * a.Hkv + h) * a.S * 128;
    src.kbase = a.ks + off;
    src.vbase = a.vs + off;
    src.kend = kend;
    suffix_walk<V>(a, smem, src, n, h, nh, split, kbeg);
  }
}


// Suffix items, after the prefix launch has written the prefix partials.
template <int kPaged, class V>
__global__ __launch_bounds__(256) void prefix_partial_kernel(PrefixArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kAttnSmemBytes];
  suffix_item<kPaged, V>(a, smem, blockIdx.x);
}

// Counting sort of the requests by decreasing suffix length (256 buckets), run by one workgroup of the prefix
// launch so the suffix launch can dispatch its longest items first.  Only the schedule depends on it: every item
// computes the same values whatever order it runs in.
template <int NT>
__device__ void build_suffix_order(const PrefixArgs& a, uint32_t* cnt /* LDS, 256 */) {
  const int tid = threadIdx.x;
  const int bw = a.S / 256 + 1;
  for (int i = tid; i < 256; i += NT) cnt[i] = 0;
  __syncthreads();
  for (int n = tid; n < a.N; n += NT) atomicAdd(&cnt[255 - suffix_len(a, n) / bw], 1u);
  __syncthreads();
  if (tid < 64) {                                          // exclusive scan, 4 buckets per lane
    uint32_t c[4], t = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) { c[k] = cnt[4 * tid + k]; t += c[k]; }
    uint32_t x = t;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(x, o, 64);
      if (tid >= o) x += y;
    }
    uint32_t run = x - t;
#pragma unroll
    for (int k = 0; k < 4; ++k) { cnt[4 * tid + k] = run; run += c[k]; }
  }
  __syncthreads();
  for (int n = tid; n < a.N; n += NT) {
    const int len = suffix_len(a, n);
    a.order[atomicAdd(&cnt[255 - len / bw], 1u)] = int2{n, len};
  }
  __syncthreads();
}

// Prefix item (KV head h, row block rb, prefix chunk): NW waves own 32 of the N*G rows each and share one LDS ring,
// so the prefix chunk is streamed from HBM once per 32*NW rows.
template <int NW, int kPaged, class V, bool kMF = false>
__device__ __forceinline__ void prefix_rows_item(const PrefixArgs& a, char* smem, int item) {
  const int split = item % a.nsplit_p;
  const int rb = (item / a.nsplit_p) % a.nrb_p;
  const int h = item / (a.nsplit_p * a.nrb_p);
  const int kbeg = split * a.chunk_p;
  const int kend = min(a.P, kbeg + a.chunk_p);
  const int ntiles = (kend - kbeg + kTile - 1) / kTile;
  const int row0 = rb * NW * 32;
  const size_t rows_wg = 32 * NW;
  auto walk = [&](const auto& src) {
    attend_wg_rows<NW, V, kMF>(smem, src,
                       [&](int r) {
                         const int qr = row0 + r, n = qr / a.G, gg = qr % a.G;
                         return a.q + ((size_t)n * a.Hq + h * a.G + gg) * 128;
                       },
                       a.N * a.G - row0, kbeg, ntiles,
                       reinterpret_cast<part_t<elem_t<V>>*>(a.po_p) + (size_t)item * rows_wg * 128,
                       a.pml_p + (size_t)item * rows_wg * 2);
  };
  if constexpr (kPaged != kContig) {
    walk(paged_src<kPaged == kPagedNHD>(a, a.prefix_pages, a.P / a.ps, h, kbeg, kend));
  } else {
    RangeSrc src;
    src.scale = a.sl2;
    const size_t off = (size_t)h * a.P * 128;
    src.kbase = a.kp + off;
    src.vbase = a.vp + off;
    src.kend = kend;
    walk(src);
  }
  if constexpr (kMF) pfx_arrive<false>(a, h);
}

template <int NW, int kPaged, class V>
__global__ __launch_bounds__(64 * NW) void prefix_rows_kernel(PrefixArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kRowsSmemBytes];
  if (blockIdx.x == 0 && a.order) build_suffix_order<64 * NW>(a, reinterpret_cast<uint32_t*>(smem));
  prefix_rows_item<NW, kPaged, V>(a, smem, blockIdx.x);
}

// Prefix unit u (KV head h, prefix chunk) of a mixed launch when a KV head has at most 32 rows: one wave walks the
// chunk for all rows through a private ring of NS stages and writes rows 0..31 of the row-block partial, transposed
// through that ring as the row blocks do (whole rows per store instruction).  A row's arithmetic is that of a
// row-block wave (the same tiles in the same order through the same tile function), so the output bits do not depend
// on which form ran; several units share a workgroup so that the grid stays within one dispatch round when the
// row-block grid would not.
template <int NS, int kPaged, class V, bool kMF>
__device__ __forceinline__ void prefix_unit(const PrefixArgs& a, char* smem, int u, int w) {
  const int lane = threadIdx.x & 63;
  const int split = u % a.nsplit_p, h = u / a.nsplit_p;            // one row block (nrb_p == 1)
  const int kbeg = split * a.chunk_p, kend = min(a.P, kbeg + a.chunk_p);
  const int ntiles = (kend - kbeg + kTile - 1) / kTile;
  const int nrows = a.N * a.G, r = lane & 31;
  const int qr = r < nrows ? r : 0;
  V qb[8];
  load_qt(qb, a.q + ((size_t)(qr / a.G) * a.Hq + h * a.G + qr % a.G) * 128, lane >> 5, r < nrows);
  RowState st;
  row_state_init(st);
  const uint32_t ring_off = (uint32_t)w * NS * kStageBytes;
  const TileLanes tl = tile_lanes(lane, ring_off);
  auto walk = [&](const auto& src) {
    wave_walk<NS>(st, qb, smem + ring_off, smem, tl, src, kbeg, 0, ntiles, 1, lane);
  };
  if constexpr (kPaged != kContig) {
    walk(paged_src<kPaged == kPagedNHD>(a, a.prefix_pages, a.P / a.ps, h, kbeg, kend));
  } else {
    RangeSrc src;
    src.scale = a.sl2;
    const size_t off = (size_t)h * a.P * 128;
    src.kbase = a.kp + off;
    src.vbase = a.vp + off;
    src.kend = kend;
    walk(src);
  }
  const size_t rows_wg = 32 * a.WRp;
  static_assert(NS * kStageBytes >= 32 * 128 * 4, "a unit's ring holds its 32 rows of 128 floats");
  part_t<elem_t<V>>* po = reinterpret_cast<part_t<elem_t<V>>*>(a.po_p) + (size_t)u * rows_wg * 128;
  float* pml = a.pml_p + (size_t)u * rows_wg * 2;
  // Whole rows per store beyond 16 rows (C1, 32 rows: 11.52 us against 12.00, half the written bytes; N = 6 at G = 4:
  // 10.96 against 11.11); up to 16 rows half of each transposed pass would be empty, and the LDS round trip costs more
  // than it saves (N = 4 at G = 4: 10.70 against 10.35 us when every unit transposed).  Both store the same values.
  if (nrows > 16)
    store_partial_rows_wave<kMF>(smem + ring_off, po, pml, st, lane, nrows);
  else
    store_partial<kMF>(po, pml, st, lane, nrows);
  if constexpr (kMF) pfx_arrive<true>(a, h);
}

// Both item kinds in one grid when a KV head has at most 128 rows: prefix items first (row blocks of 4 waves
// sharing a ring, or a.units single-wave units per workgroup), then suffix items.  kMF: whole-suffix items wait for
// their head's prefix partials and write the outputs (a.mfuse); otherwise no item depends on another and the suffix
// items write partials for the merge launch.
constexpr int kMixedSmemBytes = kRowsSmemBytes > kAttnSmemBytes ? kRowsSmemBytes : kAttnSmemBytes;
template <int kPaged, class V, bool kMF>
__global__ __launch_bounds__(256) void prefix_mixed_kernel(PrefixArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kMixedSmemBytes];
  const int upw = a.units;
  const int npw = upw ? (a.n_prefix_items + upw - 1) / upw : a.n_prefix_items;
  if ((int)blockIdx.x >= npw) {
    suffix_item<kPaged, V>(a, smem, blockIdx.x - npw);
  } else if (upw == 0) {
    prefix_rows_item<4, kPaged, V, kMF>(a, smem, blockIdx.x);
  } else {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), u = (int)blockIdx.x * upw + w;
    if (w < upw && u < a.n_prefix_items) {
      static_assert(2 * 4 * kStageBytes <= kMixedSmemBytes && 4 * 2 * kStageBytes <= kMixedSmemBytes, "unit rings");
      if (upw == 2)
        prefix_unit<4, kPaged, V, kMF>(a, smem, u, w);              // a whole chunk of up to 128 keys in flight
      else
        prefix_unit<2, kPaged, V, kMF>(a, smem, u, w);
    }
  }
}

// After a mixed launch with whole suffixes: the final merge of the G rows of (request, KV head), by the functions a
// fused suffix item uses and from the same partial values, so the output bits do not depend on which path ran.
template <class E>
__global__ __launch_bounds__(256) void prefix_merge_kernel(PrefixArgs a) {
  const int nh = blockIdx.x, n = nh / a.Hkv, h = nh % a.Hkv;
  typedef part_t<E> PT;
  const PT* lpo = reinterpret_cast<const PT*>(a.po_s) + (size_t)nh * 32 * 128;   // one suffix split per (n, h)
  const float* lpml = a.pml_s + (size_t)nh * 32 * 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (a.G <= 4 && a.nsplit_p <= kPrefetchSplits) {
    if (wave < a.G) {
      PrefixRow pr;
      prefetch_prefix_row<PT>(a, pr, n, h, wave, lane);
      merge_prefetched_row<E>(a, pr, lpo, lpml, n, h, wave, lane);
    }
  } else {
    merge_prefix_rows<E>(a, lpo, lpml, n, h);
  }
}

// One workgroup (128 threads = head-dims) per output row (n, hq): merge the prefix splits of KV head h and the
// suffix chunks of request n.
template <class E>
__global__ __launch_bounds__(128) void prefix_combine_kernel(PrefixArgs a) {
  const int rowg = blockIdx.x;                 // n * Hq + hq
  const int n = rowg / a.Hq, hq = rowg % a.Hq;
  const int h = hq / a.G, gg = hq % a.G;
  const int prow = n * a.G + gg;               // row of this output among the N*G rows of KV head h
  const int rows_p = 32 * a.WRp;
  const int rb = prow / rows_p, rl = prow % rows_p;
  const size_t pitem0 = ((size_t)h * a.nrb_p + rb) * a.nsplit_p;
  const int np = a.P > 0 ? a.nsplit_p : 0;
  const int sn = suffix_len(a, n);
  const int ns = (sn + a.chunk_s - 1) / a.chunk_s;
  const size_t sitem0 = ((size_t)n * a.Hkv + h) * a.nsplit_s;
  typedef part_t<E> PT;
  combine_row<128, 1, PT>(np + ns,
                          [&](int s, const float*& ml, const PT*& o) {
                            if (s < np) {
                              const size_t base = (pitem0 + s) * rows_p + rl;
                              ml = a.pml_p + base * 2;
                              o = reinterpret_cast<const PT*>(a.po_p) + base * 128;
                            } else {
                              const size_t base = (sitem0 + (s - np)) * 32 + gg;
                              ml = a.pml_s + base * 2;
                              o = reinterpret_cast<const PT*>(a.po_s) + base * 128;
                            }
                          },
                          reinterpret_cast<E*>(a.out) + (size_t)rowg * 128);
}

struct PrefixPlan {
  int WRp, nrb_p, nsplit_p, chunk_p, nsplit_s, chunk_s;
  size_t po_p, pml_p, po_s, pml_s, order;
  int n_prefix_items, n_items;
  int units, n_wg_mixed;    // mixed launch: prefix units per workgroup (0: row blocks) and its grid
  bool fuse;
};

// Every choice that shapes a row's arithmetic depends on P, S and G only, never on N: a request's rows go through
// the same prefix chunks, tile order and merges whatever batch they are in, so a batch row is bit-equal to the same
// request alone.  N only sets how many row blocks there are (and the row-block width, which groups rows that share
// a ring without changing any row's arithmetic).
static PrefixPlan prefix_plan(int64_t N, int64_t Hq, int64_t Hkv, int64_t P, int64_t S) {
  PrefixPlan p;
  const int64_t G = Hq / Hkv, R = N * G;
  p.WRp = R <= 128 ? 4 : 8;                                  // waves sharing one ring, 32 rows each
  const int64_t rows_wg = 32 * p.WRp;
  p.nrb_p = (int)((R + rows_wg - 1) / rows_wg);
  // Prefix chunks of P/32 keys in whole tiles, within [64, 1024] (C1: 64, C2: 512).  The 64-key floor halves each
  // busy wave's serial walk for short prefixes: N = 1, P = 2048, S = 256 takes 9.98 us against 11.18 with a 128-key
  // floor, N = 32, P = 1024, S = 512 21.45 against 22.73; C1 12.18 against 12.13, N = 64 at P = 2048 34.04 against
  // 34.16 (one process, A/B).
  int64_t chunk = (P + 31) / 32;
  chunk = (chunk + kTile - 1) / kTile * kTile;
  chunk = std::min<int64_t>(1024, std::max<int64_t>(64, chunk));
  p.chunk_p = (int)chunk;
  p.nsplit_p = P > 0 ? (int)((P + chunk - 1) / chunk) : 0;
  p.n_prefix_items = (int)(Hkv * p.nrb_p * p.nsplit_p);
  // Suffix chunks of up to 2048 keys (a whole suffix at the BASELINE shapes): one long-lived workgroup per
  // (request, KV head); the hardware dispatcher balances the ragged lengths.  Rows are only the G heads of a request.
  int64_t cs = 2048;
  if (S < cs) cs = std::max<int64_t>(kTile, (S + kTile - 1) / kTile * kTile);
  p.chunk_s = (int)cs;
  p.nsplit_s = (int)((S + cs - 1) / cs);
  p.n_items = p.n_prefix_items + (int)(N * Hkv * p.nsplit_s);
  p.po_p = (size_t)p.n_prefix_items * rows_wg * 128;
  p.pml_p = (size_t)p.n_prefix_items * rows_wg * 2;
  p.po_s = (size_t)N * Hkv * p.nsplit_s * 32 * 128;
  p.pml_s = (size_t)N * Hkv * p.nsplit_s * 32 * 2;
  p.order = (size_t)2 * N;
  // With the prefix partials finished by the prefix launch, whole-suffix items finish their rows themselves.
  p.fuse = p.n_prefix_items > 0 && p.nsplit_s == 1;
  // Mixed launch (R <= 128): one workgroup per prefix item while the grid fits one dispatch round (each workgroup
  // holds 128 KB of LDS, so one per CU); with R <= 32, 2 or 4 single-wave units per workgroup otherwise.  The units
  // compute the same bits as the row blocks, so this choice (which depends on N) does not break batch invariance.
  const int n_suffix = p.n_items - p.n_prefix_items;
  p.units = 0;
  if (p.WRp == 4 && R <= 32 && p.n_items > kDeviceCUs) {
    p.units = 2;
    if ((p.n_prefix_items + 1) / 2 + n_suffix > kDeviceCUs) p.units = 4;
  }
  p.n_wg_mixed = p.units ? (p.n_prefix_items + p.units - 1) / p.units + n_suffix : p.n_items;
  return p;
}

// Plan, workspace carve-up and launches of one prefix call (contiguous or paged; a's K/V pointers are set).
template <int kPaged, class V>
static int prefix_launch(PrefixArgs& a, const void* q, void* out, const void* slens, bool ragged, int64_t N,
                         int64_t Hq, int64_t Hkv, int64_t D, int64_t P, int64_t S, void* workspace, hipStream_t s) {
  PrefixPlan p = prefix_plan(N, Hq, Hkv, P, S);
  a.q = (const f16*)q;
  a.slens = ragged ? (const int*)slens : nullptr;
  a.out = (f16*)out;
  // Partial regions are sized for fp32 rows; fp16 partials use the first half of theirs.
  a.po_p = align_up((char*)workspace + kWsHead, 256);
  a.pml_p = (float*)align_up((float*)a.po_p + p.po_p, 256);
  a.po_s = align_up(a.pml_p + p.pml_p, 256);
  a.pml_s = (float*)align_up((float*)a.po_s + p.po_s, 256);
  // Up to 128 rows per KV head, prefix and suffix items share one launch; a merge (or combine) launch follows.
  // Beyond, the prefix launch runs first and whole-suffix items merge its partials themselves.
  const bool mixed = p.WRp == 4;
  // The schedule order is built by the prefix launch, so only when that runs before the suffix items.
  a.order = (ragged && p.n_prefix_items > 0 && !mixed) ? (int2*)align_up(a.pml_s + p.pml_s, 256) : nullptr;
  a.fuse = p.fuse && !mixed ? 1 : 0;
  // Mixed with whole suffixes: the suffix items merge in the same launch when each wave finishes one row from
  // registers (the form the two-launch fused path uses); else a merge launch follows.
  a.mfuse = p.fuse && mixed && Hq / Hkv <= 4 && p.nsplit_p <= kPrefetchSplits && Hkv <= kPrefixSyncHeads ? 1 : 0;
  a.merge = p.fuse && mixed && !a.mfuse ? 1 : 0;
  a.sync = (uint32_t*)((char*)workspace + kPrefixSync);
  // In a mixed launch every prefix item's busy waves walk a whole prefix chunk (chunk_p / 32 tiles), a suffix item's
  // four waves share its chunk (chunk_s / 128 tiles each).  A suffix item with fewer tiles than that has slack: it
  // waits about 3,000 cycles, so that its loads do not compete with the prefix items' first tiles (C1: 12.3 against
  // 12.8 us; the suffix items' results are needed only after the prefix items').
  a.sfx_delay = mixed && (p.chunk_s / kTile + 3) / 4 < p.chunk_p / kTile ? 3 : 0;
  a.units = mixed ? p.units : 0;
  a.N = (int)N; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv); a.P = (int)P; a.S = (int)S;
  a.WRp = p.WRp; a.nrb_p = p.nrb_p; a.nsplit_p = p.nsplit_p; a.chunk_p = p.chunk_p;
  a.nsplit_s = p.nsplit_s; a.chunk_s = p.chunk_s; a.n_prefix_items = p.n_prefix_items;
  a.sl2 = (float)(1.0 / sqrt((double)D)) * kLog2e;
  prof_before(kKPrefixPartial, s);
  if (mixed) {
    if (a.mfuse)
      hipLaunchKernelGGL((prefix_mixed_kernel<kPaged, V, true>), dim3((unsigned)p.n_wg_mixed), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((prefix_mixed_kernel<kPaged, V, false>), dim3((unsigned)p.n_wg_mixed), dim3(256), 0, s, a);
    VMK_CHECK_HIP(hipGetLastError());
  } else {
    if (p.n_prefix_items > 0) {
      hipLaunchKernelGGL((prefix_rows_kernel<8, kPaged, V>), dim3((unsigned)p.n_prefix_items), dim3(512), 0, s, a);
      VMK_CHECK_HIP(hipGetLastError());
    }
    if (p.n_items > p.n_prefix_items) {
      hipLaunchKernelGGL((prefix_partial_kernel<kPaged, V>), dim3((unsigned)(p.n_items - p.n_prefix_items)),
                         dim3(256), 0, s, a);
      VMK_CHECK_HIP(hipGetLastError());
    }
  }
  prof_after(kKPrefixPartial, s);
  if (a.merge) {
    prof_before(kKPrefixCombine, s);
    hipLaunchKernelGGL(prefix_merge_kernel<elem_t<V>>, dim3((unsigned)(N * Hkv)), dim3(256), 0, s, a);
    prof_after(kKPrefixCombine, s);
    VMK_CHECK_HIP(hipGetLastError());
  } else if (!a.fuse && !a.mfuse) {
    prof_before(kKPrefixCombine, s);
    hipLaunchKernelGGL(prefix_combine_kernel<elem_t<V>>, dim3((unsigned)(N * Hq)), dim3(128), 0, s, a);
    prof_after(kKPrefixCombine, s);
    VMK_CHECK_HIP(hipGetLastError());
  }
  return 0;
}

}  // namespace vmk

using namespace vmk;

extern "C" size_t vmk_prefix_workspace_size(int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t P, int64_t S,
                                            int64_t ragged) {
  (void)ragged;
  if (N <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || D != 128 || P < 0 || S < 0 || P + S <= 0) return 0;
  PrefixPlan p = prefix_plan(N, Hq, Hkv, P, S);
  return kWsHead + (p.po_p + p.pml_p + p.po_s + p.pml_s + p.order) * sizeof(float) + 5 * 256;
}

template <class V>
static int prefix_decode(const void* q, const void* kp, const void* vp, const void* ks, const void* vs,
                         const void* slens, void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t P,
                         int64_t S, int64_t ragged, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(q && out && (P == 0 || (kp && vp)) && (S == 0 || (ks && vs)), "null pointer argument");
  VMK_CHECK(N > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "bad head/request sizes");
  VMK_CHECK(D == 128, "only head_dim 128 is supported");
  VMK_CHECK(Hq / Hkv <= 32, "at most 32 query heads per KV head");
  VMK_CHECK(P >= 0 && S >= 0 && P + S > 0, "P and S must be >= 0 with P + S > 0");
  VMK_CHECK(!ragged || slens, "ragged=1 needs slens");
  VMK_CHECK(P < (1 << 30) && S < (1 << 30) && N * (Hq / Hkv) < (1 << 20), "sizes out of range");
  VMK_CHECK(aligned16(q) && aligned16(out) && (P == 0 || (aligned16(kp) && aligned16(vp))) &&
                (S == 0 || (aligned16(ks) && aligned16(vs))),
            "tensors must be 16-byte aligned");
  const size_t need = vmk_prefix_workspace_size(N, Hq, Hkv, D, P, S, ragged);
  VMK_CHECK(workspace && ws_bytes >= need, "workspace too small (query vmk_prefix_workspace_size)");
  PrefixArgs a;
  a.q = (const f16*)q; a.kp = (const f16*)kp; a.vp = (const f16*)vp; a.ks = (const f16*)ks; a.vs = (const f16*)vs;
  a.prefix_pages = a.suffix_pages = nullptr;
  a.ps = a.max_sp = a.num_pages = 0;
  return prefix_launch<kContig, V>(a, q, out, slens, ragged != 0, N, Hq, Hkv, D, P, S, workspace, (hipStream_t)stream);
}

extern "C" int vmk_prefix_decode(const void* q, const void* kp, const void* vp, const void* ks, const void* vs,
                                 const void* slens, void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D,
                                 int64_t P, int64_t S, int64_t ragged, void* workspace, size_t ws_bytes,
                                 void* stream) {
  return prefix_decode<half8>(q, kp, vp, ks, vs, slens, out, N, Hq, Hkv, D, P, S, ragged, workspace, ws_bytes,
                              stream);
}

extern "C" int vmk_prefix_decode_bf16(const void* q, const void* kp, const void* vp, const void* ks, const void* vs,
                                      const void* slens, void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t P, int64_t S, int64_t ragged, void* workspace, size_t ws_bytes,
                                      void* stream) {
  return prefix_decode<bf16x8>(q, kp, vp, ks, vs, slens, out, N, Hq, Hkv, D, P, S, ragged, workspace, ws_bytes,
                               stream);
}

extern "C" size_t vmk_prefix_paged_workspace_size(int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t P,
                                                  int64_t page_size, int64_t max_suffix_pages) {
  if (page_size < 32 || page_size % 32 || page_size > (1 << 20) || P < 0 || P % page_size || max_suffix_pages < 0)
    return 0;
  return vmk_prefix_workspace_size(N, Hq, Hkv, D, P, page_size * max_suffix_pages, 1);
}

template <int kLayout, class V>
static int prefix_decode_paged(const void* q, const void* k_pages, const void* v_pages, const void* prefix_pages,
                               const void* suffix_pages, const void* slens, void* out, int64_t N, int64_t Hq,
                               int64_t Hkv, int64_t D, int64_t num_pages, int64_t page_size, int64_t P,
                               int64_t max_suffix_pages, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(q && out && k_pages && v_pages && (P == 0 || prefix_pages) && (max_suffix_pages == 0 || suffix_pages),
            "null pointer argument");
  VMK_CHECK(N > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "bad head/request sizes");
  VMK_CHECK(D == 128, "only head_dim 128 is supported");
  VMK_CHECK(Hq / Hkv <= 32, "at most 32 query heads per KV head");
  VMK_CHECK(page_size >= 32 && page_size % 32 == 0 && page_size <= (1 << 20), "page_size must be a multiple of 32");
  VMK_CHECK(P >= 0 && P % page_size == 0, "P must be a whole number of pages");
  VMK_CHECK(max_suffix_pages >= 0 && P + page_size * max_suffix_pages > 0, "no keys: P and max_suffix_pages are 0");
  VMK_CHECK(num_pages > 0 && num_pages < (1 << 30) && num_pages * Hkv * page_size <= ((int64_t)1 << 34),
            "num_pages out of range");
  VMK_CHECK(P < (1 << 30) && page_size * max_suffix_pages < (1 << 30) && N * (Hq / Hkv) < (1 << 20),
            "sizes out of range");
  VMK_CHECK(aligned16(q) && aligned16(out) && aligned16(k_pages) && aligned16(v_pages),
            "tensors must be 16-byte aligned");
  VMK_CHECK(kLayout != kPagedNHD || Hkv <= 4096, "NHD pages: at most 4096 KV heads");
  const int64_t S = page_size * max_suffix_pages;
  const size_t need = vmk_prefix_paged_workspace_size(N, Hq, Hkv, D, P, page_size, max_suffix_pages);
  VMK_CHECK(workspace && ws_bytes >= need, "workspace too small (query vmk_prefix_paged_workspace_size)");
  PrefixArgs a;
  a.q = (const f16*)q; a.kp = (const f16*)k_pages; a.vp = (const f16*)v_pages; a.ks = a.vs = nullptr;
  a.prefix_pages = (const int*)prefix_pages;
  a.suffix_pages = (const int*)suffix_pages;
  a.ps = (int)page_size; a.max_sp = (int)max_suffix_pages; a.num_pages = (int)num_pages;
  return prefix_launch<kLayout, V>(a, q, out, slens, slens != nullptr, N, Hq, Hkv, D, P, S, workspace,
                                (hipStream_t)stream);
}

extern "C" int vmk_prefix_decode_paged(const void* q, const void* k_pages, const void* v_pages,
                                       const void* prefix_pages, const void* suffix_pages, const void* slens,
                                       void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t num_pages,
                                       int64_t page_size, int64_t P, int64_t max_suffix_pages, void* workspace,
                                       size_t ws_bytes, void* stream) {
  return prefix_decode_paged<kPagedHND, half8>(q, k_pages, v_pages, prefix_pages, suffix_pages, slens, out, N, Hq,
                                               Hkv, D, num_pages, page_size, P, max_suffix_pages, workspace,
                                               ws_bytes, stream);
}

extern "C" int vmk_prefix_decode_paged_bf16(const void* q, const void* k_pages, const void* v_pages,
                                            const void* prefix_pages, const void* suffix_pages, const void* slens,
                                            void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D,
                                            int64_t num_pages, int64_t page_size, int64_t P, int64_t max_suffix_pages,
                                            void* workspace, size_t ws_bytes, void* stream) {
  return prefix_decode_paged<kPagedHND, bf16x8>(q, k_pages, v_pages, prefix_pages, suffix_pages, slens, out, N, Hq,
                                                Hkv, D, num_pages, page_size, P, max_suffix_pages, workspace,
                                                ws_bytes, stream);
}

extern "C" int vmk_prefix_decode_paged_nhd(const void* q, const void* k_pages, const void* v_pages,
                                           const void* prefix_pages, const void* suffix_pages, const void* slens,
                                           void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D,
                                           int64_t num_pages, int64_t page_size, int64_t P, int64_t max_suffix_pages,
                                           void* workspace, size_t ws_bytes, void* stream) {
  return prefix_decode_paged<kPagedNHD, half8>(q, k_pages, v_pages, prefix_pages, suffix_pages, slens, out, N, Hq,
                                               Hkv, D, num_pages, page_size, P, max_suffix_pages, workspace,
                                               ws_bytes, stream);
}

extern "C" int vmk_prefix_decode_paged_nhd_bf16(const void* q, const void* k_pages, const void* v_pages,
                                                const void* prefix_pages, const void* suffix_pages,
                                                const void* slens, void* out, int64_t N, int64_t Hq, int64_t Hkv,
                                                int64_t D, int64_t num_pages, int64_t page_size, int64_t P,
                                                int64_t max_suffix_pages, void* workspace, size_t ws_bytes,
                                                void* stream) {
  return prefix_decode_paged<kPagedNHD, bf16x8>(q, k_pages, v_pages, prefix_pages, suffix_pages, slens, out, N, Hq,
                                                Hkv, D, num_pages, page_size, P, max_suffix_pages, workspace,
                                                ws_bytes, stream);
}
