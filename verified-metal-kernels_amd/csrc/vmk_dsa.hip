// DeepSeek Sparse Attention decode on gfx950: indexer -> exact top-2048 -> sparse absorbed-MLA attention.
//
// Replaces the reference's dsa_indexer / dsa_select / dsa_qk / dsa_pv / dsa_red Metal kernels
// (kernels/dsa_opus55_v7.py:27-98, 100-307, 309-535, 553-605, 629-727) behind the
// kernel(q, kv, iq, ik, w, lens) contract of ops/dsa.py:1-9.
//
// Workspace layout (after the zero-invariant head, which holds the histograms when B <= 64):
//   hist   : B x 8192 uint32   per-request histogram of the top 13 bits of the score key
//   chist  : B x 256 uint32    per-request histogram of the top 8 bits
//   scores : B x Ls   float    indexer scores (Ls = L rounded up to whole 4096-position scan slices)
//   glist, ekey, epos : B x Ls select_scan's per-slice compacted lists; gcnt, ecnt: their lengths
//   po/pml : attention partials [b][head block][chunk][32][512] and [..][32][2]
#include "attn_core.h"
#include "select_math.h"
#include "vmk_internal.h"

namespace vmk {

constexpr int kH = 128, kDK = 576, kDC = 512, kHI = 64, kDI = 128, kTopK = 2048;
constexpr int kBins = kSelBins;    // first radix digit: key bits 31..19
constexpr int kCBins = kSelCBins;  // coarse bins of the first digit (key bits 31..24)
constexpr int kIdxWG = 1024;       // positions per indexer workgroup (8 waves x 4 tiles of 32)
constexpr int kIdxWaves = 8;       // two waves per SIMD hide each other's LDS and MFMA latencies
constexpr int kIdxStages = 2;      // private DMA ring stages per indexer wave
constexpr int kIdxStageBytes = 8192;   // one tile: 32 positions x 256 bytes of ik
constexpr int kChunk = 128;        // selected keys per attention workgroup
constexpr int kNChunk = kTopK / kChunk;
constexpr int kCand = 4096;        // LDS candidate capacity of the select kernel
constexpr int kScanWG = 4096;      // positions per select_scan workgroup (256 threads x 16)
constexpr int kMaxSlices = 1024;   // the select handles up to 1024 scan slices (L <= 4M)
constexpr int kCandAttn = 1024;    // LDS candidate capacity of the select in an attention workgroup

struct DsaArgs {
  const f16* q;         // (B, 128, 576)
  const f16* kv;        // (B, L, 576)
  const f16* iq;        // (B, 64, 128)
  const f16* ik;        // (B, L, 128)
  const float* w;       // (B, 64)
  const int* lens;      // (B,) or null
  int* idx;             // (B, 2048)
  int* cnt;             // (B,)
  f16* out;             // (B, 128, 512)
  uint32_t* hist;       // (B, hcopies, 8192): the fine histogram of request b is the sum of its hcopies copies
  float* scores;        // (B, Ls)
  void* po;             // (B, 4, kNChunk, 32, 512) normalised O of type part_t
  float* pml;           // (B, 4, kNChunk, 32, 2)
  int* glist;           // (B, L) per scan slice: positions above the threshold bucket, in position order
  uint32_t* ekey;       // (B, L) per scan slice: keys of the threshold bucket's positions, in position order
  int* epos;            // (B, L) ... and their positions
  int* gcnt;            // (B, nb) list lengths per slice
  int* ecnt;            // (B, nb)
  int B, L, nb;         // nb = scan slices per request
  int Ls;               // row stride of scores and the scan lists: nb * kScanWG
  int hist_in_head;     // 1: hist lives in the zero-invariant workspace head (no zero-fill launch needed)
  int hcopies;          // copies of each request's fine histogram (workgroup w of a request adds into copy w % hcopies)
  int fused_select;     // 1: every attention workgroup selects its own chunk (decode entry); 0: idx/cnt are inputs
  int scores_only;      // 1: the indexer writes scores (row stride Ls) and no histograms (vmk_dsa_indexer)
  const float* scores_in;  // (B, L) caller scores for vmk_dsa_topk, copied into `scores` by dsa_scores_hist_kernel
  uint32_t* chist;      // (B, 256) coarse histogram: 32 first-digit bins per coarse bin (zero-invariant like hist)
  float sl2;            // attention scale * log2(e)
  uint32_t* sync;       // single-launch decode: grid-barrier counters and the timeout flag (workspace head)
};

// Order-preserving float -> uint32 map: a < b as floats  <=>  fkey(a) < fkey(b) (NaN above +inf).
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int valid_len(const DsaArgs& a, int b) {
  return a.lens ? min(max(a.lens[b], 0), a.L) : a.L;
}

// Copy c of request b's fine histogram.  The workgroups of a request add their counts into hcopies copies instead
// of one, so that fewer of them add into the same words at once (device-scope adds to one word are serialised: in a
// microbenchmark, 64 workgroups adding into the same 300 bins take about 4.5 us longer than an empty launch, into 8
// copies 1.4 us); a reader sums the copies, which gives the same integers.
__device__ __forceinline__ uint32_t* fine_hist(const DsaArgs& a, int b, int c) {
  return a.hist + ((size_t)b * a.hcopies + c) * kBins;
}
constexpr int kMaxFineCopies = 2;
// Bin `bin` of request b's fine histogram, summed over its copies.  Every copy's word is loaded before the first is
// added: a loop over the run-time count would wait for each load before issuing the next.
__device__ __forceinline__ uint32_t fine_bin_sum(const DsaArgs& a, int b, int bin) {
  uint32_t v[kMaxFineCopies];
#pragma unroll
  for (int c = 0; c < kMaxFineCopies; ++c) v[c] = fine_hist(a, b, min(c, a.hcopies - 1))[bin];
  uint32_t t = v[0];
#pragma unroll
  for (int c = 1; c < kMaxFineCopies; ++c) t += c < a.hcopies ? v[c] : 0u;
  return t;
}

// ------------------------------------------------------------------------------------------------ indexer
// Block-wide exclusive prefix sum of v over thread ids (NT threads); *total receives the sum of all v.  The block
// helpers exchange data through LDS only, so their barriers wait for LDS operations only: global loads of the
// caller stay in flight across them.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* red, uint32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan(v);  // inclusive prefix within the wave
  if (lane == 63) red[wave] = x;
  lds_barrier();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int w2 = 0; w2 < NT / 64; ++w2) {
    const uint32_t t = red[w2];
    all += t;
    if (w2 < wave) before += t;
  }
  lds_barrier();
  *total = all;
  return before + x - v;
}

// Finds, in hist[0..NBINS) (NBINS a multiple of NT), the bin holding the need-th largest element: out[0] = bin,
// out[1] = need minus the count strictly above that bin.  Every thread of the block must call it.  Each thread reads
// its NBINS / NT bins once into registers.  The per-thread arithmetic is select_math.h's, which
// vmk_debug_select_threshold replays on the host.
template <int NT, int NBINS>
__device__ void find_threshold(const uint32_t* hist, uint32_t need, uint32_t* red, uint32_t* out) {
  static_assert(NBINS % NT == 0, "whole bins per thread");
  constexpr int kPer = NBINS / NT;
  // Defaults (bin 0) for a histogram that holds fewer than `need` elements, so callers that index with out[0]
  // stay in bounds; the barriers of the scan below order these writes before the finder's.
  if (threadIdx.x == 0) {
    out[0] = 0;
    out[1] = 0;
  }
  const int lo = threshold_range_lo(threadIdx.x, NT, kPer);   // a prefix scan over thread ids runs top-down
  uint32_t bins[kPer], local = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    bins[i] = hist[lo + i];
    local += bins[i];
  }
  uint32_t total;
  const uint32_t above = block_excl_scan<NT>(local, red, &total);
  Threshold t;
  // A range whose counts cannot reach the need-th element from `above` has no hit; skip its walk.
  if (above < need && above + local >= need && threshold_in_range(bins, 0, kPer, above, need, &t)) {
    out[0] = (uint32_t)lo + t.bin;
    out[1] = t.rest;
  }
  lds_barrier();
}

// ik rows of one request as a key source of the DMA tile loader (K half of a stage only).
struct IkSrc {
  const f16* kbase;
  const f16* vbase;
  int kend;
  static constexpr bool kStrided = false;   // rows 256 bytes apart
  __device__ const f16* ktile(int key0) const { return kbase + (size_t)key0 * kDI; }
  __device__ const f16* vtile(int key0) const { return ktile(key0); }
};

// S = iq . ik^T per 32-position tile (M = 64 heads as two 32-row MFMA tiles, N = positions, K = 128 dims), then
// score = sum_h w[h] * max(S[h], 0) in fp32, and histograms of fkey(score) >> 19 (fine) and >> 24 (coarse) per
// request.  One item = positions [1024 bx, 1024 bx + 1024) of request b, by NW waves (64 NW threads); each wave
// streams its 32 / NW tiles through a private NS-stage ring of direct-to-LDS loads; the B operand (ik^T) is read from
// the stage with the attention core's K-operand offsets.  LDS: ring (NW * NS * 8 KB), hist2 (16 KB), chist (1 KB).
template <class V, int NW, int NS>
__device__ __forceinline__ void indexer_item(const DsaArgs& a, int bx, int b, char* __restrict__ ring,
                                             uint32_t* __restrict__ hist2, uint32_t* __restrict__ chist) {
  static_assert(NS >= 2 && NS <= 4 && NW * 64 >= kCBins && 16 % NW == 0 && NW >= 3,
                "iq, w in the last stage of waves 0-2; 16 iq loads split over the waves");
  const int tid = threadIdx.x;
  const int n = valid_len(a, b);
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, g = lane >> 5;
  // Every wave needs all of iq (16 KB) and w (256 B) as operands.  They are loaded once per workgroup, by direct-to-
  // LDS loads into the last ring stage of waves 0, 1 and 2 (which the walk fills last), ahead of the ring's first
  // tiles: per-wave loads would push NW x the bytes through the CU's load path in front of tile 0.  iq row r lands
  // at byte 256 r of its half (heads 0-31, 32-63) with 16-byte chunk c at position c ^ (r & 15), so the operand
  // reads below, 32 rows at one chunk, hit 16 distinct bank groups.
  V qa[2][8];                                                // filled from LDS before the walk
  float wv[2][16];
  const f16* iqb = a.iq + (size_t)b * kHI * kDI;
  char* const iq_lds0 = ring + (0 * NS + NS - 1) * kIdxStageBytes;
  char* const iq_lds1 = ring + (1 * NS + NS - 1) * kIdxStageBytes;
  char* const w_lds = ring + (2 * NS + NS - 1) * kIdxStageBytes;
  constexpr int kIqPerWave = 16 / NW;
  {
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(iqb), 0, kHI * kDI * 2, 0x00020000);
#pragma unroll
    for (int q = 0; q < kIqPerWave; ++q) {
      const int j = kIqPerWave * wave + q;                   // rows 4j .. 4j + 3
      const int row = 4 * j + (lane >> 4);
      const uint32_t off = (uint32_t)(row * 256 + (((lane & 15) ^ (row & 15)) << 4));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, VMK_LPTR((j < 8 ? iq_lds0 : iq_lds1) + (j & 7) * 1024), 16, off,
                                               0, 0, 0);
    }
    if (wave == 0) {
      const __amdgpu_buffer_rsrc_t rw =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.w + b * kHI), 0, kHI * 4, 0x00020000);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, VMK_LPTR(w_lds), 4, (uint32_t)lane * 4, 0, 0, 0);
    }
  }

  IkSrc src;
  src.kbase = a.ik + (size_t)b * a.L * kDI;
  src.vbase = src.kbase;
  src.kend = n;
  constexpr int kTilesPerWave = kIdxWG / kTile / NW;
  const int t0 = bx * (kIdxWG / kTile) + wave * kTilesPerWave;   // this wave's first tile
  const int nt = max(0, min(kTilesPerWave, (n + kTile - 1) / kTile - t0));
  const uint32_t ring_off = (uint32_t)wave * NS * kIdxStageBytes;
  const TileLanes tl = tile_lanes(lane, ring_off);
  char* wring = ring + ring_off;
  float* sc = a.scores + (size_t)b * a.Ls;
  auto issue = [&](char* stage, int j) {
    const int key0 = (t0 + j) * kTile;
    if (key0 + kTile <= n) {
#pragma unroll
      for (int i = 0; i < 8; ++i) issue_dma_full(stage, src, key0, i, tl.dma[i & 3]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) issue_dma_part(stage, src, key0, i, tl.dma[i & 3], lane);
    }
  };
  auto compute = [&](const char* stage, int j) {
    u32x4 kk[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) kk[t] = *reinterpret_cast<const u32x4*>(stage + tl.k[t]);
    floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      s0 = mfma32(qa[0][t], as_v8<V>(kk[t]), s0);
      s1 = mfma32(qa[1][t], as_v8<V>(kk[t]), s1);
    }
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) part += wv[0][i] * fmaxf(s0[i], 0.f) + wv[1][i] * fmaxf(s1[i], 0.f);
    const float tot = part + xor32(part);
    const int pos = (t0 + j) * kTile + r;
    if (g == 0 && pos < n) {
      sc[pos] = tot;
      if (!a.scores_only) {
        const uint32_t bin = fkey(tot) >> 19;
        atomicAdd(&hist2[bin >> 1], 1u << (16 * (bin & 1)));
        atomicAdd(&chist[bin >> 5], 1u);
      }
    }
  };
  auto pre = [&](auto S) {
    if (S >= nt) return false;
    issue(wring + S * kIdxStageBytes, S);
    return true;
  };
  unroll_while<0, NS - 1>(pre);
  // The histogram is cleared while the loads fly; the wait lets only the ring's first tiles (issued after iq and w)
  // stay in flight, so after the barrier every wave's part of iq and w is in LDS.  A second barrier frees the last
  // stages for the walk.
  for (int i = tid; i < kBins / 2; i += 64 * NW) hist2[i] = 0;
  if (tid < kCBins) chist[tid] = 0;
  wait_vmem_dyn(8 * min(NS - 1, nt));
  lds_barrier();
#pragma unroll
  for (int s = 0; s < 8; ++s) {                              // Q^T operand: head r's dims 64g + 8s .. (chunk 8g + s)
    const int pos = ((8 * g + s) ^ (r & 15)) << 4;
    qa[0][s] = as_v8<V>(*reinterpret_cast<const u32x4*>(iq_lds0 + r * 256 + pos));
    qa[1][s] = as_v8<V>(*reinterpret_cast<const u32x4*>(iq_lds1 + r * 256 + pos));
  }
#pragma unroll
  for (int ht = 0; ht < 2; ++ht)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {                         // weights of the rows 8 i4 + 4g .. + 3 of S^T
      const floatx4 v = *reinterpret_cast<const floatx4*>(w_lds + 4 * (ht * 32 + 8 * i4 + 4 * g));
#pragma unroll
      for (int e = 0; e < 4; ++e) wv[ht][4 * i4 + e] = v[e];
    }
  lds_barrier();
  for (int j0 = 0; j0 < nt; j0 += NS) {
    auto step = [&](auto S) {
      const int j = j0 + S, jn = j + NS - 1;
      if (j >= nt) return false;
      asm volatile("" ::: "memory");
      if (jn < nt) issue(wring + ((S + NS - 1) % NS) * kIdxStageBytes, jn);
      wait_vmem_dyn(8 * min(NS - 1, nt - 1 - j));
      compute(ring + S * kIdxStageBytes, j);
      return true;
    };
    if (!unroll_while<0, NS>(step)) break;
  }
  if (a.scores_only) return;                                // uniform: no histograms to add
  __syncthreads();
  uint32_t* gh = fine_hist(a, b, bx % a.hcopies);
  for (int i = tid; i < kBins / 2; i += 64 * NW) {
    const uint32_t c = hist2[i];
    if (c & 0xFFFFu) atomicAdd(&gh[2 * i], c & 0xFFFFu);
    if (c >> 16) atomicAdd(&gh[2 * i + 1], c >> 16);
  }
  if (tid < kCBins) {
    const uint32_t c = chist[tid];
    if (c) atomicAdd(&a.chist[(size_t)b * kCBins + tid], c);
  }
}

template <class V>
__global__ __launch_bounds__(64 * kIdxWaves) void dsa_indexer_kernel(DsaArgs a) {
  __shared__ __attribute__((aligned(16))) char ring[kIdxWaves * kIdxStages * kIdxStageBytes];
  __shared__ uint32_t hist2[kBins / 2];                     // two 16-bit bin counts per word (<= 1024 per bin)
  __shared__ uint32_t chist[kCBins];
  indexer_item<V, kIdxWaves, kIdxStages>(a, blockIdx.x, blockIdx.y, ring, hist2, chist);
}

// ------------------------------------------------------------------------------------------------ select
// Exact top-2048 per request in two launches.  Radix digits of the score key: bits 31..19 (the indexer's histogram),
// 18..8 and 7..0 (LDS histograms over the threshold bucket's candidates).
//   select_scan  (4096 positions per workgroup): with the threshold bucket b1 the indexer found, every workgroup
//                compacts its slice: positions above b1 to glist, bucket-b1 (key, position) pairs to ekey/epos;
//   select_final (one workgroup per request): concatenates the slices' lists in slice order, refines the bucket to
//                the exact threshold key T and emits the remaining picks.
// All compaction uses block scans over thread-contiguous position ranges, so the output order (positions above the
// bucket in increasing order, then the bucket's picks in increasing order, ties at T broken by position) does not
// depend on scheduling, and neither do the attention sums that follow.

// vmk_dsa_topk: caller scores (B, L) into the workspace's scores (row stride Ls, the padding zero-filled) and the same
// histograms the indexer builds, 1024 positions per workgroup (4 per thread).
__global__ __launch_bounds__(256) void dsa_scores_hist_kernel(DsaArgs a) {
  __shared__ uint32_t hist2[kBins / 2];
  __shared__ uint32_t chist[kCBins];
  const int b = blockIdx.y, tid = threadIdx.x;
  const int n = valid_len(a, b);
  for (int i = tid; i < kBins / 2; i += 256) hist2[i] = 0;
  chist[tid] = 0;
  __syncthreads();
  const float* src = a.scores_in + (size_t)b * a.L;
  float* dst = a.scores + (size_t)b * a.Ls;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int p = blockIdx.x * 1024 + k * 256 + tid;       // < Ls by the grid
    const float v = p < a.L ? src[p] : 0.f;
    dst[p] = v;
    if (p < n) {
      const uint32_t bin = fkey(v) >> 19;
      atomicAdd(&hist2[bin >> 1], 1u << (16 * (bin & 1)));
      atomicAdd(&chist[bin >> 5], 1u);
    }
  }
  __syncthreads();
  uint32_t* gh = fine_hist(a, b, blockIdx.x % a.hcopies);
  for (int i = tid; i < kBins / 2; i += 256) {
    const uint32_t c = hist2[i];
    if (c & 0xFFFFu) atomicAdd(&gh[2 * i], c & 0xFFFFu);
    if (c >> 16) atomicAdd(&gh[2 * i + 1], c >> 16);
  }
  const uint32_t c = chist[tid];
  if (c) atomicAdd(&a.chist[(size_t)b * kCBins + tid], c);
}

// LDS of one select_scan item.
struct ScanShared {
  uint32_t cnt[kCBins], red[4], thr[2], b1s;
};

// One select_scan item: slice wg (positions [4096 wg, 4096 wg + 4096)) of request b, by 256 threads.
__device__ __forceinline__ void select_scan_item(const DsaArgs& a, int wg, int b, ScanShared& sh) {
  uint32_t* const cnt = sh.cnt;
  uint32_t* const red = sh.red;
  uint32_t* const thr = sh.thr;
  uint32_t& b1s = sh.b1s;
  const int tid = threadIdx.x;
  const int n = valid_len(a, b);
  const int base = wg * kScanWG;
  if (n <= kTopK || base >= n) {                   // whole workgroup: nothing of this slice is selected
    if (tid == 0) { a.gcnt[b * a.nb + wg] = 0; a.ecnt[b * a.nb + wg] = 0; }
    return;
  }
  // This thread's 16 positions (4 float4), loaded while the threshold bucket is found.
  const float* sc = a.scores + (size_t)b * a.Ls;
  const int p0 = base + tid * 16;
  uint32_t key[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = p0 + 4 * i;
    const floatx4 v = *reinterpret_cast<const floatx4*>(sc + p);   // rows are padded to whole slices
#pragma unroll
    for (int e = 0; e < 4; ++e) key[4 * i + e] = fkey(v[e]);
  }
  // Threshold bucket b1: the coarse histogram gives the coarse bin and the picks left in it, its 32 fine bins b1.
  cnt[tid] = a.chist[(size_t)b * kCBins + tid];
  if (tid == 0) b1s = 0;
  __syncthreads();
  find_threshold<256, kCBins>(cnt, kTopK, red, thr);
  if (tid < 64) {
    const int f0 = coarse_bin_clamped(thr[0]) * 32;
    uint32_t v = 0u;                                         // lane i: fine bin 31 - i (top first)
    if (tid < 32) v = fine_bin_sum(a, b, f0 + 31 - tid);
    const uint32_t x = wave_incl_scan(v);                    // inclusive prefix from the top
    if (tid < 32 && fine_hit(x, v, thr[1])) b1s = fine_bin(thr[0], tid);
  }
  __syncthreads();
  const int nv = n - p0;                           // positions p0 + i with i < nv are valid
  const uint32_t b1 = b1s;
  uint32_t c_gt = 0, c_eq = 0, t_gt, t_eq;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    c_gt += i < nv && (key[i] >> 19) > b1;
    c_eq += i < nv && (key[i] >> 19) == b1;
  }
  uint32_t o_gt = block_excl_scan<256>(c_gt, red, &t_gt);
  uint32_t o_eq = block_excl_scan<256>(c_eq, red, &t_eq);
  int* gl = a.glist + (size_t)b * a.Ls + base;
  uint32_t* ek = a.ekey + (size_t)b * a.Ls + base;
  int* ep = a.epos + (size_t)b * a.Ls + base;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t bin = key[i] >> 19;
    if (i >= nv) break;
    if (bin > b1) gl[o_gt++] = p0 + i;
    else if (bin == b1) { ek[o_eq] = key[i]; ep[o_eq] = p0 + i; ++o_eq; }
  }
  if (tid == 0) { a.gcnt[b * a.nb + wg] = (int)t_gt; a.ecnt[b * a.nb + wg] = (int)t_eq; }
}

__global__ __launch_bounds__(256) void dsa_select_scan_kernel(DsaArgs a) {
  __shared__ ScanShared sh;
  select_scan_item(a, blockIdx.x, blockIdx.y, sh);
}

// LDS of the select: the second and third radix digits' histogram, the threshold bucket's candidates when there are
// at most CAND of them (more are read from the slices' lists in memory), and both lists' slice offsets.
template <int CAND>
struct SelectShared {
  uint32_t hist[2048];           // second digit (bits 18..8)
  uint32_t hist3[1024];          // third digit (bits 7..0): 256 bins, or one per thread of a larger block
  uint32_t cand_key[CAND];
  int cand_pos[CAND];
  uint32_t goff[kMaxSlices + 1], eoff[kMaxSlices + 1];
  uint32_t red[16], thr[2];
};

// Slice holding list element e, given exclusive offsets off[0..ns] (off[ns] = total).
__device__ __forceinline__ int slice_of(const uint32_t* off, int ns, uint32_t e) {
  int lo = 0, hi = ns - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= e) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// A compile-time bool as a type (selects an instantiation of a generic lambda).
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

// The picks of output slots [lo, hi) of request b, after select_scan.  Every form of the select produces the same
// order: the positions above the threshold bucket b1 in increasing order (the slices' lists back to back), then the
// bucket's keys above the exact threshold key T in position order, then its first need_eq keys equal to T in
// position order; a request with n <= 2048 valid positions selects 0..n-1 and fills the other slots with 0.  The
// bucket is refined to T by the second (bits 18..8) and third (bits 7..0) digits over LDS histograms.  None of this
// depends on NT, the block size, or on which window is asked for: every result is an integer count or a position.
// emit(slot, position) is called for each slot of the window that holds a pick (every slot, for consistent inputs).
// The window holds at most W slots (hi - lo <= W).  Returns the request's count, min(n, 2048).  Every thread of the
// block calls it.
template <int NT, int W, int CAND, class Emit>
__device__ int select_window(const DsaArgs& a, SelectShared<CAND>& sh, int b, int lo, int hi, Emit emit) {
  static_assert(kMaxSlices % NT == 0, "slices per thread");
  // The third digit's histogram: 256 bins, or one per thread when the block is larger (the upper bins stay zero).
  constexpr int kH3 = NT > 256 ? NT : 256;
  static_assert(kH3 <= (int)(sizeof(sh.hist3) / sizeof(sh.hist3[0])), "third-digit bins");
  const int tid = threadIdx.x;
  const int n = valid_len(a, b);
  if (n <= kTopK) {
    for (int s = lo + tid; s < hi; s += NT) emit(s, s < n ? s : 0);
    return n;
  }
  // The digits' histograms are cleared while the first loads fly (the scans' barriers below order it).
  for (int i = tid; i < 2048; i += NT) sh.hist[i] = 0;
  for (int i = tid; i < kH3; i += NT) sh.hist3[i] = 0;
  const int ns = (n + kScanWG - 1) / kScanWG;
  const int* glb = a.glist + (size_t)b * a.Ls;
  const uint32_t* ekb = a.ekey + (size_t)b * a.Ls;
  const int* epb = a.epos + (size_t)b * a.Ls;
  // Up to kSpecSlices slices, the first kSpecCand bucket candidates of every slice (its list starts at a fixed
  // offset) are loaded together with the counts, so a bucket that fits needs no second round trip.  Entries past a
  // list's length are loaded too (inside the slice's kScanWG entries) and dropped.
  constexpr int kSpecSlices = 16, kSpecCand = 64, kTps = NT / kSpecSlices, kEpt = kSpecCand / kTps;
  static_assert(NT % kSpecSlices == 0 && kSpecCand % kTps == 0, "candidate heads per thread");
  const bool spec = ns <= kSpecSlices;
  const int spec_sl = tid / kTps, spec_e0 = (tid % kTps) * kEpt;
  uint32_t sk[kEpt];
  int sp[kEpt];
  if (spec && spec_sl < ns)
#pragma unroll
    for (int k = 0; k < kEpt; ++k) {
      sk[k] = ekb[spec_sl * kScanWG + spec_e0 + k];
      sp[k] = epb[spec_sl * kScanWG + spec_e0 + k];
    }
  // Slice offsets of both lists: thread t owns slices [t per, t per + per).
  constexpr int kPer = kMaxSlices / NT;
  const int per = (ns + NT - 1) / NT;
  const int sbase = tid * per;
  uint32_t gc[kPer], ec[kPer], g = 0, e = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int sl = sbase + k;
    gc[k] = k < per && sl < ns ? (uint32_t)a.gcnt[b * a.nb + sl] : 0u;
    ec[k] = k < per && sl < ns ? (uint32_t)a.ecnt[b * a.nb + sl] : 0u;
    g += gc[k];
    e += ec[k];
  }
  uint32_t n_gt, ncand;
  uint32_t go = block_excl_scan<NT>(g, sh.red, &n_gt);
  uint32_t eo = block_excl_scan<NT>(e, sh.red, &ncand);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int sl = sbase + k;
    if (k < per && sl < ns) {
      sh.goff[sl] = go;
      sh.eoff[sl] = eo;
    }
    go += gc[k];
    eo += ec[k];
  }
  if (tid == 0) {
    sh.goff[ns] = n_gt;
    sh.eoff[ns] = ncand;
  }
  lds_barrier();
  // Positions above the bucket: loaded now, emitted once the bucket's picks are known too, so that a window that
  // also refines the bucket does so while these loads fly (the refine's barriers wait for LDS only).
  constexpr int kGPer = (W + NT - 1) / NT;
  const int gend = min(hi, (int)min(n_gt, (uint32_t)kTopK));
  int gpos[kGPer];
#pragma unroll
  for (int k = 0; k < kGPer; ++k) {
    const int s = lo + tid + k * NT;
    if (s < gend) {
      const int sl = slice_of(sh.goff, ns, (uint32_t)s);
      gpos[k] = glb[sl * kScanWG + (s - (int)sh.goff[sl])];
    }
  }
  auto emit_above = [&]() {
#pragma unroll
    for (int k = 0; k < kGPer; ++k) {
      const int s = lo + tid + k * NT;
      if (s < gend) emit(s, gpos[k]);
    }
  };
  if (n_gt >= (uint32_t)hi) {                                 // the window holds no pick from the bucket
    emit_above();
    return kTopK;
  }
  // The bucket's candidates in position order.
  const bool in_lds = ncand <= (uint32_t)CAND;
  if (in_lds) {
    if (spec && spec_sl < ns) {
      const uint32_t e0 = sh.eoff[spec_sl], elen = sh.eoff[spec_sl + 1] - e0;
#pragma unroll
      for (int k = 0; k < kEpt; ++k)
        if ((uint32_t)(spec_e0 + k) < elen) {
          sh.cand_key[e0 + spec_e0 + k] = sk[k];
          sh.cand_pos[e0 + spec_e0 + k] = sp[k];
        }
    }
    for (uint32_t c = tid; c < ncand; c += NT) {
      const int sl = slice_of(sh.eoff, ns, c);
      const uint32_t o = c - sh.eoff[sl];
      if (spec && o < (uint32_t)kSpecCand) continue;            // placed from the heads above
      sh.cand_key[c] = ekb[sl * kScanWG + o];
      sh.cand_pos[c] = epb[sl * kScanWG + o];
    }
  }
  auto gcand = [&](int c, uint32_t& key, int& pos) {
    const int sl = slice_of(sh.eoff, ns, (uint32_t)c);
    const size_t o = (size_t)sl * kScanWG + (c - sh.eoff[sl]);
    key = ekb[o];
    pos = epb[o];
  };
  lds_barrier();                                              // the candidates in LDS
  // The refine, instantiated separately for candidates in LDS and in the global lists, so that the LDS form never
  // waits for a global load of the other form (a merged form shares registers and waits between them).
  auto refine = [&](auto LDS) -> int {
    constexpr bool kLds = decltype(LDS)::value;
    // b1 from the first candidate (the bucket is non-empty: at least one pick comes from it).
    uint32_t key0;
    int pos0;
    if constexpr (kLds) key0 = sh.cand_key[0];
    else gcand(0, key0, pos0);
    const uint32_t b1 = key0 >> 19;
    const uint32_t need = kTopK - n_gt;                       // picks to make from the bucket (>= 1)
    // Candidate walk over thread-contiguous ranges of the ordered candidate list.
    const int cper = (int)((ncand + NT - 1) / NT);
    const int c_lo = min((int)ncand, tid * cper), c_hi = min((int)ncand, c_lo + cper);
    auto for_each = [&](auto&& f) {
      for (int c = c_lo; c < c_hi; ++c) {
        if constexpr (kLds) {
          f(sh.cand_key[c], sh.cand_pos[c]);
        } else {
          uint32_t key;
          int pos;
          gcand(c, key, pos);
          f(key, pos);
        }
      }
    };
    for_each([&](uint32_t key, int) { atomicAdd(&sh.hist[(key >> 8) & 0x7FF], 1u); });
    lds_barrier();
    find_threshold<NT, 2048>(sh.hist, need, sh.red, sh.thr);
    const uint32_t b2 = sh.thr[0];
    const uint32_t need2 = sh.thr[1];
    for_each([&](uint32_t key, int) {
      if (((key >> 8) & 0x7FF) == b2) atomicAdd(&sh.hist3[key & 0xFF], 1u);
    });
    lds_barrier();
    find_threshold<NT, kH3>(sh.hist3, need2, sh.red, sh.thr);
    const uint32_t T = (b1 << 19) | (b2 << 8) | sh.thr[0];
    const uint32_t need_eq = sh.thr[1];
    // Bucket picks: keys above T, then the first need_eq keys equal to T in position order.  With the candidates
    // in LDS (at most CAND < 2^16 of them) both counts travel in one scan, 16 bits each.
    uint32_t c_above = 0, c_tie = 0, above_total, tie_total, o_above, o_tie;
    for_each([&](uint32_t key, int) { c_above += key > T; c_tie += key == T; });
    if constexpr (kLds) {
      static_assert(CAND < 65536, "16-bit packed counts");
      uint32_t tot;
      const uint32_t o = block_excl_scan<NT>(c_above | (c_tie << 16), sh.red, &tot);
      o_above = o & 0xFFFFu;
      o_tie = o >> 16;
      above_total = tot & 0xFFFFu;
      tie_total = tot >> 16;
    } else {
      o_above = block_excl_scan<NT>(c_above, sh.red, &above_total);
      o_tie = block_excl_scan<NT>(c_tie, sh.red, &tie_total);
    }
    for_each([&](uint32_t key, int p) {
      if (key > T) {
        const uint32_t slot = n_gt + o_above++;
        if (slot >= (uint32_t)lo && slot < (uint32_t)hi && slot < (uint32_t)kTopK) emit((int)slot, p);
      } else if (key == T) {
        const uint32_t slot = n_gt + above_total + o_tie;
        if (o_tie < need_eq && slot >= (uint32_t)lo && slot < (uint32_t)hi && slot < (uint32_t)kTopK)
          emit((int)slot, p);
        ++o_tie;
      }
    });
    return kTopK;
  };
  const int count = in_lds ? refine(BoolC<true>{}) : refine(BoolC<false>{});
  emit_above();
  return count;
}

// Leaves request b's histograms zero for the next call, after the indexer ran: fine bins [fine0, fine1) and the
// coarse bins they make up, by nthr threads.
__device__ __forceinline__ void clear_histograms(const DsaArgs& a, int b, int fine0, int fine1, int tid, int nthr) {
  if (a.L <= kTopK) return;
  for (int c = 0; c < a.hcopies; ++c) {
    uint32_t* gh = fine_hist(a, b, c);
    for (int i = fine0 + tid; i < fine1; i += nthr) gh[i] = 0;
  }
  for (int i = fine0 / 32 + tid; i < fine1 / 32; i += nthr) a.chist[(size_t)b * kCBins + i] = 0;
}

// The whole selection of one request (one 1024-thread workgroup): idx, cnt, and the histograms left zero.  Used by
// the indexer-select entry; the decode entry lets every attention workgroup select its own chunk instead.
__global__ __launch_bounds__(1024) void dsa_select_final_kernel(DsaArgs a) {
  __shared__ SelectShared<kCand> sh;
  const int b = blockIdx.x, tid = threadIdx.x;
  int* idx = a.idx + (size_t)b * kTopK;
  const int cnt = select_window<1024, kTopK>(a, sh, b, 0, kTopK, [&](int s, int p) { idx[s] = p; });
  clear_histograms(a, b, 0, kBins, tid, 1024);
  if (tid == 0) a.cnt[b] = cnt;
}

// Zero-fills request b's histograms before the indexer accumulates into them (when they are not in the head), by NT
// threads (NT >= kCBins).
template <int NT>
__device__ __forceinline__ void hist_zero_item(const DsaArgs& a, int b) {
  static_assert(NT >= kCBins, "one coarse bin per thread");
  for (int c = 0; c < a.hcopies; ++c) {
    uint32_t* gh = fine_hist(a, b, c);
    for (int i = threadIdx.x; i < kBins; i += NT) gh[i] = 0;
  }
  if (threadIdx.x < kCBins) a.chist[(size_t)b * kCBins + threadIdx.x] = 0;
}

__global__ __launch_bounds__(1024) void dsa_hist_zero_kernel(DsaArgs a) { hist_zero_item<1024>(a, blockIdx.x); }

// ------------------------------------------------------------------------------------------------ sparse MLA
// Workgroup = (request b, block of 32 heads, chunk of 128 selected keys); 4 waves.  Wave w computes the share of
// the S^T tile over QK dims [144w, 144w+144) and the four shares are summed through LDS in a fixed order, so all
// four waves hold bit-identical scores, softmax state and P; wave w owns the value dims [128w, 128w+128) of O.
// The selected latent rows of the chunk's four 32-key tiles are gathered by direct-to-LDS buffer loads into three
// stages: tiles 0-2 are requested before the first tile is computed and tile 3 replaces tile 0.  In a stage,
// row r starts at byte r * kLatStride: 1152 bytes of the row plus 16 of padding, so the 73-chunk stride is odd and
// 16 consecutive rows at one chunk fall on 16 distinct bank groups (conflict-free K-operand reads).  DMA block j
// (0 <= j < 37) fills stage bytes [1024j, 1024j + 1024): lane i's 16 bytes go to slot 64j + i, which is chunk
// (slot % 73) of row (slot / 73); padding slots and slots past the 32 rows take copies of real chunks.  Wave w
// fills blocks w + 4q (q < 9) and all four waves fill block 36 with the same bytes, so every wave issues exactly
// kLatPerWave loads per tile.  V^T is read from the same rows with the transposing LDS read.
constexpr int kSSlot = 16 * 64;          // floats of one wave's share of an S^T tile
constexpr int kLatChunks = kDK / 8;      // 72 chunks of 16 bytes per latent row
constexpr int kLatStride = (kLatChunks + 1) * 16;           // 1168 bytes
constexpr int kLatInstr = 37;            // DMA blocks per tile (>= 32 * 73 / 64 slots)
constexpr int kLatPerWave = 10;          // DMA loads per wave and tile
constexpr int kLatStageBytes = kLatInstr * 1024;
constexpr int kLatStages = 3;                                // tile 3 of a chunk reuses stage 0
constexpr int kQkSteps = kDK / 16 / 4;                       // QK k-steps of one wave (a quarter of the 576 dims)
static_assert(kLatInstr * 64 >= kTile * (kLatChunks + 1) && kLatInstr == 4 * (kLatPerWave - 1) + 1,
              "a stage holds 32 padded rows; block 36 is shared");
// The gather addresses a request's rows by 32-bit offsets from one buffer resource, and an offset of 2^31 (past
// every row) reads zeros: the source of every key past the selected count.
constexpr int64_t kMaxAttnL = ((int64_t)1 << 31) / (kDK * 2) - 1;
constexpr uint32_t kZeroOffset = 0x80000000u;

__device__ __forceinline__ int lat_block(int w, int q) { return q < kLatPerWave - 1 ? w + 4 * q : kLatInstr - 1; }

// The kLatPerWave DMA loads of wave w for the tile at key0.  The selected positions are read from LDS first, all
// ten together, so the loads issue back to back.
__device__ __forceinline__ void dsa_issue_rows(char* __restrict__ stage, __amdgpu_buffer_rsrc_t rows,
                                               const int* __restrict__ sidx, int kbeg, int kend, int key0,
                                               const int (&drow)[10], const int (&dchk)[10], int w) {
  int pos[kLatPerWave];
#pragma unroll
  for (int q = 0; q < kLatPerWave; ++q) pos[q] = sidx[key0 - kbeg + drow[q]];   // < kChunk: key0 - kbeg <= 96
#pragma unroll
  for (int q = 0; q < kLatPerWave; ++q) {
    const uint32_t off = key0 + drow[q] < kend ? (uint32_t)pos[q] * (kDK * 2) + 16 * dchk[q] : kZeroOffset;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rows, VMK_LPTR(stage + lat_block(w, q) * 1024), 16, off, 0, 0, 0);
  }
}

// This wave's share of S^T for the tile in stage: QK dims 144w .. 144w + 143 (k-steps 9w .. 9w + 8), nine MFMAs in
// the same order in every workgroup.  The nine K operands are read from LDS before the first MFMA.
template <class V>
__device__ __forceinline__ floatx16 dsa_qk_part(const char* __restrict__ stage, const V (&qb)[kQkSteps], int r,
                                                int g, int w) {
  const char* kb = stage + r * kLatStride + (2 * kQkSteps * w + g) * 16;
  u32x4 k[kQkSteps];
#pragma unroll
  for (int j = 0; j < kQkSteps; ++j) k[j] = *reinterpret_cast<const u32x4*>(kb + 2 * j * 16);
  floatx16 s = floatx16{};
#pragma unroll
  for (int j = 0; j < kQkSteps; ++j) s = mfma32(as_v8<V>(k[j]), qb[j], s);
  return s;
}

// Full S^T from the four waves' shares: each wave stores its share in its slot of sred (register-major, so every
// 16-byte access of a wave covers 1 KB contiguously), and after the barrier every wave adds the four slots in the
// order 0, 1, 2, 3, so all waves hold bit-identical scores.
__device__ __forceinline__ floatx16 dsa_reduce_s(float* __restrict__ sred, const floatx16& part, int lane, int w) {
#pragma unroll
  for (int i4 = 0; i4 < 4; ++i4)
    *reinterpret_cast<floatx4*>(sred + w * kSSlot + (i4 * 64 + lane) * 4) =
        floatx4{part[4 * i4], part[4 * i4 + 1], part[4 * i4 + 2], part[4 * i4 + 3]};
  lds_barrier();
  floatx16 s;
#pragma unroll
  for (int v = 0; v < 4; ++v)
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const floatx4 x = *reinterpret_cast<const floatx4*>(sred + v * kSSlot + (i4 * 64 + lane) * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) s[4 * i4 + e] = v == 0 ? x[e] : s[4 * i4 + e] + x[e];
    }
  return s;
}

// O^T += V^T . P^T over this wave's 128 value dims.  V^T operand of (d-tile dt, step tt): source lane l addresses
// key 16tt + 8rr + 4g + ((l & 15) >> 2) at value dim 128w + 32dt + 16((l >> 4) & 1) + 4(l & 3); the transposed read
// gives lane l the dim 128w + 32dt + (l & 31) of the four keys 16tt + 8rr + 4g + e, e = 0..3, the keys of P^T's
// elements 4rr..4rr+3.
template <class V>
__device__ __forceinline__ void dsa_pv(RowState& st, const char* __restrict__ stage, const V (&pb)[2], int lane,
                                       int w) {
  const int g = lane >> 5, e = (lane & 15) >> 2, hc = (lane >> 4) & 1, a4 = lane & 3;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      u32x2 part[2];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int row = 16 * tt + 8 * rr + 4 * g + e;
        const int col = 128 * w + 32 * dt + 16 * hc + 4 * a4;         // halfs
        part[rr] = lds_read_tr16(stage + row * kLatStride + (col >> 3) * 16 + (col & 7) * 2);
      }
      const V va = as_v8<V>(u32x4{part[0][0], part[0][1], part[1][0], part[1][1]});
      st.o[dt] = mfma32(va, pb[tt], st.o[dt]);
    }
}

// s_waitcnt vmcnt(n) as the compiler's own builtin (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt
// left at their maxima), so that the compiler's wait insertion knows which loads are complete after it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One tile: this wave's QK share, the cross-wave sum of S^T, masked online softmax (identical in every wave), PV
// over this wave's value dims.
template <class V>
__device__ __forceinline__ void dsa_tile(RowState& st, const V (&qb)[kQkSteps], const char* __restrict__ stage,
                                         float* __restrict__ sred, int key0, int kend, float sl2, int lane, int w) {
  const int r = lane & 31, g = lane >> 5;
  floatx16 s = dsa_reduce_s(sred, dsa_qk_part(stage, qb, r, g, w), lane, w);
  if (key0 + kTile > kend)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key0 + 8 * blk + 4 * g + c >= kend) s[4 * blk + c] = kNegInf;
  V pb[2];
  softmax_update(st, s, sl2, pb);
  dsa_pv(st, stage, pb, lane, w);
}

// Walk over the chunk's four tiles through three stages: tiles 0-2 are requested up front (rows past kend read
// zeros) and tile 3 goes into stage 0 once every wave has finished tile 0 (the barrier before tile 1).  Before a tile
// a wave waits until only its loads of later tiles are in flight, i.e. its part of this tile (and every older load,
// such as the Q operands) has landed, and the barrier makes every wave's part visible.  The stages are separate LDS
// arrays and every LDS array the walk touches is a restrict-qualified parameter, so the compiler can tell them apart
// (it would otherwise wait for every load in flight before each LDS read).  The last wait drains every load, so no
// DMA is still writing LDS when the workgroup ends.
template <class V>
__device__ __forceinline__ void dsa_chunk_walk(char* __restrict__ st0, char* __restrict__ st1, char* __restrict__ st2,
                                               float* __restrict__ sred, RowState& st, const V (&qb)[kQkSteps],
                                               __amdgpu_buffer_rsrc_t rows, const int* __restrict__ sidx, int kbeg,
                                               int kend, int ntiles, const int (&drow)[10], const int (&dchk)[10],
                                               float sl2, int lane, int w) {
  static_assert(kLatStages == 3 && kChunk == 4 * kTile && 2 * kLatPerWave < 64, "three stages, vmcnt range");
  dsa_issue_rows(st0, rows, sidx, kbeg, kend, kbeg, drow, dchk, w);
  dsa_issue_rows(st1, rows, sidx, kbeg, kend, kbeg + kTile, drow, dchk, w);
  dsa_issue_rows(st2, rows, sidx, kbeg, kend, kbeg + 2 * kTile, drow, dchk, w);
  if (ntiles > 0) {
    wait_vmcnt<2 * kLatPerWave>();
    lds_barrier();
    dsa_tile(st, qb, st0, sred, kbeg, kend, sl2, lane, w);
  }
  if (ntiles > 1) {
    wait_vmcnt<kLatPerWave>();
    lds_barrier();                              // every wave is done with stage 0
    if (ntiles > 3) dsa_issue_rows(st0, rows, sidx, kbeg, kend, kbeg + 3 * kTile, drow, dchk, w);
    dsa_tile(st, qb, st1, sred, kbeg + kTile, kend, sl2, lane, w);
  }
  if (ntiles > 3) {
    wait_vmcnt<kLatPerWave>();
  } else {
    wait_vmcnt<0>();
  }
  if (ntiles > 2) {
    lds_barrier();
    dsa_tile(st, qb, st2, sred, kbeg + 2 * kTile, kend, sl2, lane, w);
  }
  wait_vmcnt<0>();
  if (ntiles > 3) {
    lds_barrier();
    dsa_tile(st, qb, st0, sred, kbeg + 3 * kTile, kend, sl2, lane, w);
  }
}

// One attention item = (request b, head block hb, chunk), item = (b * 4 + hb) * kNChunk + chunk, by 256 threads.
template <class V>
__device__ __forceinline__ void attn_item(const DsaArgs& a, int item, char* __restrict__ st0,
                                          char* __restrict__ st1, char* __restrict__ st2, float* __restrict__ sred,
                                          int* __restrict__ sidx, SelectShared<kCandAttn>& sel) {
  const int chunk = item % kNChunk;
  const int hb = (item / kNChunk) % 4;
  const int b = item / (kNChunk * 4);
  const int kbeg = chunk * kChunk;
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 31, g = lane >> 5;

  // Q^T operand of this wave's k-step j: head r's dims 16c + 8g .. 16c + 8g + 7 with c = 9w + j (chunk 2c + g of
  // the query row).
  const f16* qrow = a.q + ((size_t)b * kH + hb * 32 + r) * kDK + 16 * kQkSteps * w + 8 * g;
  V qb[kQkSteps];
#pragma unroll
  for (int j = 0; j < kQkSteps; ++j) qb[j] = as_v8<V>(ld16(qrow + 16 * j));

  // The chunk's selected positions.  Decode entry: the workgroup selects them itself from select_scan's lists
  // (select_window, the same picks as select_final's), and the workgroups of head block 0 write idx, cnt and clear
  // their share of the histograms.  Sparse-attention entry: idx holds kTopK entries per request, so every thread
  // loads one without waiting for the count (entries past it are masked below).  No branch depends on the count: a
  // chunk past it (lens, or L < kTopK) runs no tiles and writes an empty partial, which the combine does not read.
  int cnt;
  if (a.fused_select) {
    int* idxo = a.idx + (size_t)b * kTopK;
    cnt = select_window<256, kChunk>(a, sel, b, kbeg, kbeg + kChunk, [&](int s, int p) {
      sidx[s - kbeg] = p;
      if (hb == 0) idxo[s] = p;
    });
    if (hb == 0) {
      clear_histograms(a, b, chunk * (kBins / kNChunk), (chunk + 1) * (kBins / kNChunk), threadIdx.x, 256);
      if (chunk == 0 && threadIdx.x == 0) a.cnt[b] = cnt;
    }
    lds_barrier();                              // sidx; the Q loads and the idx and histogram stores stay in flight
    // Clamped into the cache; keys past kend read the zero row whatever their entry holds.
    if (threadIdx.x < kChunk) sidx[threadIdx.x] = min(max(sidx[threadIdx.x], 0), a.L - 1);
  } else {
    const int* ip = a.idx + (size_t)b * kTopK;
    const int sl = ip[kbeg + (int)(threadIdx.x & (kChunk - 1))];
    cnt = min(max(a.cnt[b], 0), kTopK);                // a caller's count outside [0, kTopK] is clamped
    // Threads t and t + kChunk store the same value.
    sidx[threadIdx.x & (kChunk - 1)] = min(max(sl, 0), a.L - 1);
  }
  const int kend = max(kbeg, min(cnt, kbeg + kChunk));
  const int ntiles = (kend - kbeg + kTile - 1) / kTile;

  // This wave's DMA loads q (block lat_block(w, q)): the (row, chunk) its lane fetches for each.
  int drow[kLatPerWave], dchk[kLatPerWave];
#pragma unroll
  for (int q = 0; q < kLatPerWave; ++q) {
    const int slot = 64 * lat_block(w, q) + lane;
    const int rr = slot / (kLatChunks + 1), cc = slot % (kLatChunks + 1);
    drow[q] = rr < kTile ? rr : kTile - 1;
    dchk[q] = (rr < kTile && cc < kLatChunks) ? cc : 0;
  }
  lds_barrier();                                // sidx; waits for LDS only, the Q loads stay in flight
  const __amdgpu_buffer_rsrc_t rows =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(a.kv + (size_t)b * a.L * kDK), 0, a.L * kDK * 2, 0x00020000);
  RowState st;
  row_state_init(st);
  dsa_chunk_walk(st0, st1, st2, sred, st, qb, rows, sidx, kbeg, kend, ntiles, drow, dchk, a.sl2, lane, w);
  // Partial: O[head][128w + d'] / l for this wave's value dims, in the partial type; m and l are identical in all
  // waves.  The wave's 32 x 128 block goes through LDS (stages 0 and 1 are free once every wave is past its last
  // tile), row r's 16-byte chunk c at position (c + r) & 31, so that every store instruction writes two whole pieces
  // of rows instead of pieces of 32 rows.
  const float ltot = st.l + xor32(st.l);
  const float inv = part_inv(ltot);
  __syncthreads();
  float* lds = reinterpret_cast<float*>(w < 2 ? st0 : st1) + (w & 1) * 32 * 128;
  static_assert(2 * 32 * 128 * 4 <= kLatStageBytes, "two waves' blocks per stage");
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
      *reinterpret_cast<floatx4*>(lds + r * 128 + (((dt * 8 + 2 * blk + g) + r) & 31) * 4) =
          floatx4{st.o[dt][4 * blk], st.o[dt][4 * blk + 1], st.o[dt][4 * blk + 2], st.o[dt][4 * blk + 3]} * inv;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");       // the wave reads back only its own block
  part_t<elem_t<V>>* po = reinterpret_cast<part_t<elem_t<V>>*>(a.po) + (size_t)item * 32 * kDC + 128 * w;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 2 * i + g;
    store_part4(po + row * kDC + r * 4, *reinterpret_cast<const floatx4*>(lds + row * 128 + ((r + row) & 31) * 4));
  }
  if (w == 0 && g == 0) {
    a.pml[((size_t)item * 32 + r) * 2] = st.m;
    a.pml[((size_t)item * 32 + r) * 2 + 1] = ltot;
  }
}

template <class V>
__global__ __launch_bounds__(256) void dsa_attn_kernel(DsaArgs a) {
  __shared__ __attribute__((aligned(16))) char st0[kLatStageBytes], st1[kLatStageBytes], st2[kLatStageBytes];
  __shared__ __attribute__((aligned(16))) float sred[4 * kSSlot];
  __shared__ int sidx[kChunk];
  __shared__ SelectShared<kCandAttn> sel;
  attn_item<V>(a, blockIdx.x, st0, st1, st2, sred, sidx, sel);
}

// One workgroup (256 threads, 2 value dims each) per (b, head): LSE merge over the chunks; E is the output type.
template <class E>
__device__ __forceinline__ void combine_item(const DsaArgs& a, int bh) {
  const int b = bh / kH, head = bh % kH, hb = head / 32, hr = head % 32;
  const int cnt = min(max(a.cnt[b], 0), kTopK);     // as in dsa_attn_kernel; cnt = 0 merges no chunk (NaN)
  const int nch = (cnt + kChunk - 1) / kChunk;
  const size_t item0 = ((size_t)b * 4 + hb) * kNChunk;
  typedef part_t<E> PT;
  combine_row<256, 2, PT>(nch,
                          [&](int c, const float*& ml, const PT*& o) {
                            const size_t base = (item0 + c) * 32 + hr;
                            ml = a.pml + base * 2;
                            o = reinterpret_cast<const PT*>(a.po) + base * kDC;
                          },
                          reinterpret_cast<E*>(a.out) + (size_t)bh * kDC);
}

template <class E>
__global__ __launch_bounds__(256) void dsa_combine_kernel(DsaArgs a) {
  combine_item<E>(a, blockIdx.x);
}

// ------------------------------------------------------------------------------------------------ single launch
// The whole decode (indexer, select_scan, attention with its own selection, combine) in one launch of at most one
// 256-thread workgroup per CU, every workgroup taking the items of each phase in turn (item = workgroup id, then
// + grid size), with a grid barrier between phases.  The phases are the four-launch chain's item bodies, except the
// indexer, which runs as 4 waves with 4-stage rings (the same arithmetic per position; the chain uses 8 waves with
// 2-stage rings), so the outputs are bit-identical to vmk_dsa_decode's.
// Grid barrier k: every workgroup makes its stores visible to the device (agent-scope release: every wave's stores
// are complete at the workgroup barrier before it, then the L2 is written back), adds 1 to counter k, and waits
// until the counter reaches the grid size, then acquires (L1 and L2 invalidated) before anyone reads what other
// workgroups wrote.  The wait is bounded: after kSyncSpinLimit polls the workgroup sets the timeout flag and goes
// on, and a set flag ends every other wait; the call then reports cnt[b] = -1 for every request, and so does every
// later call on that workspace (the flag is sticky) until its head is zeroed again.  Counters return to zero within
// the call: workgroup 0 clears counter k - 1 once barrier k is complete, and the last workgroup to finish clears the
// last barrier's counter and the exit counter.
constexpr int kSyncLine = 64;                    // uint32 per 256-byte counter line
constexpr int kMaxSyncBarriers = 4;              // histogram zero-fill, indexer, select_scan, attention
constexpr int kSyncExit = kMaxSyncBarriers;      // line of the exit counter
constexpr int kSyncFlag = kMaxSyncBarriers + 1;  // line of the timeout flag
constexpr uint32_t kSyncSpinLimit = 1u << 17;    // polls of about 1 us: a wait gives up after ~0.1-0.2 s
constexpr int kFusedIdxWaves = 4, kFusedIdxStages = 4;

// LDS of the single launch: one pool that every phase carves up in turn.
constexpr int kFusedAttnSred = 3 * kLatStageBytes;
constexpr int kFusedAttnSidx = kFusedAttnSred + 4 * kSSlot * 4;
constexpr int kFusedAttnSel = kFusedAttnSidx + kChunk * 4;
constexpr int kFusedAttnEnd = kFusedAttnSel + (int)sizeof(SelectShared<kCandAttn>);
constexpr int kFusedIdxHist = kFusedIdxWaves * kFusedIdxStages * kIdxStageBytes;
constexpr int kFusedIdxChist = kFusedIdxHist + kBins / 2 * 4;
constexpr int kFusedIdxEnd = kFusedIdxChist + kCBins * 4;
constexpr int kFusedPool = kFusedAttnEnd > kFusedIdxEnd ? kFusedAttnEnd : kFusedIdxEnd;
static_assert(kFusedAttnSel % 16 == 0 && kFusedIdxHist % 16 == 0 && (int)sizeof(ScanShared) <= kFusedPool,
              "pool layout");

__device__ __forceinline__ uint32_t* sync_line(const DsaArgs& a, int k) { return a.sync + k * kSyncLine; }

// Grid barrier k of the single launch (every thread of every workgroup calls it); *timed_out (LDS) becomes 1 when
// this workgroup's wait gave up or saw the flag.
__device__ __forceinline__ void grid_sync(const DsaArgs& a, int k, uint32_t nblocks, int* timed_out) {
  __syncthreads();                                 // every wave's stores are complete (vmcnt(0) before s_barrier)
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    uint32_t* c = sync_line(a, k);
    uint32_t* flag = sync_line(a, kSyncFlag);
    __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int gave_up = 0;
    uint32_t spins = 0;
    while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < nblocks) {
      if ((spins & 31) == 31 && __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
        gave_up = 1;
        break;
      }
      if (++spins >= kSyncSpinLimit) {
        __hip_atomic_fetch_or(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gave_up = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (!gave_up && k > 0 && blockIdx.x == 0)      // every workgroup has left barrier k - 1's wait
      __hip_atomic_fetch_and(sync_line(a, k - 1), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (gave_up) *timed_out = 1;
  }
  __syncthreads();
}

template <class V>
__global__ __launch_bounds__(256) void dsa_decode_single_kernel(DsaArgs a) {
  __shared__ __attribute__((aligned(16))) char pool[kFusedPool];
  __shared__ int timed_out;
  typedef elem_t<V> E;
  const uint32_t G = gridDim.x;
  if (threadIdx.x == 0)
    timed_out = __hip_atomic_load(sync_line(a, kSyncFlag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
  __syncthreads();
  if (timed_out) {                                 // an earlier call's wait gave up: report it and do nothing
    if (blockIdx.x == 0)
      for (int b = threadIdx.x; b < a.B; b += 256) a.cnt[b] = -1;
    return;
  }
  int k = 0;
  if (a.L > kTopK) {
    if (!a.hist_in_head) {
      for (int it = blockIdx.x; it < a.B; it += G) hist_zero_item<256>(a, it);
      grid_sync(a, k++, G, &timed_out);
    }
    const int nblk = (a.L + kIdxWG - 1) / kIdxWG;
    for (int it = blockIdx.x; it < a.B * nblk; it += G) {
      indexer_item<V, kFusedIdxWaves, kFusedIdxStages>(a, it % nblk, it / nblk, pool,
                                                       reinterpret_cast<uint32_t*>(pool + kFusedIdxHist),
                                                       reinterpret_cast<uint32_t*>(pool + kFusedIdxChist));
      __syncthreads();
    }
    grid_sync(a, k++, G, &timed_out);
    for (int it = blockIdx.x; it < a.B * a.nb; it += G) {
      select_scan_item(a, it % a.nb, it / a.nb, *reinterpret_cast<ScanShared*>(pool));
      __syncthreads();
    }
    grid_sync(a, k++, G, &timed_out);
  }
  for (int it = blockIdx.x; it < a.B * 4 * kNChunk; it += G) {
    attn_item<V>(a, it, pool, pool + kLatStageBytes, pool + 2 * kLatStageBytes,
                 reinterpret_cast<float*>(pool + kFusedAttnSred), reinterpret_cast<int*>(pool + kFusedAttnSidx),
                 *reinterpret_cast<SelectShared<kCandAttn>*>(pool + kFusedAttnSel));
    __syncthreads();
  }
  grid_sync(a, k++, G, &timed_out);
  for (int it = blockIdx.x; it < a.B * kH; it += G) {
    combine_item<E>(a, it);
    __syncthreads();
  }
  // Exit: the last workgroup out clears the last barrier's counter and the exit counter.
  if (threadIdx.x == 0) {
    if (!timed_out) {
      const uint32_t old =
          __hip_atomic_fetch_add(sync_line(a, kSyncExit), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == G - 1) {
        __hip_atomic_fetch_and(sync_line(a, k - 1), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_and(sync_line(a, kSyncExit), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (__hip_atomic_load(sync_line(a, kSyncFlag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) timed_out = 1;
  }
  __syncthreads();
  if (timed_out)
    for (int b = threadIdx.x; b < a.B; b += 256) a.cnt[b] = -1;
}

// The single-launch decode's grid-barrier block in the workspace head's counter part, past the coarse histograms
// (B * 1 KB <= 64 KB when they live there): one 256-byte line per counter, then the timeout flag.
constexpr size_t kSyncOffset = kWsCounters + ((size_t)1 << 20);

struct DsaLayout {
  size_t hist, chist, scores, glist, ekey, epos, gcnt, ecnt, po, pml, total;
  bool hist_in_head;
  int hcopies;
};

// The per-request histograms live in the zero-invariant workspace head when they fit (B <= 64: fine histograms in
// its histogram part, coarse ones in its counter part); otherwise in the data region, zero-filled by a launch.
static DsaLayout dsa_layout(int64_t B, int64_t L) {
  DsaLayout l;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  // Fine-histogram copies per request: two while they fit in the head's histogram part (B <= 32; C5: 42.3 us against
  // 43.7 with 8 copies, 44.5 with one, and 46.6 with 16, whose clearing costs more than it saves), else one.
  l.hcopies = (int)std::max<int64_t>(1, std::min<int64_t>(kMaxFineCopies,
                                                           (int64_t)(kWsCounters / ((size_t)B * kBins * 4))));
  size_t hist_bytes = (size_t)B * l.hcopies * kBins * 4;
  l.hist_in_head = hist_bytes <= kWsCounters;
  if (!l.hist_in_head) {
    l.hcopies = 1;
    hist_bytes = (size_t)B * kBins * 4;
  }
  size_t o = kWsHead;
  l.hist = l.hist_in_head ? 0 : o;
  if (!l.hist_in_head) o = up(o + hist_bytes);
  l.chist = l.hist_in_head ? kWsCounters : o;
  if (!l.hist_in_head) o = up(o + (size_t)B * kCBins * 4);
  const int64_t nb = (L + kScanWG - 1) / kScanWG;
  const size_t row = (size_t)B * nb * kScanWG * 4;     // rows padded to whole scan slices
  l.scores = o;            o = up(o + row);
  l.glist = o;             o = up(o + row);
  l.ekey = o;              o = up(o + row);
  l.epos = o;              o = up(o + row);
  l.gcnt = o;              o = up(o + (size_t)B * nb * 4);
  l.ecnt = o;              o = up(o + (size_t)B * nb * 4);
  l.po = o;                o = up(o + (size_t)B * 4 * kNChunk * 32 * kDC * 4);
  l.pml = o;               o = up(o + (size_t)B * 4 * kNChunk * 32 * 2 * 4);
  l.total = o + 256;
  return l;
}

static int dsa_fill_args(DsaArgs& a, const void* q, const void* kv, const void* iq, const void* ik, const void* w,
                         const void* lens, void* out, void* idx, void* cnt, int64_t B, int64_t L, void* ws) {
  const DsaLayout lay = dsa_layout(B, L);
  char* base = (char*)align_up(ws, 256);
  a.q = (const f16*)q; a.kv = (const f16*)kv; a.iq = (const f16*)iq; a.ik = (const f16*)ik; a.w = (const float*)w;
  a.lens = (const int*)lens; a.out = (f16*)out; a.idx = (int*)idx; a.cnt = (int*)cnt;
  a.hist = (uint32_t*)(base + lay.hist);
  a.chist = (uint32_t*)(base + lay.chist);
  a.scores = (float*)(base + lay.scores);
  a.glist = (int*)(base + lay.glist);
  a.ekey = (uint32_t*)(base + lay.ekey);
  a.epos = (int*)(base + lay.epos);
  a.gcnt = (int*)(base + lay.gcnt);
  a.ecnt = (int*)(base + lay.ecnt);
  a.po = base + lay.po;                              // sized for fp32 rows; fp16 partials use the first half
  a.pml = (float*)(base + lay.pml);
  a.B = (int)B; a.L = (int)L;
  a.nb = (int)((L + kScanWG - 1) / kScanWG);
  a.Ls = a.nb * kScanWG;
  a.hist_in_head = lay.hist_in_head ? 1 : 0;
  a.hcopies = lay.hcopies;
  a.fused_select = 0;
  a.scores_only = 0;
  a.scores_in = nullptr;
  a.sl2 = (float)(1.0 / sqrt(192.0)) * kLog2e;
  a.sync = (uint32_t*)(base + kSyncOffset);
  return 0;
}

// V: operand type of iq/ik (half8: fp16, bf16x8: bf16); the select works on fp32 scores.
template <class V>
static int launch_index_select(const DsaArgs& a, hipStream_t s, bool final_select) {
  if (a.L > kTopK) {
    if (!a.hist_in_head) {
      hipLaunchKernelGGL(dsa_hist_zero_kernel, dim3((unsigned)a.B), dim3(1024), 0, s, a);
      VMK_CHECK_HIP(hipGetLastError());
    }
    prof_before(kKDsaIndexer, s);
    hipLaunchKernelGGL(dsa_indexer_kernel<V>, dim3((unsigned)((a.L + kIdxWG - 1) / kIdxWG), (unsigned)a.B),
                       dim3(64 * kIdxWaves), 0, s, a);
    prof_after(kKDsaIndexer, s);
    VMK_CHECK_HIP(hipGetLastError());
    prof_before(kKDsaSelectScan, s);
    hipLaunchKernelGGL(dsa_select_scan_kernel, dim3((unsigned)a.nb, (unsigned)a.B), dim3(256), 0, s, a);
    prof_after(kKDsaSelectScan, s);
    VMK_CHECK_HIP(hipGetLastError());
  }
  if (final_select) {
    prof_before(kKDsaSelect, s);
    hipLaunchKernelGGL(dsa_select_final_kernel, dim3((unsigned)a.B), dim3(1024), 0, s, a);
    prof_after(kKDsaSelect, s);
    VMK_CHECK_HIP(hipGetLastError());
  }
  return 0;
}

// The select from caller scores (vmk_dsa_topk): scores into the workspace with the histograms, then the two select
// launches, as after the indexer.
static int launch_topk(const DsaArgs& a, hipStream_t s) {
  if (a.L > kTopK) {
    if (!a.hist_in_head) {
      hipLaunchKernelGGL(dsa_hist_zero_kernel, dim3((unsigned)a.B), dim3(1024), 0, s, a);
      VMK_CHECK_HIP(hipGetLastError());
    }
    hipLaunchKernelGGL(dsa_scores_hist_kernel, dim3((unsigned)(a.Ls / 1024), (unsigned)a.B), dim3(256), 0, s, a);
    VMK_CHECK_HIP(hipGetLastError());
    hipLaunchKernelGGL(dsa_select_scan_kernel, dim3((unsigned)a.nb, (unsigned)a.B), dim3(256), 0, s, a);
    VMK_CHECK_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(dsa_select_final_kernel, dim3((unsigned)a.B), dim3(1024), 0, s, a);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

// V: operand type of q/kv; the output has its element type.
template <class V>
static int launch_attention(const DsaArgs& a, hipStream_t s) {
  prof_before(kKDsaAttn, s);
  hipLaunchKernelGGL(dsa_attn_kernel<V>, dim3((unsigned)(a.B * 4 * kNChunk)), dim3(256), 0, s, a);
  prof_after(kKDsaAttn, s);
  VMK_CHECK_HIP(hipGetLastError());
  prof_before(kKDsaCombine, s);
  hipLaunchKernelGGL(dsa_combine_kernel<elem_t<V>>, dim3((unsigned)(a.B * kH)), dim3(256), 0, s, a);
  prof_after(kKDsaCombine, s);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

}  // namespace vmk

using namespace vmk;

extern "C" size_t vmk_dsa_workspace_size(int64_t B, int64_t L) {
  if (B <= 0 || L <= 0) return 0;
  return dsa_layout(B, L).total;
}

#define DSA_COMMON_CHECKS()                                                                    \
  VMK_CHECK(B > 0 && L > 0 && L <= (int64_t)kMaxSlices * kScanWG && B < (1 << 20), "bad B or L (L <= 4M)"); \
  VMK_CHECK(workspace && ws_bytes >= vmk_dsa_workspace_size(B, L),                             \
            "workspace too small (query vmk_dsa_workspace_size)")

template <class V>
static int dsa_indexer_select(const void* iq, const void* ik, const void* w, const void* lens, void* idx, void* cnt,
                              int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(iq && ik && w && idx && cnt, "null pointer argument");
  DSA_COMMON_CHECKS();
  VMK_CHECK(aligned16(iq) && aligned16(ik), "iq/ik must be 16-byte aligned");
  DsaArgs a;
  dsa_fill_args(a, nullptr, nullptr, iq, ik, w, lens, nullptr, idx, cnt, B, L, workspace);
  return launch_index_select<V>(a, (hipStream_t)stream, true);
}

// Indexer scores only: written into the caller's (B, L) buffer (row stride L), no histograms, so the workspace head
// stays zero.
template <class V>
static int dsa_indexer_only(const void* iq, const void* ik, const void* w, const void* lens, void* scores, int64_t B,
                            int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(iq && ik && w && scores, "null pointer argument");
  DSA_COMMON_CHECKS();
  VMK_CHECK(aligned16(iq) && aligned16(ik), "iq/ik must be 16-byte aligned");
  DsaArgs a;
  dsa_fill_args(a, nullptr, nullptr, iq, ik, w, lens, nullptr, nullptr, nullptr, B, L, workspace);
  a.scores = (float*)scores;
  a.Ls = (int)L;
  a.scores_only = 1;
  hipLaunchKernelGGL(dsa_indexer_kernel<V>, dim3((unsigned)((L + kIdxWG - 1) / kIdxWG), (unsigned)B),
                     dim3(64 * kIdxWaves), 0, (hipStream_t)stream, a);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

template <class V>
static int dsa_sparse_mla(const void* q, const void* kv, const void* idx, const void* cnt, void* out, int64_t B,
                          int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(q && kv && idx && cnt && out, "null pointer argument");
  DSA_COMMON_CHECKS();
  VMK_CHECK(aligned16(q) && aligned16(kv), "q/kv must be 16-byte aligned");
  VMK_CHECK(L <= kMaxAttnL, "sparse attention needs L * 1152 bytes < 2 GiB per request (L <= 1864134)");
  DsaArgs a;
  dsa_fill_args(a, q, kv, nullptr, nullptr, nullptr, nullptr, out, (void*)idx, (void*)cnt, B, L, workspace);
  return launch_attention<V>(a, (hipStream_t)stream);
}

template <class V>
static int dsa_decode(const void* q, const void* kv, const void* iq, const void* ik, const void* w, const void* lens,
                      void* out, void* idx, void* cnt, int64_t B, int64_t L, void* workspace, size_t ws_bytes,
                      void* stream) {
  VMK_CHECK(q && kv && iq && ik && w && out && idx && cnt, "null pointer argument");
  DSA_COMMON_CHECKS();
  VMK_CHECK(aligned16(q) && aligned16(kv) && aligned16(iq) && aligned16(ik), "tensors must be 16-byte aligned");
  VMK_CHECK(L <= kMaxAttnL, "sparse attention needs L * 1152 bytes < 2 GiB per request (L <= 1864134)");
  DsaArgs a;
  dsa_fill_args(a, q, kv, iq, ik, w, lens, out, idx, cnt, B, L, workspace);
  a.fused_select = 1;                                // the attention workgroups select their own chunks
  hipStream_t s = (hipStream_t)stream;
  if (int rc = launch_index_select<V>(a, s, false)) return rc;
  return launch_attention<V>(a, s);
}

// Workgroups of the single launch on the stream's device: at most one round of co-resident workgroups (the
// occupancy of its 256-thread, ~156 KB-LDS workgroup times the CU count, looked up once per device), and no more
// than the largest phase has items.
template <class V>
static int single_grid(hipStream_t s, int64_t items, int* grid) {
  constexpr int kDevs = 64;
  static int cap[kDevs];
  int dev = -1;
  if (s) {
    VMK_CHECK_HIP(hipStreamGetDevice(s, &dev));
  } else {
    VMK_CHECK_HIP(hipGetDevice(&dev));
  }
  VMK_CHECK(dev >= 0 && dev < kDevs, "device index beyond the single-launch table");
  if (!cap[dev]) {
    int cur = -1, per_cu = 0, cus = 0;
    VMK_CHECK_HIP(hipGetDevice(&cur));
    if (cur != dev) VMK_CHECK_HIP(hipSetDevice(dev));
    const hipError_t e1 = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, reinterpret_cast<const void*>(dsa_decode_single_kernel<V>), 256, 0);
    const hipError_t e2 = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cur != dev) VMK_CHECK_HIP(hipSetDevice(cur));
    VMK_CHECK_HIP(e1);
    VMK_CHECK_HIP(e2);
    VMK_CHECK(per_cu >= 1 && cus >= 1, "the single-launch kernel cannot be resident on this device");
    cap[dev] = per_cu * cus;
  }
  *grid = (int)std::min<int64_t>(items, cap[dev]);
  return 0;
}

template <class V>
static int dsa_decode_single(const void* q, const void* kv, const void* iq, const void* ik, const void* w,
                             const void* lens, void* out, void* idx, void* cnt, int64_t B, int64_t L,
                             void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(q && kv && iq && ik && w && out && idx && cnt, "null pointer argument");
  DSA_COMMON_CHECKS();
  VMK_CHECK(aligned16(q) && aligned16(kv) && aligned16(iq) && aligned16(ik), "tensors must be 16-byte aligned");
  VMK_CHECK(L <= kMaxAttnL, "sparse attention needs L * 1152 bytes < 2 GiB per request (L <= 1864134)");
  DsaArgs a;
  dsa_fill_args(a, q, kv, iq, ik, w, lens, out, idx, cnt, B, L, workspace);
  a.fused_select = 1;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nblk = (L + kIdxWG - 1) / kIdxWG;
  const int64_t items = std::max<int64_t>(L > kTopK ? B * nblk : 0, B * (int64_t)kH);
  int grid = 0;
  if (int rc = single_grid<V>(s, items, &grid)) return rc;
  prof_before(kKDsaSingle, s);
  hipLaunchKernelGGL(dsa_decode_single_kernel<V>, dim3((unsigned)grid), dim3(256), 0, s, a);
  prof_after(kKDsaSingle, s);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

extern "C" int vmk_dsa_decode_single(const void* q, const void* kv, const void* iq, const void* ik, const void* w,
                                     const void* lens, void* out, void* idx, void* cnt, int64_t B, int64_t L,
                                     void* workspace, size_t ws_bytes, void* stream) {
  return dsa_decode_single<half8>(q, kv, iq, ik, w, lens, out, idx, cnt, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_decode_single_bf16(const void* q, const void* kv, const void* iq, const void* ik,
                                          const void* w, const void* lens, void* out, void* idx, void* cnt,
                                          int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  return dsa_decode_single<bf16x8>(q, kv, iq, ik, w, lens, out, idx, cnt, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_indexer(const void* iq, const void* ik, const void* w, const void* lens, void* scores, int64_t B,
                               int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  return dsa_indexer_only<half8>(iq, ik, w, lens, scores, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_indexer_bf16(const void* iq, const void* ik, const void* w, const void* lens, void* scores,
                                    int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  return dsa_indexer_only<bf16x8>(iq, ik, w, lens, scores, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_topk(const void* scores, const void* lens, void* idx, void* cnt, int64_t B, int64_t L,
                            void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(scores && idx && cnt, "null pointer argument");
  DSA_COMMON_CHECKS();
  DsaArgs a;
  dsa_fill_args(a, nullptr, nullptr, nullptr, nullptr, nullptr, lens, nullptr, idx, cnt, B, L, workspace);
  a.scores_in = (const float*)scores;
  return launch_topk(a, (hipStream_t)stream);
}

extern "C" int vmk_dsa_indexer_select(const void* iq, const void* ik, const void* w, const void* lens, void* idx,
                                      void* cnt, int64_t B, int64_t L, void* workspace, size_t ws_bytes,
                                      void* stream) {
  return dsa_indexer_select<half8>(iq, ik, w, lens, idx, cnt, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_indexer_select_bf16(const void* iq, const void* ik, const void* w, const void* lens, void* idx,
                                           void* cnt, int64_t B, int64_t L, void* workspace, size_t ws_bytes,
                                           void* stream) {
  return dsa_indexer_select<bf16x8>(iq, ik, w, lens, idx, cnt, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_sparse_mla(const void* q, const void* kv, const void* idx, const void* cnt, void* out,
                                  int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  return dsa_sparse_mla<half8>(q, kv, idx, cnt, out, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_sparse_mla_bf16(const void* q, const void* kv, const void* idx, const void* cnt, void* out,
                                       int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  return dsa_sparse_mla<bf16x8>(q, kv, idx, cnt, out, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_decode(const void* q, const void* kv, const void* iq, const void* ik, const void* w,
                              const void* lens, void* out, void* idx, void* cnt, int64_t B, int64_t L,
                              void* workspace, size_t ws_bytes, void* stream) {
  return dsa_decode<half8>(q, kv, iq, ik, w, lens, out, idx, cnt, B, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_dsa_decode_bf16(const void* q, const void* kv, const void* iq, const void* ik, const void* w,
                                   const void* lens, void* out, void* idx, void* cnt, int64_t B, int64_t L,
                                   void* workspace, size_t ws_bytes, void* stream) {
  return dsa_decode<bf16x8>(q, kv, iq, ik, w, lens, out, idx, cnt, B, L, workspace, ws_bytes, stream);
}

// Host replay of select_scan's threshold-bucket search on histograms in host memory (a test hook; no GPU work):
// the coarse search as find_threshold<256> runs it (256 thread ranges of one bin, scanned from the top), then the
// fine bin as the first wave picks it.  out[0] = coarse bin, out[1] = picks left in it, out[2] = fine bucket b1
// (0 when no fine bin qualifies, as in the kernel).  Returns 1 on a null pointer.
extern "C" int vmk_debug_select_threshold(const uint32_t* coarse_hist, const uint32_t* fine_hist, uint32_t need,
                                          uint32_t* out) {
  using namespace vmk;
  VMK_CHECK(coarse_hist && fine_hist && out, "null pointer argument");
  uint32_t thr[2] = {0, 0};
  uint32_t above = 0;
  for (int tid = 0; tid < kCBins; ++tid) {         // thread order = exclusive-scan order
    const int lo = threshold_range_lo(tid, kCBins, 1);
    Threshold t;
    if (threshold_in_range(coarse_hist, lo, 1, above, need, &t)) {
      thr[0] = t.bin;
      thr[1] = t.rest;
    }
    above += coarse_hist[lo];
  }
  const uint32_t* fine = fine_hist + coarse_bin_clamped(thr[0]) * 32;
  uint32_t b1 = 0, incl = 0;
  for (int lane = 0; lane < 32; ++lane) {
    const uint32_t v = fine[31 - lane];
    incl += v;
    if (fine_hit(incl, v, thr[1])) b1 = fine_bin(thr[0], lane);
  }
  out[0] = thr[0];
  out[1] = thr[1];
  out[2] = b1;
  return 0;
}
