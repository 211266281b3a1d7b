// DSA projections on gfx950: the per-token products that make the DSA decode op's inputs from a hidden state.
//
// The reference leaves them outside its op (ops/dsa.py:8-9); this build defines them after DeepSeek-V3.2's attention
// block (MLA in absorbed form and the lightning indexer), producing the op's q (B,128,576), iq (B,64,128), w (B,64)
// and appending the new token's kv (576) and ik (128) rows to the caches.  Every product is a weight-streaming GEMV
// (B tokens against up to 100 MB of weights), so the bound is HBM: 150 MB of weights per call.
//
// Launch 1 (proj_x_kernel): the x-side rows (Wq_a 1536, Wkv_a 576, Wik 128, Wiw 64 = 2304 rows of 7168) in row blocks
//   of 32 and eight K parts of 896; partial sums per K part.
// Launch 2 (proj_fin_kernel): per request, sums the K parts in order, RMSNorms cq (kept as the 16-bit operand of
//   launch 3) and kv_c, LayerNorms ik, applies RoPE, writes the cache rows and w.
// Launch 3 (proj_q_kernel): Wq_b (24576 rows) and Wiq_b (8192 rows) against cq, two row blocks of 32 per workgroup.
// Launch 4 (proj_absorb_kernel): per head and quarter of its 512 latent dims, the absorbed product of the 16-bit nope
//   part with W_uk[h] (512 x 128), RoPE of the pe parts, the q and iq outputs.
// GEMV tiles use the 32x32x16 MFMA with weight rows as A and the batch (up to 32 tokens per tile) as B; every wave
// issues all its weight loads before its first MFMA, and the K split inside a workgroup is summed through LDS in
// wave order, so results do not depend on scheduling.
#include "vmk.h"
#include "vmk_common.h"
#include "vmk_internal.h"

namespace vmk {

constexpr int kPDim = 7168, kPQl = 1536, kPH = 128, kPDn = 128, kPDr = 64, kPDc = 512, kPHi = 64, kPDi = 128;
constexpr int kPQRows = kPH * (kPDn + kPDr);                 // 24576 rows of Wq_b
constexpr int kPIRows = kPHi * kPDi;                         // 8192 rows of Wiq_b
constexpr int kPXRows = kPQl + kPDc + kPDr + kPDi + kPHi;    // 2304 rows from x
constexpr int kPXKv = kPQl, kPXIk = kPQl + kPDc + kPDr, kPXIw = kPXIk + kPDi;   // row offsets inside the x rows
constexpr int kPKs = 8;                                      // K parts of launch 1
constexpr int kPKPart = kPDim / kPKs;                        // 896
constexpr int kPCols = 32;                                   // tokens per GEMV tile
constexpr float kPEps = 1e-6f;
static_assert(kPKPart % (4 * 16) == 0 && kPQl % (4 * 16) == 0, "K splits of whole MFMA steps");
constexpr int kPQBlocks = 2;                                 // row blocks per workgroup of launch 3

struct ProjArgs {
  const f16* x;            // (B, 7168)
  const int* pos;          // (B,)
  const float* rcos;       // (rope_rows, 32)
  const float* rsin;
  int rope_rows;
  const f16 *wq_a, *wq_b, *w_uk, *wkv_a, *iwq_b, *iwk, *iw;
  const float *q_norm, *kv_norm, *ik_w, *ik_b;
  f16* q;                  // (B, 128, 576)
  f16* iq;                 // (B, 64, 128)
  float* w;                // (B, 64)
  f16* kv;                 // (B, L, 576)
  f16* ik;                 // (B, L, 128)
  int B, L;
  float* yx;               // (kPKs, B, kPXRows)
  f16* cqn;                // (B, 1536)
  float* yq;               // (B, kPQRows + kPIRows)
};

// A GEMV tile: acc (32 weight rows x 32 token columns, the mfma32 D layout) += W[r0 + r][k] * X[col][k] over NS
// steps of 16 k from k0.  gemv_issue loads the wave's weights (all NS loads in flight together; W row-major with
// row stride ldw, rows at or past nrows read row nrows - 1, whose results are never stored); gemv_mma multiplies
// them with X in LDS (row stride ldx halves, column c's row min(c, ncol - 1), columns past ncol never stored, k
// relative to xk0).  A and B share the k map: lane group g takes k0 + 16 s + 8 g .. + 8 in step s.
template <int NS>
__device__ __forceinline__ void gemv_issue(u32x4 (&wv)[NS], const f16* W, size_t ldw, int r0, int nrows, int k0,
                                           int lane) {
  const f16* wp = W + (size_t)min(r0 + (lane & 31), nrows - 1) * ldw + k0 + 8 * (lane >> 5);
#pragma unroll
  for (int s = 0; s < NS; ++s) wv[s] = ldg16(wp + 16 * s);
  asm volatile("" ::: "memory");                              // every load issued before what follows
}
template <class V, int NS>
__device__ __forceinline__ void gemv_mma(floatx16& acc, const u32x4 (&wv)[NS], int k0, const f16* xs, int ldx,
                                         int xk0, int ncol, int lane) {
  const f16* xp = xs + min(lane & 31, ncol - 1) * ldx + (k0 - xk0) + 8 * (lane >> 5);
#pragma unroll
  for (int s = 0; s < NS; ++s)
    acc = mfma32(as_v8<V>(wv[s]), as_v8<V>(*reinterpret_cast<const u32x4*>(xp + 16 * s)), acc);
}

// Stages rows [c0, c0 + ncol) of a 16-bit (B, ldsrc) matrix, columns [k0, k0 + nk), into LDS as ncol x nk (16 bytes
// per thread and step; nk a multiple of 8).
__device__ __forceinline__ void stage_rows(f16* xs, const f16* src, size_t ldsrc, int c0, int ncol, int k0, int nk) {
  const int per_row = nk / 8;
  for (int i = threadIdx.x; i < ncol * per_row; i += blockDim.x) {
    const int c = i / per_row, k = (i % per_row) * 8;
    *reinterpret_cast<u32x4*>(xs + (size_t)c * nk + k) = ldg16(src + (size_t)(c0 + c) * ldsrc + k0 + k);
  }
}

// The four waves' accumulators (same tile, different k ranges) summed in wave order: wave w then holds, in
// out[0..3], rows 8 w + 4 g + c (c < 4) of column lane % 32.  slots: 4 x 4 KB of LDS.
__device__ __forceinline__ void sum_waves(const floatx16& acc, float* slots, int w, int lane, float (&out)[4]) {
  floatx4* sl = reinterpret_cast<floatx4*>(slots);
#pragma unroll
  for (int blk = 0; blk < 4; ++blk)
    sl[(w * 4 + blk) * 64 + lane] = floatx4{acc[4 * blk], acc[4 * blk + 1], acc[4 * blk + 2], acc[4 * blk + 3]};
  __syncthreads();
  floatx4 t = sl[(0 * 4 + w) * 64 + lane];
#pragma unroll
  for (int k = 1; k < 4; ++k) t += sl[(k * 4 + w) * 64 + lane];
#pragma unroll
  for (int c = 0; c < 4; ++c) out[c] = t[c];
}

// x-side rows of row block rb (of 72) as (matrix, first row, rows of that matrix, row offset in yx).
__device__ __forceinline__ const f16* x_rows(const ProjArgs& a, int row, int& local, int& nrows) {
  if (row < kPXKv) { local = row; nrows = kPQl; return a.wq_a; }
  if (row < kPXIk) { local = row - kPXKv; nrows = kPDc + kPDr; return a.wkv_a; }
  if (row < kPXIw) { local = row - kPXIk; nrows = kPDi; return a.iwk; }
  local = row - kPXIw; nrows = kPHi; return a.iw;
}

// Launch 1: grid (72 row blocks * kPKs, token blocks), 256 threads; dynamic LDS max(ncol * kPKPart * 2, 16 KB).
template <class V>
__global__ __launch_bounds__(256) void proj_x_kernel(ProjArgs a) {
  extern __shared__ __attribute__((aligned(16))) char pl[];
  f16* xs = reinterpret_cast<f16*>(pl);
  const int rb = blockIdx.x / kPKs, ks = blockIdx.x % kPKs;
  const int c0 = blockIdx.y * kPCols, ncol = min(kPCols, a.B - c0);
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int local, nrows;
  const f16* W = x_rows(a, rb * 32, local, nrows);           // a row block never straddles two matrices
  const int kw = ks * kPKPart + w * (kPKPart / 4);
  constexpr int NS = kPKPart / 4 / 16;
  u32x4 wv[NS];
  gemv_issue(wv, W, kPDim, local, nrows, kw, lane);          // the weights fly while x is staged
  stage_rows(xs, a.x, kPDim, c0, ncol, ks * kPKPart, kPKPart);
  __syncthreads();
  floatx16 acc = {};
  gemv_mma<V>(acc, wv, kw, xs, kPKPart, ks * kPKPart, ncol, lane);
  __syncthreads();                                            // every wave is done with xs: it becomes the slots
  float out[4];
  sum_waves(acc, reinterpret_cast<float*>(pl), w, lane, out);
  const int col = lane & 31, g = lane >> 5;
  if (col < ncol) {
    float* y = a.yx + ((size_t)ks * a.B + c0 + col) * kPXRows + rb * 32;
#pragma unroll
    for (int c = 0; c < 4; ++c) y[8 * w + 4 * g + c] = out[c];
  }
}
static_assert(kPQl % 32 == 0 && (kPDc + kPDr) % 32 == 0 && kPDi % 32 == 0 && kPHi % 32 == 0, "whole row blocks");

// Block sum of one value per thread (256 threads), returned to every thread.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float yx_sum(const ProjArgs& a, int b, int row) {
  float s = a.yx[(size_t)b * kPXRows + row];
#pragma unroll
  for (int ks = 1; ks < kPKs; ++ks) s += a.yx[((size_t)ks * a.B + b) * kPXRows + row];
  return s;
}

// Launch 2: one workgroup of 256 threads per request.
template <class V>
__global__ __launch_bounds__(256) void proj_fin_kernel(ProjArgs a) {
  typedef elem_t<V> E;
  __shared__ float red[4];
  const int b = blockIdx.x, t = threadIdx.x;
  const int p = a.pos[b];
  const int pr = min(max(p, 0), a.rope_rows - 1);            // the table row (clamped into the table)
  const bool store = p >= 0 && p < a.L;                       // cache rows are written only inside the cache
  // cq: 6 values per thread.
  float cq[kPQl / 256], ss = 0.f;
#pragma unroll
  for (int i = 0; i < kPQl / 256; ++i) {
    cq[i] = yx_sum(a, b, t + 256 * i);
    ss += cq[i] * cq[i];
  }
  const float rq = 1.f / sqrtf(block_sum256(ss, red) / kPQl + kPEps);
  E* cqn = reinterpret_cast<E*>(a.cqn) + (size_t)b * kPQl;
#pragma unroll
  for (int i = 0; i < kPQl / 256; ++i) cqn[t + 256 * i] = (E)(cq[i] * rq * a.q_norm[t + 256 * i]);
  // kv_c: 2 values per thread; k_pe: pairs on threads 0..31.
  float kc[2];
  ss = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    kc[i] = yx_sum(a, b, kPXKv + t + 256 * i);
    ss += kc[i] * kc[i];
  }
  const float rk = 1.f / sqrtf(block_sum256(ss, red) / kPDc + kPEps);
  E* kvr = reinterpret_cast<E*>(a.kv) + ((size_t)b * a.L + (store ? p : 0)) * (kPDc + kPDr);
  if (store) {
#pragma unroll
    for (int i = 0; i < 2; ++i) kvr[t + 256 * i] = (E)(kc[i] * rk * a.kv_norm[t + 256 * i]);
  }
  const float cs = a.rcos[(size_t)pr * 32 + (t & 31)], sn = a.rsin[(size_t)pr * 32 + (t & 31)];
  if (t < 32 && store) {
    const float x0 = yx_sum(a, b, kPXKv + kPDc + 2 * t), x1 = yx_sum(a, b, kPXKv + kPDc + 2 * t + 1);
    kvr[kPDc + 2 * t] = (E)(x0 * cs - x1 * sn);
    kvr[kPDc + 2 * t + 1] = (E)(x0 * sn + x1 * cs);
  }
  // ik: LayerNorm over 128 values (threads 0..127), then RoPE on its first 64 (pairs on threads 0..31).
  const float v = t < kPDi ? yx_sum(a, b, kPXIk + t) : 0.f;
  const float mean = block_sum256(v, red) / kPDi;
  const float d = t < kPDi ? v - mean : 0.f;
  const float ri = 1.f / sqrtf(block_sum256(d * d, red) / kPDi + kPEps);
  __shared__ float ikn[kPDi];
  if (t < kPDi) ikn[t] = d * ri * a.ik_w[t] + a.ik_b[t];
  __syncthreads();
  E* ikr = reinterpret_cast<E*>(a.ik) + ((size_t)b * a.L + (store ? p : 0)) * kPDi;
  if (store && t < kPDi) {
    float o;
    if (t < kPDr) {
      const int i = t >> 1;
      const float c2 = a.rcos[(size_t)pr * 32 + i], s2 = a.rsin[(size_t)pr * 32 + i];
      const float x0 = ikn[2 * i], x1 = ikn[2 * i + 1];
      o = (t & 1) ? x0 * s2 + x1 * c2 : x0 * c2 - x1 * s2;
    } else {
      o = ikn[t];
    }
    ikr[t] = (E)o;
  }
  // w: 64 values.
  if (t < kPHi) a.w[(size_t)b * kPHi + t] = yx_sum(a, b, kPXIw + t) * (0.125f * 0.08838834764831845f);
}

// Launch 3: grid ((kPQRows + kPIRows) / (32 * kPQBlocks), token blocks), 256 threads; dynamic LDS
// max(ncol * 1536 * 2, 16 KB) + 16 KB (the reduction slots).  Every wave issues the weights of all kPQBlocks row
// blocks before the first MFMA.
template <class V>
__global__ __launch_bounds__(256) void proj_q_kernel(ProjArgs a) {
  extern __shared__ __attribute__((aligned(16))) char pl[];
  f16* xs = reinterpret_cast<f16*>(pl);
  // The reduction slots follow the staged tokens, at the offset the host sized the LDS with.
  float* slots = reinterpret_cast<float*>(pl + max(min(kPCols, a.B) * kPQl * 2, 16384));
  const int c0 = blockIdx.y * kPCols, ncol = min(kPCols, a.B - c0);
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int NS = kPQl / 4 / 16;
  u32x4 wv[kPQBlocks][NS];
#pragma unroll
  for (int j = 0; j < kPQBlocks; ++j) {
    const int row0 = (blockIdx.x * kPQBlocks + j) * 32;
    const bool qrows = row0 < kPQRows;                      // the q rows end on a block boundary
    gemv_issue(wv[j], qrows ? a.wq_b : a.iwq_b, kPQl, qrows ? row0 : row0 - kPQRows, qrows ? kPQRows : kPIRows,
               w * (kPQl / 4), lane);
  }
  stage_rows(xs, a.cqn, kPQl, c0, ncol, 0, kPQl);
  __syncthreads();
  const int col = lane & 31, g = lane >> 5;
#pragma unroll
  for (int j = 0; j < kPQBlocks; ++j) {
    floatx16 acc = {};
    gemv_mma<V>(acc, wv[j], w * (kPQl / 4), xs, kPQl, 0, ncol, lane);
    float out[4];
    sum_waves(acc, slots, w, lane, out);
    if (col < ncol) {
      float* y = a.yq + (size_t)(c0 + col) * (kPQRows + kPIRows) + (blockIdx.x * kPQBlocks + j) * 32;
#pragma unroll
      for (int c = 0; c < 4; ++c) y[8 * w + 4 * g + c] = out[c];
    }
    __syncthreads();                                          // the slots are reused by the next block
  }
}
static_assert(kPQRows % (32 * kPQBlocks) == 0 && kPIRows % (32 * kPQBlocks) == 0, "whole row blocks");

// Launch 4: grid (128 heads * 4 quarters, token blocks), 256 threads.  Wave w of quarter qt computes rows (latent
// dims) [128 qt + 32 w, + 32) of head h over K = 128 (8 steps); quarter 0 also applies RoPE to the pe parts.
template <class V>
__global__ __launch_bounds__(256) void proj_absorb_kernel(ProjArgs a) {
  typedef elem_t<V> E;
  __shared__ __attribute__((aligned(16))) E xs[kPCols * kPDn];  // the tokens' 16-bit nope parts of head h
  const int h = blockIdx.x >> 2, qt = blockIdx.x & 3;
  const int c0 = blockIdx.y * kPCols, ncol = min(kPCols, a.B - c0);
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t ldy = kPQRows + kPIRows;
  const f16* W = a.w_uk + (size_t)h * kPDc * kPDn;
  constexpr int NS = kPDn / 16;
  const int r0 = 128 * qt + 32 * w;
  u32x4 wv[NS];
  gemv_issue(wv, W, kPDn, r0, kPDc, 0, lane);
  for (int i = threadIdx.x; i < ncol * kPDn; i += 256) {
    const int c = i / kPDn, d = i % kPDn;
    xs[i] = (E)a.yq[(size_t)(c0 + c) * ldy + h * (kPDn + kPDr) + d];
  }
  __syncthreads();
  const int col = lane & 31, g = lane >> 5;
  floatx16 acc = {};
  gemv_mma<V>(acc, wv, 0, reinterpret_cast<const f16*>(xs), kPDn, 0, ncol, lane);
  if (col < ncol) {
    E* qo = reinterpret_cast<E*>(a.q) + ((size_t)(c0 + col) * kPH + h) * (kPDc + kPDr) + r0;
#pragma unroll
    for (int i = 0; i < 16; ++i) qo[8 * (i / 4) + 4 * g + (i % 4)] = (E)acc[i];
  }
  if (qt != 0) return;
  // RoPE of q's pe part (and, for h < 64, the indexer head h): thread t -> token t / 32, pair t % 32.
  for (int i = threadIdx.x; i < ncol * 32; i += 256) {
    const int c = i / 32, pi = i % 32, b = c0 + c;
    const int pr = min(max(a.pos[b], 0), a.rope_rows - 1);
    const float cs = a.rcos[(size_t)pr * 32 + pi], sn = a.rsin[(size_t)pr * 32 + pi];
    const float* yb = a.yq + (size_t)b * ldy;
    const float x0 = yb[h * (kPDn + kPDr) + kPDn + 2 * pi], x1 = yb[h * (kPDn + kPDr) + kPDn + 2 * pi + 1];
    E* qo = reinterpret_cast<E*>(a.q) + ((size_t)b * kPH + h) * (kPDc + kPDr) + kPDc;
    qo[2 * pi] = (E)(x0 * cs - x1 * sn);
    qo[2 * pi + 1] = (E)(x0 * sn + x1 * cs);
    if (h < kPHi) {
      const float* yi = yb + kPQRows + h * kPDi;
      E* io = reinterpret_cast<E*>(a.iq) + ((size_t)b * kPHi + h) * kPDi;
      const float y0 = yi[2 * pi], y1 = yi[2 * pi + 1];
      io[2 * pi] = (E)(y0 * cs - y1 * sn);
      io[2 * pi + 1] = (E)(y0 * sn + y1 * cs);
      io[kPDr + 2 * pi] = (E)yi[kPDr + 2 * pi];
      io[kPDr + 2 * pi + 1] = (E)yi[kPDr + 2 * pi + 1];
    }
  }
}

struct ProjPlan {
  size_t yx, cqn, yq;      // bytes of each workspace region
};

static ProjPlan proj_plan(int64_t B) {
  ProjPlan p;
  p.yx = (size_t)kPKs * B * kPXRows * sizeof(float);
  p.cqn = (size_t)B * kPQl * 2;
  p.yq = (size_t)B * (kPQRows + kPIRows) * sizeof(float);
  return p;
}

template <class V>
static int dsa_project(const void* x, const void* pos, const void* rope_cos, const void* rope_sin, int64_t rope_rows,
                       const vmk_dsa_project_weights* wt, void* q, void* iq, void* w, void* kv, void* ik, int64_t B,
                       int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(wt, "null weights");
  VMK_CHECK(x && pos && rope_cos && rope_sin && q && iq && w && kv && ik && workspace, "null pointer argument");
  VMK_CHECK(wt->wq_a && wt->q_norm && wt->wq_b && wt->w_uk && wt->wkv_a && wt->kv_norm && wt->iwq_b && wt->iwk &&
                wt->ik_norm_w && wt->ik_norm_b && wt->iw, "null weight pointer");
  VMK_CHECK(B >= 1 && B <= (1 << 20) && L >= 1 && L <= ((int64_t)1 << 31) / (kPDc + kPDr), "B or L out of range");
  VMK_CHECK(rope_rows >= 1 && rope_rows <= (1 << 30), "rope_rows out of range");
  VMK_CHECK(aligned16(x) && aligned16(wt->wq_a) && aligned16(wt->wq_b) && aligned16(wt->w_uk) &&
                aligned16(wt->wkv_a) && aligned16(wt->iwq_b) && aligned16(wt->iwk) && aligned16(wt->iw),
            "x and the weight matrices must be 16-byte aligned");
  const ProjPlan p = proj_plan(B);
  VMK_CHECK(ws_bytes >= vmk_dsa_project_workspace_size(B), "workspace too small (query vmk_dsa_project_workspace_size)");
  ProjArgs a;
  a.x = (const f16*)x; a.pos = (const int*)pos; a.rcos = (const float*)rope_cos; a.rsin = (const float*)rope_sin;
  a.rope_rows = (int)rope_rows;
  a.wq_a = (const f16*)wt->wq_a; a.wq_b = (const f16*)wt->wq_b; a.w_uk = (const f16*)wt->w_uk;
  a.wkv_a = (const f16*)wt->wkv_a; a.iwq_b = (const f16*)wt->iwq_b; a.iwk = (const f16*)wt->iwk;
  a.iw = (const f16*)wt->iw;
  a.q_norm = (const float*)wt->q_norm; a.kv_norm = (const float*)wt->kv_norm;
  a.ik_w = (const float*)wt->ik_norm_w; a.ik_b = (const float*)wt->ik_norm_b;
  a.q = (f16*)q; a.iq = (f16*)iq; a.w = (float*)w; a.kv = (f16*)kv; a.ik = (f16*)ik;
  a.B = (int)B; a.L = (int)L;
  a.yx = (float*)align_up((char*)workspace + kWsHead, 256);
  a.cqn = (f16*)align_up((char*)a.yx + p.yx, 256);
  a.yq = (float*)align_up((char*)a.cqn + p.cqn, 256);
  hipStream_t s = (hipStream_t)stream;
  const unsigned nbb = (unsigned)((B + kPCols - 1) / kPCols);
  const int ncol = (int)std::min<int64_t>(B, kPCols);
  const size_t lds_x = std::max<size_t>((size_t)ncol * kPKPart * 2, 16384);
  const size_t lds_q = std::max<size_t>((size_t)ncol * kPQl * 2, 16384) + 16384;
  hipLaunchKernelGGL(proj_x_kernel<V>, dim3(kPXRows / 32 * kPKs, nbb), dim3(256), lds_x, s, a);
  VMK_CHECK_HIP(hipGetLastError());
  hipLaunchKernelGGL(proj_fin_kernel<V>, dim3((unsigned)B), dim3(256), 0, s, a);
  VMK_CHECK_HIP(hipGetLastError());
  prof_before(kKDsaProjectQ, s);
  hipLaunchKernelGGL(proj_q_kernel<V>, dim3((kPQRows + kPIRows) / (32 * kPQBlocks), nbb), dim3(256), lds_q, s, a);
  prof_after(kKDsaProjectQ, s);
  VMK_CHECK_HIP(hipGetLastError());
  hipLaunchKernelGGL(proj_absorb_kernel<V>, dim3(kPH * 4, nbb), dim3(256), 0, s, a);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

}  // namespace vmk

using namespace vmk;

extern "C" size_t vmk_dsa_project_workspace_size(int64_t B) {
  if (B < 1 || B > (1 << 20)) return 0;
  const ProjPlan p = proj_plan(B);
  return kWsHead + p.yx + p.cqn + p.yq + 3 * 256;
}

extern "C" int vmk_dsa_project(const void* x, const void* pos, const void* rope_cos, const void* rope_sin,
                               int64_t rope_rows, const vmk_dsa_project_weights* weights, void* q, void* iq, void* w,
                               void* kv, void* ik, int64_t B, int64_t L, void* workspace, size_t ws_bytes,
                               void* stream) {
  return dsa_project<half8>(x, pos, rope_cos, rope_sin, rope_rows, weights, q, iq, w, kv, ik, B, L, workspace,
                            ws_bytes, stream);
}

extern "C" int vmk_dsa_project_bf16(const void* x, const void* pos, const void* rope_cos, const void* rope_sin,
                                    int64_t rope_rows, const vmk_dsa_project_weights* weights, void* q, void* iq,
                                    void* w, void* kv, void* ik, int64_t B, int64_t L, void* workspace,
                                    size_t ws_bytes, void* stream) {
  return dsa_project<bf16x8>(x, pos, rope_cos, rope_sin, rope_rows, weights, q, iq, w, kv, ik, B, L, workspace,
                             ws_bytes, stream);
}
