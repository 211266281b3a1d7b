// DSA projections on gfx950: the per-token products that make the DSA decode op's inputs from a hidden state.
//
// The reference leaves them outside its op (ops/dsa.py:8-9); this build defines them after DeepSeek-V3.2's attention
// block (MLA in absorbed form and the lightning indexer), producing the op's q (B,128,576), iq (B,64,128), w (B,64)
// and appending the new token's kv (576) and ik (128) rows to the caches.  Every product is a weight-streaming GEMV
// (B tokens against up to 100 MB of weights), so the bound is HBM: 150 MB of weights per call.
//
// Launch 1 (proj_x_kernel): the x-side rows (Wq_a 1536, Wkv_a 576, Wik 128, Wiw 64 = 2304 rows of 7168) in row blocks
//   of 64 and seven K parts of 1024: 252 workgroups of 8 waves, one dispatch round; partial sums per K part.
// Launch 2 (proj_heads_kernel): 256 workgroups of 8 waves, each 128 rows of Wq_b or Wiq_b against cq.  Workgroup h
//   (< 128) takes MLA head h's nope rows and then the absorbed product with W_uk[h] (512 x 128); workgroups 128 + p
//   take the pe rows of heads 2p and 2p + 1 (RoPE) and finish token p's cache rows and w; workgroups 192 + j take
//   indexer head j's rows (RoPE on the first 64, pairs (i, i + 32)).  Every workgroup first sums cq's K parts and RMSNorms it itself
//   (the same arithmetic in each), so no launch runs between the two.
// GEMV tiles use the 32x32x16 MFMA with weight rows as A and the batch (up to 32 tokens per tile) as B; every wave
// issues all its weight loads before its first MFMA, and the K split inside a workgroup is summed through LDS in
// K order, so results do not depend on scheduling.
#include "vmk.h"
#include "vmk_common.h"
#include "vmk_internal.h"

namespace vmk {

constexpr int kPDim = 7168, kPQl = 1536, kPH = 128, kPDn = 128, kPDr = 64, kPDc = 512, kPHi = 64, kPDi = 128;
constexpr int kPQRows = kPH * (kPDn + kPDr);                 // 24576 rows of Wq_b
constexpr int kPIRows = kPHi * kPDi;                         // 8192 rows of Wiq_b
constexpr int kPXRows = kPQl + kPDc + kPDr + kPDi + kPHi;    // 2304 rows from x
constexpr int kPXKv = kPQl, kPXIk = kPQl + kPDc + kPDr, kPXIw = kPXIk + kPDi;   // row offsets inside the x rows
constexpr int kPKs = 7;                                      // K parts of launch 1
constexpr int kPKPart = kPDim / kPKs;                        // 1024
constexpr int kPXBlock = 64;                                 // rows per workgroup of launch 1
constexpr int kPCols = 32;                                   // tokens per GEMV tile
constexpr float kPEps = 1e-6f;
constexpr int kPHeadsWG = kPH + kPH / 2 + kPHi;              // workgroups of launch 2 per token block: 128 + 64 + 64
static_assert(kPDim % kPKs == 0 && kPKPart % (4 * 16) == 0 && kPQl % (4 * 16) == 0, "K splits of whole MFMA steps");
static_assert(kPQl % 64 == 0 && (kPDc + kPDr) % 64 == 0 && kPDi % 64 == 0 && kPHi % 64 == 0,
              "a row block of launch 1 never straddles two matrices");

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

// The accumulators of four waves (the same tile over K quarters q = 0..3) summed in K order: the wave of quarter q
// then holds, in out[0..3], rows 8 q + 4 g + c (c < 4) of column lane % 32.  slots: the four waves' 16 KB of LDS.
// Every thread of the workgroup calls it (it holds a workgroup barrier).
__device__ __forceinline__ void sum_quarters(const floatx16& acc, float* slots, int q, int lane, float (&out)[4]) {
  floatx4* sl = reinterpret_cast<floatx4*>(slots);
#pragma unroll
  for (int blk = 0; blk < 4; ++blk)
    sl[(q * 4 + blk) * 64 + lane] = floatx4{acc[4 * blk], acc[4 * blk + 1], acc[4 * blk + 2], acc[4 * blk + 3]};
  __syncthreads();
  floatx4 t = sl[(0 * 4 + q) * 64 + lane];
#pragma unroll
  for (int k = 1; k < 4; ++k) t += sl[(k * 4 + q) * 64 + lane];
#pragma unroll
  for (int c = 0; c < 4; ++c) out[c] = t[c];
}

// x-side rows from `row` on as (matrix, its first row, rows of that matrix).
__device__ __forceinline__ const f16* x_rows(const ProjArgs& a, int row, int& local, int& nrows) {
  if (row < kPXKv) { local = row; nrows = kPQl; return a.wq_a; }
  if (row < kPXIk) { local = row - kPXKv; nrows = kPDc + kPDr; return a.wkv_a; }
  if (row < kPXIw) { local = row - kPXIk; nrows = kPDi; return a.iwk; }
  local = row - kPXIw; nrows = kPHi; return a.iw;
}

// Launch 1: grid (36 row blocks * kPKs, token blocks), 512 threads; dynamic LDS max(ncol * kPKPart * 2, 32 KB).
// Wave w takes the 32-row tile w & 1 of the block over K quarter w >> 1 of the part.
template <class V>
__global__ __launch_bounds__(512) void proj_x_kernel(ProjArgs a) {
  extern __shared__ __attribute__((aligned(16))) char pl[];
  f16* xs = reinterpret_cast<f16*>(pl);
  const int rb = blockIdx.x / kPKs, ks = blockIdx.x % kPKs;
  const int c0 = blockIdx.y * kPCols, ncol = min(kPCols, a.B - c0);
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rt = w & 1, kq = w >> 1;
  int local, nrows;
  const f16* W = x_rows(a, rb * kPXBlock, local, nrows);
  const int kw = ks * kPKPart + kq * (kPKPart / 4);
  constexpr int NS = kPKPart / 4 / 16;
  u32x4 wv[NS];
  gemv_issue(wv, W, kPDim, local + 32 * rt, nrows, kw, lane);     // the weights fly while x is staged
  stage_rows(xs, a.x, kPDim, c0, ncol, ks * kPKPart, kPKPart);
  __syncthreads();
  floatx16 acc = {};
  gemv_mma<V>(acc, wv, kw, xs, kPKPart, ks * kPKPart, ncol, lane);
  __syncthreads();                                                // every wave is done with xs: it becomes the slots
  float out[4];
  sum_quarters(acc, reinterpret_cast<float*>(pl) + rt * 4096, kq, lane, out);
  const int col = lane & 31, g = lane >> 5;
  if (col < ncol) {
    float* y = a.yx + ((size_t)ks * a.B + c0 + col) * kPXRows + rb * kPXBlock + 32 * rt;
#pragma unroll
    for (int c = 0; c < 4; ++c) y[8 * kq + 4 * g + c] = out[c];
  }
}

// Block sum of one value per thread (512 threads), returned to every thread; red: 8 floats of LDS.
__device__ __forceinline__ float block_sum512(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) s += red[i];
  return s;
}

// x-side row `row` of token b: its K parts summed in part order.
__device__ __forceinline__ float yx_sum(const ProjArgs& a, int b, int row) {
  float s = a.yx[(size_t)b * kPXRows + row];
#pragma unroll
  for (int ks = 1; ks < kPKs; ++ks) s += a.yx[((size_t)ks * a.B + b) * kPXRows + row];
  return s;
}

__device__ __forceinline__ int rope_row(const ProjArgs& a, int b) { return min(max(a.pos[b], 0), a.rope_rows - 1); }

// Token b's cache rows (kv: RMSNorm of kv_c, interleaved RoPE of k_pe; ik: LayerNorm, RoPE of its first 64 on the
// pairs (i, i + 32)) and w, by 512 threads.
// Rows are written only for a position inside the cache.
template <class E>
__device__ void finish_token(const ProjArgs& a, int b, float* red, float* ikn) {
  const int t = threadIdx.x;
  const int p = a.pos[b], pr = rope_row(a, b);
  const bool store = p >= 0 && p < a.L;
  const float kc = yx_sum(a, b, kPXKv + t);                   // kv_c: one value per thread
  const float rk = 1.f / sqrtf(block_sum512(kc * kc, red) / kPDc + kPEps);
  E* kvr = reinterpret_cast<E*>(a.kv) + ((size_t)b * a.L + (store ? p : 0)) * (kPDc + kPDr);
  if (store) kvr[t] = (E)(kc * rk * a.kv_norm[t]);
  if (t < 32 && store) {                                      // k_pe: pair t
    const float cs = a.rcos[(size_t)pr * 32 + t], sn = a.rsin[(size_t)pr * 32 + t];
    const float x0 = yx_sum(a, b, kPXKv + kPDc + 2 * t), x1 = yx_sum(a, b, kPXKv + kPDc + 2 * t + 1);
    kvr[kPDc + 2 * t] = (E)(x0 * cs - x1 * sn);
    kvr[kPDc + 2 * t + 1] = (E)(x0 * sn + x1 * cs);
  }
  const float v = t < kPDi ? yx_sum(a, b, kPXIk + t) : 0.f;   // ik: LayerNorm over 128 values
  const float mean = block_sum512(v, red) / kPDi;
  const float d = t < kPDi ? v - mean : 0.f;
  const float ri = 1.f / sqrtf(block_sum512(d * d, red) / kPDi + kPEps);
  if (t < kPDi) ikn[t] = d * ri * a.ik_w[t] + a.ik_b[t];
  __syncthreads();
  if (store && t < kPDi) {
    E* ikr = reinterpret_cast<E*>(a.ik) + ((size_t)b * a.L + p) * kPDi;
    float o = ikn[t];
    if (t < kPDr) {                                           // indexer RoPE: pairs (i, i + 32), not interleaved
      const int i = t & 31;
      const float c2 = a.rcos[(size_t)pr * 32 + i], s2 = a.rsin[(size_t)pr * 32 + i];
      const float x0 = ikn[i], x1 = ikn[i + 32];
      o = (t & 32) ? x0 * s2 + x1 * c2 : x0 * c2 - x1 * s2;
    }
    ikr[t] = (E)o;
  }
  if (t < kPHi) a.w[(size_t)b * kPHi + t] = yx_sum(a, b, kPXIw + t) * (0.125f * 0.08838834764831845f);
}

// Launch 2: grid (kPHeadsWG, token blocks), 512 threads; dynamic LDS max(ncol * 1536 * 2, 64 KB + ncol * 256).
// Wave w takes row blocks 2 (w >> 2) and 2 (w >> 2) + 1 of the workgroup's four over K quarter w & 3.
template <class V>
__global__ __launch_bounds__(512) void proj_heads_kernel(ProjArgs a) {
  typedef elem_t<V> E;
  extern __shared__ __attribute__((aligned(16))) char pl[];
  __shared__ float red[8], ikn[kPDi];
  E* xs = reinterpret_cast<E*>(pl);                           // cq of the token block (ncol x 1536)
  const int c0 = blockIdx.y * kPCols, ncol = min(kPCols, a.B - c0);
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = w & 3, bp = w >> 2;
  const int wg = blockIdx.x;
  // The workgroup's four row blocks: rows of Wq_b (nope of head wg, or pe of heads 2p, 2p + 1) or of Wiq_b.
  auto block_rows = [&](int i, const f16*& W, int& nrows) -> int {
    if (wg < kPH) { W = a.wq_b; nrows = kPQRows; return wg * (kPDn + kPDr) + 32 * i; }
    if (wg < kPH + kPH / 2) {
      const int hp = 2 * (wg - kPH) + (i >> 1);
      W = a.wq_b; nrows = kPQRows; return hp * (kPDn + kPDr) + kPDn + 32 * (i & 1);
    }
    W = a.iwq_b; nrows = kPIRows; return (wg - kPH - kPH / 2) * kPDi + 32 * i;
  };
  constexpr int NS = kPQl / 4 / 16;
  u32x4 wv[2][NS];
  // cq first (its loads need most of the registers the weights take): wave w takes tokens w, w + 8, ...; lane l the
  // rows [24 l, 24 l + 24), its K parts summed in part order.
  for (int c = w; c < ncol; c += 8) {
    const int b = c0 + c;
    float v[24];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      floatx4 s = *reinterpret_cast<const floatx4*>(a.yx + (size_t)b * kPXRows + 24 * lane + 4 * i);
#pragma unroll
      for (int ks = 1; ks < kPKs; ++ks)
        s += *reinterpret_cast<const floatx4*>(a.yx + ((size_t)ks * a.B + b) * kPXRows + 24 * lane + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * i + e] = s[e];
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 24; ++k) ss += v[k] * v[k];
    const float rq = 1.f / sqrtf(wave_sum(ss) / kPQl + kPEps);
#pragma unroll
    for (int k = 0; k < 24; ++k) xs[c * kPQl + 24 * lane + k] = (E)(v[k] * rq * a.q_norm[24 * lane + k]);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const f16* W;
    int nrows;
    const int r0 = block_rows(2 * bp + j, W, nrows);
    gemv_issue(wv[j], W, kPQl, r0, nrows, kq * (kPQl / 4), lane);
  }
  __syncthreads();                                            // cq staged
  floatx16 acc[2] = {};
#pragma unroll
  for (int j = 0; j < 2; ++j) gemv_mma<V>(acc[j], wv[j], kq * (kPQl / 4), reinterpret_cast<const f16*>(xs), kPQl, 0,
                                          ncol, lane);
  // MLA head workgroups: W_uk[h] rows [64 w, 64 w + 64) fly while the K quarters are summed.
  constexpr int NU = kPDn / 16;
  u32x4 wu[2][NU];
  if (wg < kPH) {
#pragma unroll
    for (int j = 0; j < 2; ++j) gemv_issue(wu[j], a.w_uk + (size_t)wg * kPDc * kPDn, kPDn, 64 * w + 32 * j, kPDc, 0,
                                           lane);
  }
  __syncthreads();                                            // every wave is done with xs: it becomes the slots
  float out[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) sum_quarters(acc[j], reinterpret_cast<float*>(pl) + (bp * 2 + j) * 4096, kq, lane,
                                           out[j]);
  // This wave now holds rows 8 kq + 4 g + c (c < 4) of blocks 2 bp + j for token column col.
  const int col = lane & 31, g = lane >> 5, b = c0 + col;
  const bool live = col < ncol;
  if (wg < kPH) {
    // The nope part, rounded to the operand type, is the absorbed product's B operand (ncol x 128 after the slots).
    E* xn = reinterpret_cast<E*>(pl + 65536);
    if (live) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) xn[col * kPDn + 32 * (2 * bp + j) + 8 * kq + 4 * g + c] = (E)out[j][c];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      floatx16 qa = {};
      gemv_mma<V>(qa, wu[j], 0, reinterpret_cast<const f16*>(xn), kPDn, 0, ncol, lane);
      if (live) {
        E* qo = reinterpret_cast<E*>(a.q) + ((size_t)b * kPH + wg) * (kPDc + kPDr) + 64 * w + 32 * j;
#pragma unroll
        for (int i = 0; i < 16; ++i) qo[8 * (i / 4) + 4 * g + (i % 4)] = (E)qa[i];
      }
    }
    return;
  }
  // RoPE pairs (rows 2m, 2m + 1 are c = 0, 1 and c = 2, 3 of one lane), with token b's table row.
  const int pr = live ? rope_row(a, b) : 0;
  if (wg < kPH + kPH / 2) {
    if (live) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int i = 2 * bp + j, hp = 2 * (wg - kPH) + (i >> 1);
        E* qo = reinterpret_cast<E*>(a.q) + ((size_t)b * kPH + hp) * (kPDc + kPDr) + kPDc;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const int e = 32 * (i & 1) + 8 * kq + 4 * g + 2 * m, pi = e >> 1;
          const float cs = a.rcos[(size_t)pr * 32 + pi], sn = a.rsin[(size_t)pr * 32 + pi];
          const float x0 = out[j][2 * m], x1 = out[j][2 * m + 1];
          qo[e] = (E)(x0 * cs - x1 * sn);
          qo[e + 1] = (E)(x0 * sn + x1 * cs);
        }
      }
    }
    const int tok = wg - kPH;                                 // token of the block whose cache rows this finishes
    if (tok < ncol) finish_token<E>(a, c0 + tok, red, ikn);
    return;
  }
  if (live) {
    const int hj = wg - kPH - kPH / 2;
    E* io = reinterpret_cast<E*>(a.iq) + ((size_t)b * kPHi + hj) * kPDi;
    if (bp == 0) {
      // Blocks 0 and 1 are the 64 pe dims: this lane holds dims r and r + 32 of each rotated pair (the indexer's
      // RoPE pairs the halves, not interleaved neighbours), rotated by table entry r.
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int r = 8 * kq + 4 * g + c;
        const float cs = a.rcos[(size_t)pr * 32 + r], sn = a.rsin[(size_t)pr * 32 + r];
        const float x0 = out[0][c], x1 = out[1][c];
        io[r] = (E)(x0 * cs - x1 * sn);
        io[r + 32] = (E)(x0 * sn + x1 * cs);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) io[32 * (2 + j) + 8 * kq + 4 * g + c] = (E)out[j][c];
    }
  }
}

struct ProjPlan {
  size_t yx;               // bytes of the workspace's partial sums
};

static ProjPlan proj_plan(int64_t B) {
  ProjPlan p;
  p.yx = (size_t)kPKs * B * kPXRows * sizeof(float);
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
  hipStream_t s = (hipStream_t)stream;
  const unsigned nbb = (unsigned)((B + kPCols - 1) / kPCols);
  const int ncol = (int)std::min<int64_t>(B, kPCols);
  const size_t lds_x = std::max<size_t>((size_t)ncol * kPKPart * 2, 32768);
  const size_t lds_h = std::max<size_t>((size_t)ncol * kPQl * 2, 65536 + (size_t)ncol * kPDn * 2);
  hipLaunchKernelGGL(proj_x_kernel<V>, dim3(kPXRows / kPXBlock * kPKs, nbb), dim3(512), lds_x, s, a);
  VMK_CHECK_HIP(hipGetLastError());
  prof_before(kKDsaProjectQ, s);
  hipLaunchKernelGGL(proj_heads_kernel<V>, dim3(kPHeadsWG, nbb), dim3(512), lds_h, s, a);
  prof_after(kKDsaProjectQ, s);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

}  // namespace vmk

using namespace vmk;

extern "C" size_t vmk_dsa_project_workspace_size(int64_t B) {
  if (B < 1 || B > (1 << 20)) return 0;
  const ProjPlan p = proj_plan(B);
  return kWsHead + p.yx + 256;
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
