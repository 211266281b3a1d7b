// Wave-level split-K attention pipeline shared by the prefix, spec and DSA kernels.
//
// One wave owns 32 query rows and walks 32-key tiles of one key sequence.  Per tile:
//   S^T = K . Q^T   (MFMA 32x32x16: A = the K tile read straight from HBM, B = Q^T held in registers)
//   online softmax in fp32 (exp2 domain) on S^T, whose C-layout gives every lane a single query row
//   O^T += V^T . P^T (A = V^T read from a wave-private LDS transpose of the V tile, B = P^T straight from S^T's
//                    registers, no data movement)
// so every lane's accumulators, running max and running sum belong to one query row (row = lane % 32).
//
// Lane l, k-group g = l / 32:
//   K / Q^T operand of step s (s = 0..7): 8 halfs at head-dim offset 64*g + 8*s of the lane's key / row
//   S^T register 4*blk + c: key 8*blk + 4*g + c of the tile
//   P^T operand of step t (t = 0, 1): S^T registers 8t .. 8t+7, i.e. keys 16t + 8*(j/4) + 4*g + (j%4)
//   V^T operand (d-tile dt, step t): V[key][dt*32 + l%32] for the same eight keys, two 8-byte LDS reads
//   O^T register 4*blk + c of d-tile dt: O[row][dt*32 + 8*blk + 4*g + c]
#pragma once
#include "vmk_common.h"

namespace vmk {

constexpr int kTile = 32;                 // keys per tile
constexpr int kVStride = 36;              // halfs per transposed-V LDS row (32 keys + 4 pad: conflict-free reads)
constexpr int kVTileHalfs = 128 * kVStride;

struct RowState {
  floatx16 o[4];
  float m;   // running max of scaled scores (log2 domain); equal in lanes l and l^32
  float l;   // this lane's partial sum of p (the row total is the sum over lanes l and l^32)
};

__device__ __forceinline__ void row_state_init(RowState& st) {
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) st.o[dt] = floatx16{};
  st.m = kNegInf;
  st.l = 0.f;
}

// Loads are never predicated: every address is clamped in bounds by the caller and out-of-range data is replaced
// by zeros with a select afterwards, so no register is left unwritten on some lanes.
__device__ __forceinline__ u32x4 sel16(bool keep, u32x4 x) {
  return u32x4{keep ? x[0] : 0u, keep ? x[1] : 0u, keep ? x[2] : 0u, keep ? x[3] : 0u};
}

// Q^T operand for 128 head-dims of one row (qrow must be a valid row); zeros when !valid.
__device__ __forceinline__ void load_qt(half8 (&qb)[8], const f16* qrow, int g, bool valid) {
#pragma unroll
  for (int s = 0; s < 8; ++s) qb[s] = as_h8(sel16(valid, ld16(qrow + 64 * g + 8 * s)));
}

// K operand: 128 bytes of the lane's key row (head-dims 64*g .. 64*g+63 of the 128-dim slice at krow).
__device__ __forceinline__ void load_k(u32x4 (&kr)[8], const f16* krow, int g) {
#pragma unroll
  for (int s = 0; s < 8; ++s) kr[s] = ld16(krow + 64 * g + 8 * s);
}

// V tile staging: lane (dc = l%16, kg = l/16) loads dims dc*8..dc*8+7 of keys kg*8 .. kg*8+7.
// vrow(j) returns a valid row pointer for key kg*8+j (clamped by the caller); vok(j) says whether the key belongs
// to the sequence.  Keys outside it are zeroed so that p = 0 never meets a non-finite value of a foreign row.
template <typename VRow, typename VOk>
__device__ __forceinline__ void load_v(u32x4 (&vr)[8], VRow vrow, VOk vok, int dc) {
#pragma unroll
  for (int j = 0; j < 8; ++j) vr[j] = sel16(vok(j), ld16(vrow(j) + 8 * dc));
}

// Compiler-level ordering point for the wave-private LDS tile (the hardware keeps one wave's LDS accesses in
// order; this keeps the compiler from moving loads and stores of the tile across each other).
__device__ __forceinline__ void lds_fence() { asm volatile("" ::: "memory"); }

// Writes the staged V tile transposed into this wave's LDS region: vt[d * kVStride + key].
__device__ __forceinline__ void store_vt(f16* vt, const u32x4 (&vr)[8], int dc, int kg) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    u32x4 col = column8(vr, i);
    u32x2* dst = reinterpret_cast<u32x2*>(vt + (dc * 8 + i) * kVStride + kg * 8);
    dst[0] = u32x2{col[0], col[1]};
    dst[1] = u32x2{col[2], col[3]};
  }
  lds_fence();
}

// S^T tile (unscaled scores) from the K operand and Q^T.
__device__ __forceinline__ floatx16 qk_tile(const u32x4 (&kr)[8], const half8 (&qb)[8]) {
  floatx16 acc = floatx16{};
#pragma unroll
  for (int s = 0; s < 8; ++s) acc = mfma32(as_h8(kr[s]), qb[s], acc);
  return acc;
}

// Online-softmax update with scores already scaled to the log2 domain (masked keys = -inf).  Returns P^T operands.
// Guard: while the row has seen only -inf, the subtrahend is 0 so exp2(-inf) = 0 and a NaN score still yields NaN.
__device__ __forceinline__ void softmax_update(RowState& st, floatx16& s, half8 (&pb)[2]) {
  float tmax = s[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
  tmax = fmaxf(tmax, xor32(tmax));
  const float mnew = fmaxf(st.m, tmax);
  const float muse = (mnew == kNegInf) ? 0.f : mnew;
  const float alpha = fast_exp2(st.m - muse);
  float lsum = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    s[i] = fast_exp2(s[i] - muse);
    lsum += s[i];
  }
  st.l = st.l * alpha + lsum;
  st.m = mnew;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) st.o[dt] *= alpha;
  pb[0] = pack8(s[0], s[1], s[2], s[3], s[4], s[5], s[6], s[7]);
  pb[1] = pack8(s[8], s[9], s[10], s[11], s[12], s[13], s[14], s[15]);
}

// O^T += V^T . P^T using the transposed V tile in LDS.
__device__ __forceinline__ void pv_tile(RowState& st, const f16* vt, const half8 (&pb)[2], int lane) {
  const int r = lane & 31, g = lane >> 5;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const f16* base = vt + (dt * 32 + r) * kVStride + 4 * g;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      // Same access type as store_vt (u32x2) so that type-based alias analysis cannot reorder the two.
      const u32x2 lo = *reinterpret_cast<const u32x2*>(base + 16 * t);
      const u32x2 hi = *reinterpret_cast<const u32x2*>(base + 16 * t + 8);
      const half8 a = as_h8(u32x4{lo[0], lo[1], hi[0], hi[1]});
      st.o[dt] = mfma32(a, pb[t], st.o[dt]);
    }
  }
  lds_fence();
}

// ---- one wave's walk over the tiles t0, t0+tstep, ... of a key sequence, with a one-tile-ahead prefetch held in
// two register buffers used in turn (no copies).  The key source `src` provides, for an absolute key index:
//   krow(key) / vrow(key): an in-bounds row pointer (clamped by the source),
//   valid(key):            whether the key belongs to the sequence,
//   mask_scale(s, key0, g): turns the raw S^T tile into log2-domain scores, -inf where masked.
template <class Src>
__device__ __forceinline__ void issue_tile(u32x4 (&kr)[8], u32x4 (&vr)[8], const Src& src, int key0, int lane) {
  const int r = lane & 31, g = lane >> 5, dc = lane & 15, kg = lane >> 4;
  load_k(kr, src.krow(key0 + r), g);
  load_v(vr, [&](int j) { return src.vrow(key0 + kg * 8 + j); }, [&](int j) { return src.valid(key0 + kg * 8 + j); },
         dc);
}

template <class Src>
__device__ __forceinline__ void compute_tile(RowState& st, const half8 (&qb)[8], f16* vt, const u32x4 (&kr)[8],
                                             const u32x4 (&vr)[8], const Src& src, int key0, int lane) {
  store_vt(vt, vr, lane & 15, lane >> 4);
  floatx16 s = qk_tile(kr, qb);
  src.mask_scale(s, key0, lane >> 5);
  half8 pb[2];
  softmax_update(st, s, pb);
  pv_tile(st, vt, pb, lane);
}

template <class Src>
__device__ __forceinline__ void wave_walk(RowState& st, const half8 (&qb)[8], f16* vt, const Src& src, int kbeg,
                                          int t0, int ntiles, int tstep, int lane) {
  u32x4 kA[8], vA[8], kB[8], vB[8];
  int t = t0;
  if (t < ntiles) issue_tile(kA, vA, src, kbeg + t * kTile, lane);
  while (t < ntiles) {
    const int t1 = t + tstep;
    if (t1 < ntiles) issue_tile(kB, vB, src, kbeg + t1 * kTile, lane);
    compute_tile(st, qb, vt, kA, vA, src, kbeg + t * kTile, lane);
    if (t1 >= ntiles) break;
    const int t2 = t1 + tstep;
    if (t2 < ntiles) issue_tile(kA, vA, src, kbeg + t2 * kTile, lane);
    compute_tile(st, qb, vt, kB, vB, src, kbeg + t1 * kTile, lane);
    t = t2;
  }
}

// Merge another partial state (same lane layout) into st.
__device__ __forceinline__ void merge_state(RowState& st, const floatx16 (&o2)[4], float m2, float l2) {
  const float mnew = fmaxf(st.m, m2);
  const float muse = (mnew == kNegInf) ? 0.f : mnew;
  const float a1 = fast_exp2(st.m - muse), a2 = fast_exp2(m2 - muse);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) st.o[dt] = st.o[dt] * a1 + o2[dt] * a2;
  st.l = st.l * a1 + l2 * a2;
  st.m = mnew;
}

// LDS slot of one wave's state for the cross-wave merge: register-major so every access is conflict-free.
constexpr int kSlotFloats = 66 * 64;

__device__ __forceinline__ void state_to_lds(float* slot, const RowState& st, int lane) {
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) slot[(dt * 16 + i) * 64 + lane] = st.o[dt][i];
  slot[64 * 64 + lane] = st.m;
  slot[65 * 64 + lane] = st.l;
}

__device__ __forceinline__ void merge_from_lds(RowState& st, const float* slot, int lane) {
  floatx16 o2[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o2[dt][i] = slot[(dt * 16 + i) * 64 + lane];
  merge_state(st, o2, slot[64 * 64 + lane], slot[65 * 64 + lane]);
}

// Writes one wave's partial (unnormalised O, running max m, row sum l) for its 32 rows:
//   po[row][d] (row stride 128 floats), pml[row] = (m, l).  Rows >= nvalid are skipped.
__device__ __forceinline__ void store_partial(float* po, float* pml, const RowState& st, int lane, int nvalid) {
  const int r = lane & 31, g = lane >> 5;
  const float ltot = st.l + xor32(st.l);
  if (r >= nvalid) return;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      floatx4 v = floatx4{st.o[dt][4 * blk], st.o[dt][4 * blk + 1], st.o[dt][4 * blk + 2], st.o[dt][4 * blk + 3]};
      *reinterpret_cast<floatx4*>(po + r * 128 + dt * 32 + 8 * blk + 4 * g) = v;
    }
  if (g == 0) {
    pml[2 * r] = st.m;
    pml[2 * r + 1] = ltot;
  }
}

// ---- one workgroup of WR x WK waves (WR * WK <= 4, 256 threads launched): WR row blocks of 32 rows, WK waves
// interleaving the tiles of [kbeg, kbeg + 32*ntiles).  Writes one partial (O, m, l) for the WG's 32*WR rows to
// po (row stride 128 floats) / pml; rows >= nrows are skipped.  smem must hold 3 * kSlotFloats floats.
// qrow(row) returns an in-bounds Q row pointer for a WG-local row (clamped by the caller for rows >= nrows).
template <class Src, class QRow>
__device__ __forceinline__ void attend_wg(float* smem, const Src& src, QRow qrow, int nrows, int kbeg, int ntiles,
                                          int WR, int WK, float* po, float* pml) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave % WR, wk = wave / WR;
  const bool active = wave < WR * WK;
  const int row = wr * 32 + (lane & 31);
  half8 qb[8];
  load_qt(qb, qrow(row < nrows ? row : 0), lane >> 5, row < nrows);
  f16* vt = reinterpret_cast<f16*>(smem) + wave * kVTileHalfs;
  RowState st;
  row_state_init(st);
  if (active) wave_walk(st, qb, vt, src, kbeg, wk, ntiles, WK, lane);
  if (WK > 1) {
    __syncthreads();
    if (active && wk > 0) state_to_lds(smem + (wr * (WK - 1) + wk - 1) * kSlotFloats, st, lane);
    __syncthreads();
    if (active && wk == 0)
      for (int o = 1; o < WK; ++o) merge_from_lds(st, smem + (wr * (WK - 1) + o - 1) * kSlotFloats, lane);
  }
  if (active && wk == 0) store_partial(po + (size_t)wr * 32 * 128, pml + wr * 32 * 2, st, lane, nrows - wr * 32);
}

}  // namespace vmk
