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
  float m;   // running max of scaled scores (log2 domain); equal in lanes l and l^32; -inf before the first
  float l;   // this lane's partial sum of p (the row total is the sum over lanes l and l^32)
  float mu;  // the subtrahend p = exp2(scaled score - mu) uses: m, or kMuNone while m is -inf
};

// Subtrahend of a row that has seen no finite score yet: a finite score minus it gives p = +inf, which the
// overflow check of softmax_update catches, while a masked (-inf) score still gives p = 0.
constexpr float kMuNone = -1e30f;
// A lane's sum of one tile's 16 p values at or below this bound keeps every p <= 2^15, inside fp16's range
// (65504) with a factor 2 to spare; a larger sum, or +inf, sends the tile through the exact path.
constexpr float kTileSumMax = 32768.f;

__device__ __forceinline__ void row_state_init(RowState& st) {
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) st.o[dt] = floatx16{};
  st.m = kNegInf;
  st.l = 0.f;
  st.mu = kMuNone;
}

// Loads are never predicated: every address is clamped in bounds by the caller and out-of-range data is replaced
// by zeros with a select afterwards, so no register is left unwritten on some lanes.
__device__ __forceinline__ u32x4 sel16(bool keep, u32x4 x) {
  return u32x4{keep ? x[0] : 0u, keep ? x[1] : 0u, keep ? x[2] : 0u, keep ? x[3] : 0u};
}

// One all-zero fp16 row (256 bytes, zero-initialised at load time and never written): the K/V source of every key
// outside the sequence, so a tile's spare rows are zeros and p = 0 never meets a non-finite value of a foreign row,
// and the Q source of rows outside the workgroup's range.
__device__ const f16 g_zero_row[128] = {};
// One zero tile (32 rows): the K or V tile of a key range that has no memory (an absent page of a paged cache).
__device__ __attribute__((aligned(16))) const f16 g_zero_tile[32 * 128] = {};

// Q^T operand for 128 head-dims of one row (qrow must be a valid row); zeros when !valid, read from g_zero_row rather
// than selected after the load, so nothing waits for these loads before the first MFMA that uses them (a select would
// make the compiler wait for them right away, ahead of the first tile's DMA).
// V is the operand type (half8 or bf16x8); qrow points at the row's raw 16-bit elements.
template <class V>
__device__ __forceinline__ void load_qt(V (&qb)[8], const f16* qrow, int g, bool valid) {
  const f16* p = valid ? qrow : g_zero_row;
#pragma unroll
  for (int s = 0; s < 8; ++s) qb[s] = as_v8<V>(ldg16(p + 64 * g + 8 * s));
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

// Sum of the 16 rounded p values of a lane (the P^T operands), in fp32: dot products with (1, 1) of the packed
// pairs, so the row sum counts exactly the values the P.V product multiplies.
__device__ __forceinline__ float rowsum16(const half8 (&pb)[2]) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_fdot2(h2{pb[t][2 * i], pb[t][2 * i + 1]}, h2{1, 1}, acc, false);
  return acc;
}
__device__ __forceinline__ float rowsum16(const bf16x8 (&pb)[2]) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_fdot2_f32_bf16(b2{pb[t][2 * i], pb[t][2 * i + 1]}, b2{1, 1}, acc, false);
  return acc;
}

// p = exp2(scale * s - mu) for a lane's 16 raw scores, rounded to the operand type V as the P^T operands.
template <class V>
__device__ __forceinline__ void exp_tile(const floatx16& s, float scale, float mu, V (&pb)[2]) {
  float p[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = fast_exp2(__builtin_fmaf(s[i], scale, -mu));
  pb[0] = pack8v<V>(p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
  pb[1] = pack8v<V>(p[8], p[9], p[10], p[11], p[12], p[13], p[14], p[15]);
}

// Online-softmax update of raw scores s (masked keys = -inf), returning the P^T operands; scale is the positive
// log2-domain softmax scale, so p = exp2(scale * s - mu) costs one FMA per score.
// Fast path (almost every tile): p with the row's current subtrahend mu, and no tile maximum at all.  The lane's sum
// of its 16 rounded p values bounds each of them, so a sum <= 2^15 proves that no p overflowed fp16 (or grew past
// 2^15 in bf16), and the tile is accepted as it is.  Otherwise (the first tile with a finite score, whose p are
// +inf against kMuNone, or a tile whose scores rose by more than ~11 in the log2 domain) the whole wave takes the
// exact path: row maxima over both lane halves, m moved up to them, O and l rescaled, p recomputed.
// Non-finite scores: a NaN score gives a NaN sum, which passes the check and carries NaN into P, O and l (the row's
// output is NaN, as in float64); a +inf score takes the exact path and gives m = +inf and p = NaN for it (inf - inf).
// P is rounded to the operand type V of the values it multiplies; l sums those rounded values.
template <class V>
__device__ __forceinline__ void softmax_update(RowState& st, const floatx16& s, float scale, V (&pb)[2]) {
  exp_tile(s, scale, st.mu, pb);
  float lsum = rowsum16(pb);
  if (__builtin_amdgcn_ballot_w64(lsum > kTileSumMax)) {      // rare: uniform for the wave
    // Only the rows whose own lanes overflowed move: the others keep m, get alpha = 1 and the same p bit for bit,
    // so a row's arithmetic never depends on the other rows of its wave (batch invariance).
    const float trig = lsum > kTileSumMax ? 1.f : 0.f;
    const bool row_trig = trig + xor32(trig) > 0.f;
    float tmax = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
    tmax = fmaxf(tmax, xor32(tmax)) * scale;                     // NaN scores are ignored here
    const float mnew = row_trig ? fmaxf(st.m, tmax) : st.m;
    const float munew = (mnew == kNegInf) ? kMuNone : mnew;
    const float alpha = fast_exp2(st.mu - munew);                // 0 when leaving kMuNone; 1 if unchanged
    st.l *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) st.o[dt] *= alpha;
    st.m = mnew;
    st.mu = munew;
    exp_tile(s, scale, st.mu, pb);
    lsum = rowsum16(pb);
  }
  st.l += lsum;
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

// ---- tile staging through LDS with direct-to-LDS loads (global_load_lds_dwordx4: each lane's 16 bytes land at
// LDS slot `lane` of the instruction's 1 KB block, no VGPR staging).
//
// A stage holds one 32-key tile: K rows in bytes [0, 8192), V rows in [8192, 16384), each row 256 bytes (D = 128).
// Within a row, the 16-byte chunk c is stored at chunk position c ^ swz(row), where swz swaps the two 2-bit fields of
// row & 15.  A row is exactly one pass over the 64 LDS banks, so the bank of a chunk is its position.  swz is a
// bijection on 16 consecutive rows, so the K-operand reads (16 rows, one logical chunk, per pass) are conflict-free.
// For the transposed V reads (8 rows x 4 logical chunks x 2 half-chunks per instruction) the 32 (row, chunk) pairs
// fall on all 16 positions exactly twice, i.e. the minimum two passes.
constexpr int kStageBytes = 16384;

__device__ __forceinline__ int swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }

#define VMK_GPTR(p) ((const void __attribute__((address_space(1)))*)(p))
#define VMK_LPTR(p) ((void __attribute__((address_space(3)))*)(p))

// Waits until at most n (0 <= n <= 63; larger counts wait for everything) of this wave's vector-memory operations
// are outstanding (loads return in order).  An asm statement with a memory clobber, so the compiler neither drops it
// nor moves LDS accesses across it.
__device__ __forceinline__ void wait_vmem_dyn(int n) {
#define VMK_WAIT_CASE(k) case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
  switch (n) {
    VMK_WAIT_CASE(1) VMK_WAIT_CASE(2) VMK_WAIT_CASE(3) VMK_WAIT_CASE(4) VMK_WAIT_CASE(5) VMK_WAIT_CASE(6)
    VMK_WAIT_CASE(7) VMK_WAIT_CASE(8) VMK_WAIT_CASE(9) VMK_WAIT_CASE(10) VMK_WAIT_CASE(11) VMK_WAIT_CASE(12)
    VMK_WAIT_CASE(13) VMK_WAIT_CASE(14) VMK_WAIT_CASE(15) VMK_WAIT_CASE(16) VMK_WAIT_CASE(18) VMK_WAIT_CASE(20)
    VMK_WAIT_CASE(24) VMK_WAIT_CASE(27) VMK_WAIT_CASE(28) VMK_WAIT_CASE(32) VMK_WAIT_CASE(36) VMK_WAIT_CASE(40)
    VMK_WAIT_CASE(45) VMK_WAIT_CASE(48)
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
#undef VMK_WAIT_CASE
}

// Workgroup barrier that waits for this wave's LDS operations only (s_waitcnt lgkmcnt(0), then s_barrier).  The
// compiler's __syncthreads would also wait for every direct-to-LDS load in flight (s_waitcnt vmcnt(0)), i.e. drain
// the ring each tile; the walks wait for their own tiles explicitly before barriers that publish them.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Runs f(integral_constant<int, I>) for I = 0 .. N-1 in order while it returns true; false if one returned false.
template <int I, int N, class F>
__device__ __forceinline__ bool unroll_while(F& f) {
  if constexpr (I == N) {
    return true;
  } else {
    if (!f(std::integral_constant<int, I>())) return false;
    return unroll_while<I + 1, N>(f);
  }
}

// Per-lane byte offsets that are the same for every tile, computed once per walk, so that a tile costs no address
// arithmetic: the stage is a compile-time index in the unrolled walks and lands in the instructions' immediate
// offset fields.
//   dma[j & 3]: this lane's 16 B of DMA instruction j (rows 4j..4j+3) within a tile's 32 rows of 256 B, less 1024 j:
//           logical chunk (l & 15) ^ swz(row) of row 4j + (l >> 4), which lands at chunk position l & 15 of LDS block
//           j.  swz(4j + s) = (s << 2) | (j & 3) for s < 4, so the lane part depends on j & 3 only (dma_lane);
//   k[t]:   K operand of step t: row l % 32, logical chunk 8g + t (g = l / 32), from the ring base;
//   v[2dt + rr]: V^T half rr of d-tile dt at step 0 (step 1 is 16 rows = 4096 bytes further): source row
//           8rr + 4g + ((l & 15) >> 2), head-dim 32dt + 16((l >> 4) & 1) + 4(l & 3), from the ring base.  swz of
//           row + 16 equals swz of row, so step 1 really is a constant 4096 further.
struct TileLanes {
  uint32_t dma[4];
  uint32_t k[8];
  uint32_t v[8];
};

// Lane part of DMA instruction j's source offset within a tile (the whole offset is 1024 j + dma_lane(lane, j)).
__device__ __forceinline__ uint32_t dma_lane(int lane, int j) {
  const int sub = lane >> 4, row = 4 * (j & 3) + sub;
  return sub * 256 + (((lane & 15) ^ swz(row)) << 4);
}

__device__ __forceinline__ TileLanes tile_lanes(int lane, uint32_t ring_off) {
  TileLanes tl;
  const int r = lane & 31, g = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j) tl.dma[j] = dma_lane(lane, j);
#pragma unroll
  for (int t = 0; t < 8; ++t) tl.k[t] = ring_off + r * 256 + (((8 * g + t) ^ swz(r)) << 4);
  const int e = (lane & 15) >> 2, hc = (lane >> 4) & 1, a4 = lane & 3;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int row = 8 * rr + 4 * g + e;
      const int col = 32 * dt + 16 * hc + 4 * a4;                  // halfs
      const int chunk = (col >> 3) ^ swz(row);
      tl.v[2 * dt + rr] = ring_off + 8192 + row * 256 + (chunk << 4) + ((col & 7) << 1);
    }
  return tl;
}

// Buffer resource of one 8 KB tile half (32 rows of 256 B) at a uniform address: base, 8192 bytes in range (an
// offset outside the half would read zeros, never foreign memory), raw 32-bit dword format (word 3 = 0x00020000).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const f16* tile) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(tile), 0, 8192, 0x00020000);
}

// DMA instruction i (0..15) of a tile: i < 8 loads K rows 4i..4i+3 into LDS block i, i >= 8 the V rows of block
// i - 8 into the V half.  A whole tile inside the sequence (issue_dma_full) takes the rows at uniform base + per-lane
// offset; the last, partial tile of a walk (issue_dma_part) takes keys past src.kend from g_zero_row.  Whether a tile
// is whole is the same for the whole wave, and the callers take the two cases in separate branches so that the
// whole-tile path carries none of the partial tile's per-lane pointers.
// lp = dma_lane(lane, i & 7): the rows of block j = i & 7 start 1024 j bytes into the tile half, which the load takes
// as its scalar offset: a buffer load with the half's resource in scalar registers and lp as the only per-lane
// operand, so a whole tile costs no per-lane address arithmetic.
// A source whose tile rows are not contiguous (Src::kStrided) gives the bytes from one row to the next for the tile
// at key0, uniform over the wave (src.row_bytes(key0), a multiple of 256): block j then starts 4 j rows in, lane
// quarter q (lane / 16) reads row 4 j + q, and the resource spans the 32 rows.  The LDS layout does not change.
template <class Src>
__device__ __forceinline__ void issue_dma_full(char* __restrict__ stage, const Src& src, int key0, int i,
                                               uint32_t lp) {
  const int j = i & 7;
  const f16* tile = i < 8 ? src.ktile(key0) : src.vtile(key0);
  if constexpr (Src::kStrided) {
    const uint32_t rb = src.row_bytes(key0);
    const uint32_t lps = lp + (uint32_t)((threadIdx.x & 63) >> 4) * (rb - 256);
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(tile), 0, (int)(31 * rb + 256), 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, VMK_LPTR(stage + (i < 8 ? 0 : 8192) + j * 1024), 16, lps,
                                             (int)(4 * j * rb), 0, 0);
  } else {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(tile_rsrc(tile), VMK_LPTR(stage + (i < 8 ? 0 : 8192) + j * 1024), 16,
                                             lp, 1024 * j, 0, 0);
  }
}

template <class Src>
__device__ __forceinline__ void issue_dma_part(char* __restrict__ stage, const Src& src, int key0, int i,
                                               uint32_t lp, int lane) {
  const int j = i & 7;
  const f16* tile = i < 8 ? src.ktile(key0) : src.vtile(key0);
  const int row = 4 * j + (lane >> 4);
  const f16* rowp;
  if constexpr (Src::kStrided)
    rowp = reinterpret_cast<const f16*>(reinterpret_cast<const char*>(tile) + (size_t)row * src.row_bytes(key0));
  else
    rowp = tile + row * 128;
  const char* gp = reinterpret_cast<const char*>(key0 + row < src.kend ? rowp : g_zero_row) + (lp & 255);
  __builtin_amdgcn_global_load_lds(VMK_GPTR(gp), VMK_LPTR(stage + (i < 8 ? 0 : 8192) + j * 1024), 16, 0, 0);
}

// All 16 DMA instructions of one tile from one wave.
template <class Src>
__device__ __forceinline__ void issue_tile_dma(char* __restrict__ stage, const Src& src, int key0,
                                               const TileLanes& tl, int lane) {
  if (key0 + kTile <= src.kend) {
#pragma unroll
    for (int i = 0; i < 16; ++i) issue_dma_full(stage, src, key0, i, tl.dma[i & 3]);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) issue_dma_part(stage, src, key0, i, tl.dma[i & 3], lane);
  }
}

typedef short short4v __attribute__((ext_vector_type(4)));

// Transposed 8-byte LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes, lane 4a+c receives element c of
// the 8-byte chunks addressed by lanes a, 4+a, 8+a, 12+a (in that order).
__device__ __forceinline__ u32x2 lds_read_tr16(const char* p) {
  const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (short4v __attribute__((address_space(3)))*)(VMK_LPTR(p)));
  return __builtin_bit_cast(u32x2, v);
}

// One tile from a stage (stage = LDS base + compile-time stage offset; tl's offsets include the ring base):
// S^T = K.Q^T from the K rows, masked online softmax, O^T += V^T.P^T with the V^T operand read transposed from the V
// rows (rows of keys outside the sequence were loaded from g_zero_row).  The transposed read gives lane l the dim
// 32dt + (l & 31) of the four keys 16t + 8rr + 4g + e, e = 0..3, which are exactly the keys of P^T's elements
// 4rr..4rr+3.
// Read schedule: the 8 K operands and the first 4 transposed V halves are issued up front (12 <= 15 outstanding
// LDS reads, the counter's limit), the other 12 V halves two after each of the first six QK MFMAs, so their latency
// hides behind the QK chain and the softmax instead of being paid read by read.
template <class Src, class V>
__device__ __forceinline__ void compute_tile_lds(RowState& st, const V (&qb)[8], const char* __restrict__ stage,
                                                 const TileLanes& tl, const Src& src, int key0, int lane) {
  const int g = lane >> 5;
  u32x4 kk[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) kk[t] = *reinterpret_cast<const u32x4*>(stage + tl.k[t]);
  u32x2 vv[4][2][2];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) vv[dt][t][rr] = lds_read_tr16(stage + tl.v[2 * dt + rr] + 4096 * t);
  floatx16 s = floatx16{};
#pragma unroll
  for (int t = 0; t < 8; ++t) s = mfma32(as_v8<V>(kk[t]), qb[t], s);
  __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);     // DS reads: K operands, V halves of d-tile 0
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one QK MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);    // two more V halves
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  __builtin_amdgcn_sched_barrier(0);
  src.mask(s, key0, g);
  V pb[2];
  softmax_update(st, s, src.scale, pb);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const V va = as_v8<V>(u32x4{vv[dt][t][0][0], vv[dt][t][0][1], vv[dt][t][1][0], vv[dt][t][1][1]});
      st.o[dt] = mfma32(va, pb[t], st.o[dt]);
    }
}

// ---- a ring of NS stages shared by the NW waves of a workgroup; every wave consumes every tile.  Wave w issues
// the tile's DMA instructions w, w + NW, ... (16 / NW of them) and waits for its own.  The walk goes in pairs of
// tiles with one barrier per pair: tiles t, t + 1 are waited for together, the barrier makes both visible and frees
// the stages of t - 2, t - 1, which then take tiles t + NS - 2 and t + NS - 1, so NS - 2 tiles stay in flight.
// Between two barriers the waves of a SIMD drift apart over two tiles, so one wave's softmax meets the other's
// MFMAs (with one barrier per tile they start every tile together and their softmaxes collide): C4 -2.4 %, C2
// -1.4 % against a barrier per tile, measured A/B on two boxes.  The walk is unrolled by NS so every stage index is
// a compile-time constant: compute(S, t) gets it as an integral_constant.
template <int NS, int NW, class Src, class Compute>
__device__ __forceinline__ void ring_walk(char* ring, const Src& src, int kbeg, int ntiles, int wave, int lane,
                                          Compute compute) {
  static_assert(NS % 2 == 0 && NS >= 6, "pairs of stages");
  constexpr int DPW = 16 / NW;
  uint32_t dmaw[DPW];                                       // lane parts of this wave's instructions
#pragma unroll
  for (int q = 0; q < DPW; ++q) dmaw[q] = dma_lane(lane, (wave + q * NW) & 7);
  auto issue = [&](char* stage, int t) {
    const int key0 = kbeg + t * kTile;
    if (key0 + kTile <= src.kend) {
#pragma unroll
      for (int q = 0; q < DPW; ++q) issue_dma_full(stage, src, key0, wave + q * NW, dmaw[q]);
    } else {
#pragma unroll
      for (int q = 0; q < DPW; ++q) issue_dma_part(stage, src, key0, wave + q * NW, dmaw[q], lane);
    }
  };
  auto pre = [&](auto S) {
    if (S >= ntiles) return false;
    issue(ring + S * kStageBytes, S);
    return true;
  };
  // Tiles requested before the first pair: with four waves (the mixed prefix launch's short walks of 128 rows) only
  // two, so that the first tiles land sooner (C1 12.16 against 12.49 us); the rest of the ring is requested at the
  // first barrier.  Eight waves request NS - 2 at once (fewer gave no gain at C2 and C4).
  constexpr int KI = NW == 4 ? 2 : NS - 2;
  unroll_while<0, KI>(pre);
  for (int t0 = 0; t0 < ntiles; t0 += NS) {
    auto step = [&](auto P) {
      constexpr int S = 2 * P;
      const int t = t0 + S;
      if (t >= ntiles) return false;
      bool first = false;                                   // first pair: the tiles after the KI requested
      if constexpr (KI < NS - 2) first = S == 0 && t == 0;
      if (first) {
        wait_vmem_dyn(DPW * max(0, min(KI, ntiles) - 2));
        lds_barrier();
        auto late = [&](auto S2) {
          if (S2 >= ntiles) return false;
          issue(ring + S2 * kStageBytes, S2);
          return true;
        };
        unroll_while<KI, NS>(late);
      } else {
        wait_vmem_dyn(DPW * max(0, min(NS - 4, ntiles - 2 - t)));
        lds_barrier();
        if (t + NS - 2 < ntiles) issue(ring + ((S + NS - 2) % NS) * kStageBytes, t + NS - 2);
        if (t + NS - 1 < ntiles) issue(ring + ((S + NS - 1) % NS) * kStageBytes, t + NS - 1);
      }
      compute(std::integral_constant<int, S>(), t);
      if (t + 1 < ntiles) compute(std::integral_constant<int, S + 1>(), t + 1);
      return true;
    };
    if (!unroll_while<0, NS / 2>(step)) break;
  }
}

// One wave's walk over the tiles t0, t0+tstep, ... (< ntiles) of [kbeg, ...) through a private ring of NS stages
// (NS - 1 tiles in flight while one is computed; NS <= 4 keeps the wait counts within vmcnt's range), unrolled by NS
// so every stage offset is a compile-time constant.  ring is this wave's ring (DMA destinations); base is the LDS
// address the read offsets of tl are relative to (they include the ring's offset from it).
// The key source `src` provides: ktile(key0) / vtile(key0) (the first of the 32 K / V rows of the tile starting at
// key0, a multiple of 32 from the range start; rows at or past kend are not read; the rows are 256 bytes apart, or
// src.row_bytes(key0) apart when Src::kStrided), kend, scale (log2-domain softmax scale) and mask(s, key0, g)
// (masked scores of the raw S^T tile -> -inf).
template <int NS, class Src, class V>
__device__ __forceinline__ void wave_walk(RowState& st, const V (&qb)[8], char* __restrict__ ring,
                                          const char* __restrict__ base, const TileLanes& tl, const Src& src,
                                          int kbeg, int t0, int ntiles, int tstep, int lane) {
  static_assert(NS >= 2 && NS <= 4, "1 to 3 tiles in flight");
  if (t0 >= ntiles) return;
  const int n = (ntiles - t0 + tstep - 1) / tstep;          // tiles of this wave
  auto key_of = [&](int j) { return kbeg + (t0 + j * tstep) * kTile; };
  auto pre = [&](auto S) {
    if (S >= n) return false;
    issue_tile_dma(ring + S * kStageBytes, src, key_of(S), tl, lane);
    return true;
  };
  unroll_while<0, NS - 1>(pre);
  for (int j0 = 0; j0 < n; j0 += NS) {
    auto step = [&](auto S) {
      const int j = j0 + S, jn = j + NS - 1;
      if (j >= n) return false;
      asm volatile("" ::: "memory");
      // Stage (S + NS - 1) % NS last held tile j - 1, whose LDS reads all returned before its MFMAs used them.
      if (jn < n) issue_tile_dma(ring + ((S + NS - 1) % NS) * kStageBytes, src, key_of(jn), tl, lane);
      wait_vmem_dyn(16 * min(NS - 1, n - 1 - j));
      compute_tile_lds(st, qb, base + S * kStageBytes, tl, src, key_of(j), lane);
      return true;
    };
    if (!unroll_while<0, NS>(step)) break;
  }
}

// ---- paged caches
// Keys [kbeg, kend) of one KV head of a sequence in a paged cache: pages of ps rows (ps a multiple of 32, so a tile
// never straddles two pages) laid out (num_pages, Hkv, ps, 128) (HND: a page's rows of one head are contiguous) or,
// with kNHD, (num_pages, ps, Hkv, 128) (a page's rows are Hkv * 256 bytes apart), the sequence's pages listed in
// `table`.  Lane t holds the K and V row addresses of the range's tile t (keys kbeg + 32 t ..; kbeg is a multiple of
// 32 and a range has at most 2048 keys, i.e. 64 tiles), worked out once per lane, so a tile finds its rows with
// readlanes only (no division or multiply per tile).  An id outside [0, num_pages) is an absent page: its tiles read
// a zero tile (contiguous rows in either layout) and its keys are masked out.
template <bool kNHD>
struct PagedSrc {
  const f16* kt;           // this lane's tile: K rows, or g_zero_tile when its page is absent
  const f16* vt;           //                   V rows
  int here;                // 1 when this lane's tile has a page
  int kbeg, kend;
  float scale;
  uint32_t rb_page;        // NHD: bytes between the rows of a page (Hkv * 256)
  static constexpr bool kStrided = kNHD;
  __device__ int tile(int key0) const { return (key0 - kbeg) >> 5; }
  __device__ uint32_t row_bytes(int key0) const { return present(key0) ? rb_page : 256u; }
  __device__ static const f16* lane_ptr(const f16* p, int t) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, t), hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), t);
    return reinterpret_cast<const f16*>(((uint64_t)hi << 32) | lo);
  }
  __device__ bool present(int key0) const { return __builtin_amdgcn_readlane(here, tile(key0)) != 0; }
  __device__ const f16* ktile(int key0) const { return lane_ptr(kt, tile(key0)); }
  __device__ const f16* vtile(int key0) const { return lane_ptr(vt, tile(key0)); }
  __device__ void mask(floatx16& s, int key0, int g) const {
    const bool here = present(key0);
    if (here && key0 + kTile <= kend) return;              // whole tile inside (same for the whole wave)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key = key0 + 8 * blk + 4 * g + c;
        s[4 * blk + c] = here && key < kend ? s[4 * blk + c] : kNegInf;
      }
  }
};

// The source of KV head h for keys [kbeg, kend) of a sequence whose pages `table` lists (ntable entries), in the
// pools kpool / vpool of num_pages pages of ps rows with Hkv heads; scale is the log2-domain softmax scale.
template <bool kNHD>
__device__ __forceinline__ PagedSrc<kNHD> paged_src(const f16* kpool, const f16* vpool, int ps, int Hkv,
                                                    int num_pages, float scale, const int* table, int ntable, int h,
                                                    int kbeg, int kend) {
  PagedSrc<kNHD> s;
  s.kbeg = kbeg;
  s.kend = kend;
  s.scale = scale;
  s.rb_page = (uint32_t)Hkv * 256u;
  const int key = kbeg + kTile * (int)(threadIdx.x & 63);     // this lane's tile
  const int slot = key / ps;
  const int page = key < kend && slot < ntable ? table[slot] : -1;
  s.here = (unsigned)page < (unsigned)num_pages;
  const size_t row = key - slot * ps;                        // the tile's first row within its page
  const size_t off = (kNHD ? ((size_t)page * ps + row) * Hkv + h : ((size_t)page * Hkv + h) * ps + row) * 128;
  s.kt = s.here ? kpool + off : g_zero_tile;
  s.vt = s.here ? vpool + off : g_zero_tile;
  return s;
}

// LDS slot of one wave's state for the cross-wave merge: O as 16 floatx4 per lane, register-major (each b128 access
// of a wave covers 1 KB contiguously), then (m, l) per lane.
constexpr int kSlotBytes = 64 * 64 * 4 + 64 * 8;

__device__ __forceinline__ void state_to_slot(char* slot, const RowState& st, int lane) {
  floatx4* o = reinterpret_cast<floatx4*>(slot);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
      o[(dt * 4 + blk) * 64 + lane] =
          floatx4{st.o[dt][4 * blk], st.o[dt][4 * blk + 1], st.o[dt][4 * blk + 2], st.o[dt][4 * blk + 3]};
  reinterpret_cast<float2*>(slot + 64 * 64 * 4)[lane] = float2{st.m, st.l};
}

// Writes one wave's partial for its 32 rows: po[row][d] = O / l in the partial type PT (row stride 128),
// pml[row] = (m, l).  Rows >= nvalid are skipped.  kCoherent: agent-coherent stores, for a reader in the same kernel.
template <bool kCoherent = false, class PT>
__device__ __forceinline__ void store_partial(PT* po, float* pml, const RowState& st, int lane, int nvalid) {
  const int r = lane & 31, g = lane >> 5;
  const float ltot = st.l + xor32(st.l);
  if (r >= nvalid) return;
  const float inv = part_inv(ltot);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      floatx4 v = floatx4{st.o[dt][4 * blk], st.o[dt][4 * blk + 1], st.o[dt][4 * blk + 2], st.o[dt][4 * blk + 3]};
      if constexpr (kCoherent)
        store_part4_coherent(po + r * 128 + dt * 32 + 8 * blk + 4 * g, v * inv);
      else
        store_part4(po + r * 128 + dt * 32 + 8 * blk + 4 * g, v * inv);
    }
  if (g == 0) {
    if constexpr (kCoherent) {
      store_u64_coherent(pml + 2 * r, __builtin_bit_cast(uint64_t, float2{st.m, ltot}));
    } else {
      pml[2 * r] = st.m;
      pml[2 * r + 1] = ltot;
    }
  }
}

// ---- one workgroup of WR x WK waves (WR * WK = 4, 256 threads): WR row blocks of 32 rows, WK waves interleaving the
// tiles of [kbeg, kbeg + 32*ntiles) through private rings of NSW stages.  Writes one partial (O, m, l) for the WG's
// 32*WR rows to po (row stride 128 floats) / pml; rows >= nrows are skipped.  po/pml may point into smem past
// kAttnSlotsEnd.  Cross-wave merge: every wave parks its state in a slot, then wave wk of row block wr merges
// d-tiles wk, wk + WK, ... of all WK slots and stores them, so the merge work is spread over all waves.
// qrow(row) returns an in-bounds Q row pointer for a WG-local row (clamped by the caller for rows >= nrows).
constexpr int kAttnSmemBytes = 8 * kStageBytes;
constexpr int kAttnSlotsEnd = 4 * kSlotBytes;
static_assert(kAttnSlotsEnd <= kAttnSmemBytes, "merge slots must fit in the stage memory");

template <int WR, int WK, int NSW = 2, class V = half8, class Src, class QRow, class PT>
__device__ __forceinline__ void attend_wg(char* smem, const Src& src, QRow qrow, int nrows, int kbeg, int ntiles,
                                          PT* po, float* pml) {
  static_assert(WR * WK == 4 && WR * WK * NSW <= 8, "four waves, rings within the stage memory");
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave % WR, wk = wave / WR;
  const int r = lane & 31, g = lane >> 5;
  const int row = wr * 32 + r;
  V qb[8];
  load_qt(qb, qrow(row < nrows ? row : 0), g, row < nrows);
  RowState st;
  row_state_init(st);
  const uint32_t ring_off = (uint32_t)wave * NSW * kStageBytes;
  const TileLanes tl = tile_lanes(lane, ring_off);
  wave_walk<NSW>(st, qb, smem + ring_off, smem, tl, src, kbeg, wk, ntiles, WK, lane);
  const int nvalid = nrows - wr * 32;
  PT* pob = po + (size_t)wr * 32 * 128;
  float* pmlb = pml + wr * 32 * 2;
  if constexpr (WK == 1) {
    store_partial(pob, pmlb, st, lane, nvalid);
  } else {
    __syncthreads();                                        // every walk is done: the rings become slots
    state_to_slot(smem + wave * kSlotBytes, st, lane);
    __syncthreads();
    float mk[WK], M = kNegInf;
#pragma unroll
    for (int k = 0; k < WK; ++k) {
      const float2 ml = reinterpret_cast<const float2*>(smem + (k * WR + wr) * kSlotBytes + 64 * 64 * 4)[lane];
      mk[k] = ml.x;
      M = fmaxf(M, ml.x);
    }
    const float muse = (M == kNegInf) ? 0.f : M;
    float ak[WK], l = 0.f;
#pragma unroll
    for (int k = 0; k < WK; ++k) {
      ak[k] = fast_exp2(mk[k] - muse);
      l += ak[k] * reinterpret_cast<const float2*>(smem + (k * WR + wr) * kSlotBytes + 64 * 64 * 4)[lane].y;
    }
    const float ltot = l + xor32(l);
    const float inv = part_inv(ltot);
#pragma unroll
    for (int j = 0; j < 4 / WK; ++j) {
      const int dt = wk + j * WK;
      floatx4 acc[4];
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) acc[blk] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < WK; ++k) {
        const floatx4* o = reinterpret_cast<const floatx4*>(smem + (k * WR + wr) * kSlotBytes);
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) acc[blk] += ak[k] * o[(dt * 4 + blk) * 64 + lane];
      }
      if (r < nvalid)
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) store_part4(pob + r * 128 + dt * 32 + 8 * blk + 4 * g, acc[blk] * inv);
    }
    if (wk == 0 && g == 0 && r < nvalid) {
      pmlb[2 * r] = M;
      pmlb[2 * r + 1] = ltot;
    }
  }
}

// ---- log-sum-exp merge of the partials of one output row, NT threads, PER head-dims per thread (d = tid + k*NT).
// part(i, ml, o) sets ml -> (m, l) and o -> the partial's normalised O row (type PT) of partial i (0 <= i < nparts).
// Partial i weighs w_i = exp2(m_i - M) * l_i, M the largest m: out = sum_i w_i O_i / sum_i w_i.  The m/l of a batch
// of NT partials are fetched in parallel and their weights shared through LDS, so that the O loads of the
// accumulation loop are independent of each other and can all be in flight together.
//
// Up to 32 partials (every bench shape: 8-32), the O rows are loaded into registers together with the m/l, before
// the maximum is known, so the merge waits for one round of loads instead of three.  The H loads are unconditional
// (slots past nparts reload the last partial, never used) so that they issue back to back; nparts >= 1 here, which
// combine_row guarantees.  Both forms add the same terms in the same order (partial 0 first), so they give the same
// bits.
template <int NT, int PER, int H, class PT, class Part, class E>
__device__ __forceinline__ void combine_row_held(int nparts, Part part, E* out) {
  __shared__ float sw[H], red[NT / 64];
  const int tid = threadIdx.x;
  float ov[H][PER];
#pragma unroll
  for (int j = 0; j < H; ++j) {
    const float* ml;
    const PT* o;
    part(min(j, nparts - 1), ml, o);
#pragma unroll
    for (int k = 0; k < PER; ++k) ov[j][k] = (float)o[tid + k * NT];
  }
  float m0 = kNegInf, l0 = 0.f;
  if (tid < nparts) {
    const float* ml;
    const PT* o;
    part(tid, ml, o);
    m0 = ml[0];
    l0 = ml[1];
  }
  float M = m0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = M;
  __syncthreads();
  M = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) M = fmaxf(M, red[w]);
  const float Muse = (M == kNegInf) ? 0.f : M;
  if (tid < nparts) sw[tid] = fast_exp2(m0 - Muse) * l0;
  __syncthreads();
  float num[PER], den = 0.f;
#pragma unroll
  for (int k = 0; k < PER; ++k) num[k] = 0.f;
#pragma unroll
  for (int j = 0; j < H; ++j) {
    if (j < nparts) {                                  // uniform
      const float w = sw[j];
      den += w;
#pragma unroll
      for (int k = 0; k < PER; ++k) num[k] += w * ov[j][k];
    }
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) out[tid + k * NT] = (E)(num[k] / den);
}

template <int NT, int PER, class PT, class Part, class E>
__device__ __forceinline__ void combine_row(int nparts, Part part, E* out) {
  static_assert(NT >= 32, "one thread per held partial's m/l");
  if (nparts <= 0) {                                 // uniform: no partial to merge, and none is read
    // The softmax of no keys is 0 / 0.
#pragma unroll
    for (int k = 0; k < PER; ++k) out[threadIdx.x + k * NT] = (E)__builtin_nanf("");
    return;
  }
  if (nparts <= 8) return combine_row_held<NT, PER, 8, PT>(nparts, part, out);
  if (nparts <= 16) return combine_row_held<NT, PER, 16, PT>(nparts, part, out);
  if (nparts <= 32) return combine_row_held<NT, PER, 32, PT>(nparts, part, out);
  __shared__ float sw[NT], red[NT / 64];
  const int tid = threadIdx.x;
  float M = kNegInf;
  for (int b0 = 0; b0 < nparts; b0 += NT) {
    if (b0 + tid < nparts) {
      const float* ml;
      const PT* o;
      part(b0 + tid, ml, o);
      M = fmaxf(M, ml[0]);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = M;
  __syncthreads();
  M = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) M = fmaxf(M, red[w]);
  const float Muse = (M == kNegInf) ? 0.f : M;
  float num[PER], den = 0.f;
#pragma unroll
  for (int k = 0; k < PER; ++k) num[k] = 0.f;
  for (int b0 = 0; b0 < nparts; b0 += NT) {
    const int n = min(NT, nparts - b0);
    __syncthreads();
    if (tid < n) {
      const float* ml;
      const PT* o;
      part(b0 + tid, ml, o);
      sw[tid] = fast_exp2(ml[0] - Muse) * ml[1];
    }
    __syncthreads();
#pragma unroll 8
    for (int j = 0; j < n; ++j) {
      const float* ml;
      const PT* o;
      part(b0 + j, ml, o);
      const float w = sw[j];
      den += w;
#pragma unroll
      for (int k = 0; k < PER; ++k) num[k] += w * (float)o[tid + k * NT];
    }
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) out[tid + k * NT] = (E)(num[k] / den);
}

// ---- the same merge by a group of lanes per output row, eight head-dims per lane (one 16-byte load of an fp16
// partial row, two of an fp32 one, instead of a 2-byte load per thread and partial).  part(i, ml, o) sets ml -> the
// (m, l) pair of partial i and o -> this lane's eight elements of partial i's normalised O row.  Every lane loads the
// (m, l) of every partial itself (the lanes of a row read the same addresses), so the weights need no exchange
// between lanes.  The maximum, the weights exp2(m_i - M) * l_i, their order (partial 0 first) and the arithmetic are
// those of combine_row, so both give the same bits.
template <class PT>
struct Part8 {
  static constexpr int kWords = sizeof(PT) / 2;              // 16-byte words of eight elements
  u32x4 w[kWords];
  __device__ __forceinline__ void load(const PT* p) {
#pragma unroll
    for (int i = 0; i < kWords; ++i) w[i] = ldg16(reinterpret_cast<const char*>(p) + 16 * i);
  }
  __device__ __forceinline__ float get(int k) const {
    if constexpr (kWords == 1)
      return (float)as_h8(w[0])[k];
    else
      return __uint_as_float(w[k >> 2][k & 3]);
  }
};

template <class E>
__device__ __forceinline__ void store_out8(E* out, const float (&num)[8], float den) {
  typedef E e8 __attribute__((ext_vector_type(8)));
  e8 v;
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = (E)(num[k] / den);
  *reinterpret_cast<e8*>(out) = v;
}

// Weight exp2(m - M) * l of a partial, rounded before it is used: the product is not fused into the sum of the
// weights (combine_row rounds it through LDS), so both merges add the same rounded weights.
__device__ __forceinline__ float part_weight(float2 ml, float Muse) {
#pragma clang fp contract(off)
  return fast_exp2(ml.x - Muse) * ml.y;
}

// Up to H partials, all loaded before the first is used (one memory round trip).  nparts >= 1.
template <int H, class PT, class Part, class E>
__device__ __forceinline__ void combine_vec_held(int nparts, Part part, E* out) {
  Part8<PT> ov[H];
  float2 ml[H];
#pragma unroll
  for (int j = 0; j < H; ++j) {                      // slots past nparts reload the last partial, never used
    const float* mlp;
    const PT* o;
    part(min(j, nparts - 1), mlp, o);
    ml[j] = *reinterpret_cast<const float2*>(mlp);
    ov[j].load(o);
  }
  float M = kNegInf;
#pragma unroll
  for (int j = 0; j < H; ++j)
    if (j < nparts) M = fmaxf(M, ml[j].x);
  const float Muse = (M == kNegInf) ? 0.f : M;
  float num[8], den = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) num[k] = 0.f;
#pragma unroll
  for (int j = 0; j < H; ++j) {
    if (j < nparts) {
      const float w = part_weight(ml[j], Muse);
      den += w;
#pragma unroll
      for (int k = 0; k < 8; ++k) num[k] += w * ov[j].get(k);
    }
  }
  store_out8(out, num, den);
}

template <class PT, class Part, class E>
__device__ __forceinline__ void combine_vec(int nparts, Part part, E* out) {
  if (nparts <= 0) {                                 // the softmax of no keys is 0 / 0
    float num[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) num[k] = __builtin_nanf("");
    store_out8(out, num, 1.f);
    return;
  }
  if (nparts <= 8) return combine_vec_held<8, PT>(nparts, part, out);
  if (nparts <= 16) return combine_vec_held<16, PT>(nparts, part, out);
  if (nparts <= 32 && sizeof(PT) == 2) return combine_vec_held<32, PT>(nparts, part, out);
  // More partials: the maximum over all of them first, then the weighted sum in batches of 16, in order.
  constexpr int kB = 16;
  float M = kNegInf;
  for (int b0 = 0; b0 < nparts; b0 += kB) {
    float mb[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const float* mlp;
      const PT* o;
      part(min(b0 + j, nparts - 1), mlp, o);
      mb[j] = mlp[0];
    }
#pragma unroll
    for (int j = 0; j < kB; ++j)
      if (b0 + j < nparts) M = fmaxf(M, mb[j]);
  }
  const float Muse = (M == kNegInf) ? 0.f : M;
  float num[8], den = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) num[k] = 0.f;
  for (int b0 = 0; b0 < nparts; b0 += kB) {
    Part8<PT> ov[kB];
    float2 ml[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const float* mlp;
      const PT* o;
      part(min(b0 + j, nparts - 1), mlp, o);
      ml[j] = *reinterpret_cast<const float2*>(mlp);
      ov[j].load(o);
    }
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (b0 + j < nparts) {
        const float w = part_weight(ml[j], Muse);
        den += w;
#pragma unroll
        for (int k = 0; k < 8; ++k) num[k] += w * ov[j].get(k);
      }
    }
  }
  store_out8(out, num, den);
}

// ---- one workgroup of NW waves sharing a ring of kRowsStages stages: wave w owns rows [32w, 32w+32) and every wave
// consumes every tile of [kbeg, kbeg + 32*ntiles).  Writes the WG's partial (32*NW rows) like attend_wg.
// Eight stages (128 KB): six tiles in flight beside the pair being computed, and one workgroup per CU (two would not
// fit).  LDS reads address
// stages 0-3 from the per-lane offsets of tl and stages 4-7 from those of tl_hi (64 KB further), so every stage
// offset fits the 16-bit immediate field.
constexpr int kRowsStages = 8;
constexpr int kRowsSmemBytes = kRowsStages * kStageBytes;

// The row-split workgroup's partial (NW waves x 32 rows), written through LDS so that every store instruction
// writes two whole rows (contiguous) instead of pieces of 32 rows.  Each wave parks its O^T registers, normalised by
// its rows' l, in its own 16 KB of LDS as 32 rows of 128 floats, the 16-byte chunk c of row r at chunk position
// (c + r) mod 32 (at most two lanes per bank group on the writes, none on the row reads), then stores rows 2i,
// 2i + 1 per instruction in the partial type PT, as non-temporal stores (the row split's partials are read by a
// later launch).  Called by every wave of the workgroup (it contains a barrier); rows >= nvalid are not written.
// kCoherent: agent-coherent stores instead, for a reader in the same kernel.
// store_partial_rows_wave is the same for one wave alone, through the 16 KB of LDS at wlds that no other wave uses
// (a single-wave unit's own ring, once its walk is done): no workgroup barrier.
template <bool kCoherent = false, class PT>
__device__ __forceinline__ void store_partial_rows_wave(char* wlds, PT* po, float* pml, const RowState& st, int lane,
                                                        int nvalid) {
  float* lds = reinterpret_cast<float*>(wlds);
  const int r = lane & 31, g = lane >> 5;
  const float ltot = st.l + xor32(st.l);
  const float inv = part_inv(ltot);                         // the lane's row r, normalised before the transpose
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
      *reinterpret_cast<floatx4*>(lds + r * 128 + (((dt * 8 + 2 * blk + g) + r) & 31) * 4) =
          floatx4{st.o[dt][4 * blk], st.o[dt][4 * blk + 1], st.o[dt][4 * blk + 2], st.o[dt][4 * blk + 3]} * inv;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");       // the wave reads back only its own rows
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 2 * i + g;
    const floatx4 v = *reinterpret_cast<const floatx4*>(lds + row * 128 + ((r + row) & 31) * 4);
    if (row < nvalid) {
      if constexpr (kCoherent)
        store_part4_coherent(po + row * 128 + r * 4, v);
      else
        store_part4_nt(po + row * 128 + r * 4, v);
    }
  }
  if (g == 0 && r < nvalid) {
    if constexpr (kCoherent)
      store_u64_coherent(pml + 2 * r, __builtin_bit_cast(uint64_t, float2{st.m, ltot}));
    else
      *reinterpret_cast<float2*>(pml + 2 * r) = float2{st.m, ltot};
  }
}

template <bool kCoherent = false, class PT>
__device__ __forceinline__ void store_partial_rows(char* smem, PT* po, float* pml, const RowState& st, int wave,
                                                   int lane, int nvalid) {
  __syncthreads();                                          // every wave is done with the ring
  store_partial_rows_wave<kCoherent>(smem + wave * 32 * 128 * 4, po, pml, st, lane, nvalid);
}

template <int NW, class V = half8, bool kCoherent = false, class Src, class QRow, class PT>
__device__ __forceinline__ void attend_wg_rows(char* smem, const Src& src, QRow qrow, int nrows, int kbeg,
                                               int ntiles, PT* po, float* pml) {
  static_assert(16 % NW == 0, "the 16 DMA instructions of a tile must split evenly over the waves");
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = wave * 32 + (lane & 31);
  V qb[8];
  load_qt(qb, qrow(row < nrows ? row : 0), lane >> 5, row < nrows);
  RowState st;
  row_state_init(st);
  const bool has_rows = wave * 32 < nrows;
  // Waves 0-3 and 4-7 share the SIMDs pairwise; the first of each pair issues first when both are ready, which
  // keeps the pair apart within a barrier interval (with 8 waves; C4 -0.6 % on top of the pair barriers).
  if (NW == 8 && wave < 4) __builtin_amdgcn_s_setprio(1);
  const TileLanes tl = tile_lanes(lane, 0), tl_hi = tile_lanes(lane, 4 * kStageBytes);
  ring_walk<kRowsStages, NW>(smem, src, kbeg, ntiles, wave, lane, [&](auto S, int t) {
    if (has_rows)
      compute_tile_lds(st, qb, smem + (S & 3) * kStageBytes, S < 4 ? tl : tl_hi, src, kbeg + t * kTile, lane);
  });
  static_assert(NW * 32 * 128 * 4 <= kRowsSmemBytes, "the partial's transpose fits in the ring");
  store_partial_rows<kCoherent>(smem, po + (size_t)wave * 32 * 128, pml + wave * 32 * 2, st, wave, lane,
                                nrows - wave * 32);
}

}  // namespace vmk
