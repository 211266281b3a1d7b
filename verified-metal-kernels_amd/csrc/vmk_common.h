// Shared device helpers of libvmk (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

namespace vmk {

typedef _Float16 f16;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// 32x32x16 fp16 MFMA, fp32 accumulate.  Operand layout (wave64):
//   A (32 x 16): lane l holds row l%32, k-group l/32, 8 consecutive k of that group;
//   B (16 x 32): lane l holds column l%32, same k-group/elements as A;
//   D (32 x 32): lane l holds column l%32 and rows 8*blk + 4*(l/32) + c in register 4*blk + c.
// Only the pairing of A's and B's k-elements matters for the product, so callers may map the 16 k-slots of one
// instruction onto any 16 logical k indices as long as A and B use the same map.
__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// The same with bf16 operands (same operand and result layout).
__device__ __forceinline__ floatx16 mfma32(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Element type of an 8-wide MFMA operand vector (half8 -> _Float16, bf16x8 -> __bf16): the attention core is written
// once over the operand type V; keys, values and queries are moved as raw 16-bit bits and only interpreted here.
template <class V> struct ElemOf;
template <> struct ElemOf<half8> { typedef f16 type; };
template <> struct ElemOf<bf16x8> { typedef bf16 type; };
template <class V> using elem_t = typename ElemOf<V>::type;

// Storage type of a split partial's row-normalised O (O / l), keyed by the input element type: fp16 for fp16 inputs
// (a normalised row is a convex combination of value rows, so |O / l| <= max |v| <= 65504 fits, and its rounding
// is that of one more fp16 result), fp32 for bf16 inputs (whose values can exceed fp16's range).
template <class E> struct PartOf { typedef float type; };
template <> struct PartOf<f16> { typedef f16 type; };
template <class E> using part_t = typename PartOf<E>::type;

// Four floats stored as one piece of a partial row (16 bytes of fp32 or 8 bytes of fp16), and two of them read back.
__device__ __forceinline__ void store_part4(float* p, floatx4 v) { *reinterpret_cast<floatx4*>(p) = v; }
__device__ __forceinline__ void store_part4(f16* p, floatx4 v) {
  *reinterpret_cast<half4*>(p) = half4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
}
// The same as non-temporal stores, for partials that are read back only by a later launch: they stream to memory
// instead of waiting in L2 for the end-of-kernel writeback (C2's prefix partials -2 %; partials that a combine reads
// right after, as C3's, lose by it).
__device__ __forceinline__ void store_part4_nt(float* p, floatx4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(p));
}
__device__ __forceinline__ void store_part4_nt(f16* p, floatx4 v) {
  __builtin_nontemporal_store(half4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]}, reinterpret_cast<half4*>(p));
}
// The same as agent-coherent (sc1) stores: they reach the device's coherence point, so another XCD may read them in
// the same kernel with agent-coherent loads (load_part2_coherent) once the storing waves' counters have drained.
__device__ __forceinline__ void store_u64_coherent(void* p, uint64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_part4_coherent(float* p, floatx4 v) {
  store_u64_coherent(p, __builtin_bit_cast(uint64_t, float2{v[0], v[1]}));
  store_u64_coherent(p + 2, __builtin_bit_cast(uint64_t, float2{v[2], v[3]}));
}
__device__ __forceinline__ void store_part4_coherent(f16* p, floatx4 v) {
  store_u64_coherent(p, __builtin_bit_cast(uint64_t, half4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]}));
}
__device__ __forceinline__ float2 load_part2(const float* p) { return *reinterpret_cast<const float2*>(p); }
__device__ __forceinline__ float2 load_part2(const f16* p) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = *reinterpret_cast<const h2*>(p);
  return float2{(float)v[0], (float)v[1]};
}

// Agent-coherent (sc1) loads of two partial elements and of an (m, l) pair.
__device__ __forceinline__ float2 load_part2_coherent(const float* p) {
  return __builtin_bit_cast(float2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ float2 load_part2_coherent(const f16* p) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = __builtin_bit_cast(h2, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT));
  return float2{(float)v[0], (float)v[1]};
}

// 1 / l of a partial row, or 0 when the row saw no key (l = 0, O = 0): its normalised O is then 0, not 0/0.  A NaN
// l gives NaN, which the merge carries into the output.
__device__ __forceinline__ float part_inv(float l) { return l == 0.f ? 0.f : 1.f / l; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value of lane l ^ 32.  v_permlane32_swap exchanges the upper half of its first operand with the lower half of
// its second: with both operands x, lanes 0-31 find x[l + 32] in the second result and lanes 32-63 find x[l - 32]
// in the first.  A VALU op, so it neither waits for nor queues behind outstanding LDS reads (ds_bpermute would).
__device__ __forceinline__ float xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Wave-wide reduction with DPP moves (VALU only, no LDS): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and
// row_mirror reduce each row of 16 lanes; row_bcast:15 (into rows 1, 3) and row_bcast:31 (into rows 2, 3) carry the
// row results up, so lane 63 holds the total, which is returned to every lane.  Lanes a DPP move does not write
// keep `identity`.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_move(float identity, float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}

template <class Op>
__device__ __forceinline__ float wave_reduce(float x, float identity, Op op) {
  x = op(x, dpp_move<0xB1, 0xF>(identity, x));
  x = op(x, dpp_move<0x4E, 0xF>(identity, x));
  x = op(x, dpp_move<0x141, 0xF>(identity, x));
  x = op(x, dpp_move<0x140, 0xF>(identity, x));
  x = op(x, dpp_move<0x142, 0xA>(identity, x));
  x = op(x, dpp_move<0x143, 0xC>(identity, x));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

__device__ __forceinline__ float wave_max(float x) {
  return wave_reduce(x, -__builtin_huge_valf(), [](float a, float b) { return fmaxf(a, b); });
}

__device__ __forceinline__ float wave_sum(float x) {
  return wave_reduce(x, 0.f, [](float a, float b) { return a + b; });
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves (VALU only, no LDS round trips): row_shr:1, 2, 4
// and 8 scan each row of 16 lanes (lanes shifted in from before the row's start read 0), then row_bcast:15 adds
// row 0's and row 2's totals into rows 1 and 3, and row_bcast:31 adds lane 31's prefix into rows 2 and 3.  A lane
// a DPP move does not write adds 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, false);
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += dpp_u32<0x111, 0xF>(x);
  x += dpp_u32<0x112, 0xF>(x);
  x += dpp_u32<0x114, 0xF>(x);
  x += dpp_u32<0x118, 0xF>(x);
  x += dpp_u32<0x142, 0xA>(x);
  x += dpp_u32<0x143, 0xC>(x);
  return x;
}

__device__ __forceinline__ half8 zero_h8() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }

__device__ __forceinline__ half8 as_h8(u32x4 u) { return __builtin_bit_cast(half8, u); }

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Loads through a global (address space 1) pointer: p must point to global memory.  A pointer chosen between two
// global objects is generic to the compiler, whose flat loads also count as LDS operations and order against them.
__device__ __forceinline__ u32x4 ldg16(const void* p) {
  return *reinterpret_cast<const u32x4 __attribute__((address_space(1)))*>(
      (const void __attribute__((address_space(1)))*)(p));
}
__device__ __forceinline__ uint32_t ldg4(const void* p) {
  return *reinterpret_cast<const uint32_t __attribute__((address_space(1)))*>(
      (const void __attribute__((address_space(1)))*)(p));
}

// 16-bit lane i (0..7) of eight 16-byte rows -> one 16-byte column (row j in 16-bit lane j).
__device__ __forceinline__ u32x4 column8(const u32x4 (&r)[8], int i) {
  const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
  const int w = i >> 1;
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(r[1][w], r[0][w], sel);
  o[1] = __builtin_amdgcn_perm(r[3][w], r[2][w], sel);
  o[2] = __builtin_amdgcn_perm(r[5][w], r[4][w], sel);
  o[3] = __builtin_amdgcn_perm(r[7][w], r[6][w], sel);
  return o;
}

__device__ __forceinline__ half8 pack8(float a0, float a1, float a2, float a3, float a4, float a5, float a6,
                                       float a7) {
  return half8{(f16)a0, (f16)a1, (f16)a2, (f16)a3, (f16)a4, (f16)a5, (f16)a6, (f16)a7};
}
// Eight floats rounded to the operand type V (round to nearest even).
template <class V>
__device__ __forceinline__ V pack8v(float a0, float a1, float a2, float a3, float a4, float a5, float a6, float a7) {
  typedef elem_t<V> E;
  return V{(E)a0, (E)a1, (E)a2, (E)a3, (E)a4, (E)a5, (E)a6, (E)a7};
}
template <class V> __device__ __forceinline__ V as_v8(u32x4 u) { return __builtin_bit_cast(V, u); }

}  // namespace vmk
