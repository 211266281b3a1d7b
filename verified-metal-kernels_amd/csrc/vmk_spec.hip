// Speculative chain/tree verification on gfx950: split-K flash-decoding over the kd*G query rows of one GQA group.
//
// Replaces the reference's spec_verify_qperm / spec_verify_partial_mpp / spec_verify_combine Metal kernels
// (kernels/spec_opus55_v7.py:186-199, 228-342, 344-365) behind the kernel(q, k, v, bits) contract of
// ops/spec.py:1-3.  The draft mask is applied in registers from (B, kd, W) 32-bit words, so kd is not limited to 32.
#include "attn_core.h"
#include "vmk_internal.h"


namespace vmk {

struct SpecArgs {
  const f16* q;            // (B, kd, Hq, 128)
  const f16* k;            // (B, Hkv, L, 128)
  const f16* v;
  const uint32_t* bits;    // (B, kd, W), or null: every cache position visible to every query row (plain decode)
  const int* lens;         // (B,) cache positions in use per batch entry (clamped to [kd, L]), or null: all L
  void* part_o;            // [item][32*WR][128] normalised O of type part_t, item = (grp * nrb + rb) * nsplit + split
  float* part_ml;          // [item][32*WR][2]
  f16* out;                // (B, kd, Hq, 128)
  int B, kd, Hq, Hkv, G, L, W;
  int WR, WK, nrb, nsplit, chunk;
  float sl2;               // softmax scale * log2(e)
  // Paged decode: k, v are the page pools (num_pages pages of ps rows, HND or NHD), pages the (B, max_pages) table.
  const int* pages;
  int ps, max_pages, num_pages;
};

// Keys of one (batch, KV head) for one split: rows of k/v, and the draft mask of this lane's row on the last kd
// positions, preloaded as up to kMaskWords 32-bit words (kd <= 32 * kMaskWords).
constexpr int kMaskWords = 8;

typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

// The mask words are a vector value, not an array: an array member makes the compiler keep the whole struct in LDS
// and fetch the words one dependent round trip at a time before the first tile.
struct SpecSrc {
  const f16* kbase;
  const f16* vbase;
  u32x8 mw;          // the row's mask words; words at or past nw are not used
  int nw, kend, tail0;
  float scale;
  static constexpr bool kStrided = false;   // rows 256 bytes apart
  __device__ const f16* ktile(int key0) const { return kbase + (size_t)key0 * 128; }
  __device__ const f16* vtile(int key0) const { return vbase + (size_t)key0 * 128; }
  __device__ uint32_t bit(int j) const {          // bit j of the row's mask, 0 <= j < 32 * kMaskWords
    const int wi = j >> 5;
    uint32_t w = mw[0];
#pragma unroll
    for (int i = 1; i < kMaskWords; ++i) w = wi == i ? mw[i] : w;
    return wi < nw ? (w >> (j & 31)) & 1u : 0u;
  }
  // Loads the nw (1 .. kMaskWords) mask words at mrow; every address stays inside the row.  mrow == null: the whole
  // tail is visible.
  __device__ void load_mask(const uint32_t* mrow, int n) {
    if (!mrow) {
      nw = kMaskWords;
#pragma unroll
      for (int i = 0; i < kMaskWords; ++i) mw[i] = ~0u;
      return;
    }
    nw = n;
#pragma unroll
    for (int i = 0; i < kMaskWords; ++i) mw[i] = ldg4(mrow + min(i, n - 1));
  }
  __device__ void mask(floatx16& s, int key0, int g) const {
    if (key0 + kTile <= tail0 && key0 + kTile <= kend) return;   // whole tile visible (same for the whole wave)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key = key0 + 8 * blk + 4 * g + c;
        const uint32_t vis = (key < tail0) | bit(max(key - tail0, 0));
        const bool ok = (key < kend) & (vis != 0u);
        s[4 * blk + c] = ok ? s[4 * blk + c] : kNegInf;
      }
  }
};

// Cache positions of batch entry b: lens[b] clamped to [kd, L] (the query rows are the last kd of them), or L.
__device__ __forceinline__ int batch_len(const SpecArgs& a, int b) {
  return a.lens ? min(max(a.lens[b], a.kd), a.L) : a.L;
}

// One workgroup = WR x WK waves: WR row blocks of 32 rows, WK waves interleaving the key tiles of one split.
// V is the operand type: half8 (fp16 inputs) or bf16x8 (bf16 inputs).
template <class V>
__global__ __launch_bounds__(256) void spec_partial_kernel(SpecArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kAttnSmemBytes];
  const int item = blockIdx.x;
  const int split = item % a.nsplit;
  const int rb = (item / a.nsplit) % a.nrb;
  const int grp = item / (a.nsplit * a.nrb);
  const int b = grp / a.Hkv, h = grp % a.Hkv;
  const int R = a.kd * a.G;
  const int row0 = rb * a.WR * 32;                        // first query row (i*G + gg) of this workgroup
  const int lrow = row0 + (threadIdx.x & 31) + 32 * ((threadIdx.x >> 6) % a.WR);
  const int di = (lrow < R ? lrow : 0) / a.G;

  SpecSrc src;
  const size_t kvoff = (size_t)grp * a.L * 128;
  src.kbase = a.k + kvoff;
  src.vbase = a.v + kvoff;
  src.load_mask(a.bits ? a.bits + (size_t)(b * a.kd + di) * a.W : nullptr, a.W);
  const int Lb = batch_len(a, b);
  const int kbeg = split * a.chunk;
  src.kend = min(Lb, kbeg + a.chunk);
  src.tail0 = Lb - a.kd;
  src.scale = a.sl2;
  const int ntiles = max(0, (src.kend - kbeg + kTile - 1) / kTile);
  const size_t rows_wg = 32 * a.WR;
  auto qrow = [&](int r) {
    const int qr = row0 + r, i = qr / a.G, gg = qr % a.G;
    return a.q + ((size_t)(b * a.kd + i) * a.Hq + h * a.G + gg) * 128;
  };
  part_t<elem_t<V>>* po = reinterpret_cast<part_t<elem_t<V>>*>(a.part_o) + (size_t)item * rows_wg * 128;
  float* pml = a.part_ml + (size_t)item * rows_wg * 2;
  if (a.WK == 4)
    attend_wg<1, 4, 2, V>(smem, src, qrow, R - row0, kbeg, ntiles, po, pml);
  else
    attend_wg<2, 2, 2, V>(smem, src, qrow, R - row0, kbeg, ntiles, po, pml);
}

// Paged single-token decode: the key-split kernel with request b's keys [0, lens[b]) read through its page table
// (paged_src; a split holds at most 2048 keys, the decode split size up to 16 query heads per KV head).  Absent
// pages are left out of the softmax.  With every page present the partials are those of spec_partial_kernel on the
// gathered cache, so the output is bit-equal to vmk_decode's.
template <bool kNHD, class V>
__global__ __launch_bounds__(256) void decode_paged_kernel(SpecArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kAttnSmemBytes];
  const int item = blockIdx.x;
  const int split = item % a.nsplit;
  const int grp = item / a.nsplit;                         // one row block: G <= 16 rows
  const int b = grp / a.Hkv, h = grp % a.Hkv;
  const int Lb = batch_len(a, b);
  const int kbeg = split * a.chunk;
  const int kend = min(Lb, kbeg + a.chunk);
  const int ntiles = max(0, (kend - kbeg + kTile - 1) / kTile);
  const PagedSrc<kNHD> src = paged_src<kNHD>(a.k, a.v, a.ps, a.Hkv, a.num_pages, a.sl2,
                                             a.pages + (size_t)b * a.max_pages, a.max_pages, h, kbeg, kend);
  auto qrow = [&](int r) { return a.q + ((size_t)b * a.Hq + h * a.G + r) * 128; };
  part_t<elem_t<V>>* po = reinterpret_cast<part_t<elem_t<V>>*>(a.part_o) + (size_t)item * 32 * 128;
  float* pml = a.part_ml + (size_t)item * 32 * 2;
  attend_wg<1, 4, 2, V>(smem, src, qrow, a.G, kbeg, ntiles, po, pml);
}

// Row-split variant for kd*G > 64 rows: NW waves own 32 rows each and share one LDS ring, so every K/V tile of the
// split is streamed from HBM once per workgroup of 32*NW rows.
template <int NW, class V>
__global__ __launch_bounds__(64 * NW) void spec_partial_rows_kernel(SpecArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kRowsSmemBytes];
  const int item = blockIdx.x;
  const int split = item % a.nsplit;
  const int rb = (item / a.nsplit) % a.nrb;
  const int grp = item / (a.nsplit * a.nrb);
  const int b = grp / a.Hkv, h = grp % a.Hkv;
  const int R = a.kd * a.G;
  const int row0 = rb * NW * 32;
  const int lrow = row0 + (threadIdx.x & 31) + 32 * (threadIdx.x >> 6);
  const int di = (lrow < R ? lrow : 0) / a.G;
  SpecSrc src;
  const size_t kvoff = (size_t)grp * a.L * 128;
  src.kbase = a.k + kvoff;
  src.vbase = a.v + kvoff;
  src.load_mask(a.bits ? a.bits + (size_t)(b * a.kd + di) * a.W : nullptr, a.W);
  const int Lb = batch_len(a, b);
  const int kbeg = split * a.chunk;
  src.kend = min(Lb, kbeg + a.chunk);
  src.tail0 = Lb - a.kd;
  src.scale = a.sl2;
  const int ntiles = max(0, (src.kend - kbeg + kTile - 1) / kTile);
  const size_t rows_wg = 32 * NW;
  attend_wg_rows<NW, V>(smem, src,
                     [&](int r) {
                       const int qr = row0 + r, i = qr / a.G, gg = qr % a.G;
                       return a.q + ((size_t)(b * a.kd + i) * a.Hq + h * a.G + gg) * 128;
                     },
                     R - row0, kbeg, ntiles,
                     reinterpret_cast<part_t<elem_t<V>>*>(a.part_o) + (size_t)item * rows_wg * 128,
                     a.part_ml + (size_t)item * rows_wg * 2);
}

// LSE merge of the nsplit partials of every query row; one workgroup (128 threads = head-dims) per row.  E is the
// output element type.
template <class E>
__global__ __launch_bounds__(128) void spec_combine_kernel(SpecArgs a) {
  const int R = a.kd * a.G;
  const int rowg = blockIdx.x;                 // grp * R + row
  const int grp = rowg / R, row = rowg % R;
  const int rb = row / (32 * a.WR), rl = row % (32 * a.WR);
  const size_t rows_wg = 32 * a.WR;
  const size_t item0 = (size_t)(grp * a.nrb + rb) * a.nsplit;
  const int b = grp / a.Hkv, h = grp % a.Hkv;
  const int i = row / a.G, gg = row % a.G;
  typedef part_t<E> PT;
  combine_row<128, 1, PT>(a.nsplit,
                          [&](int s, const float*& ml, const PT*& o) {
                            const size_t base = (item0 + s) * rows_wg + rl;
                            ml = a.part_ml + base * 2;
                            o = reinterpret_cast<const PT*>(a.part_o) + base * 128;
                          },
                          reinterpret_cast<E*>(a.out) + ((size_t)(b * a.kd + i) * a.Hq + h * a.G + gg) * 128);
}

// The same merge for many rows (at least kCombineVecRows): one wave per 4 rows, 16 lanes per row, each lane 8
// head-dims loaded 16 bytes at a time, so the partials stream with a quarter of the load instructions per byte.  Few
// rows take spec_combine_kernel: there the merge is latency-bound, and one thread per head-dim keeps each thread's
// chain of products short.  Both give the same bits.
constexpr int kCombineVecRows = 1024;
template <class E>
__global__ __launch_bounds__(64) void spec_combine_vec_kernel(SpecArgs a) {
  const int R = a.kd * a.G;
  const int lane = threadIdx.x, c = lane & 15;
  const int rowg = blockIdx.x * 4 + (lane >> 4);                    // grp * R + row
  if (rowg >= a.B * a.Hkv * R) return;                              // a whole row group of lanes
  const int grp = rowg / R, row = rowg % R;
  const int rb = row / (32 * a.WR), rl = row % (32 * a.WR);
  const size_t rows_wg = 32 * a.WR;
  const size_t item0 = (size_t)(grp * a.nrb + rb) * a.nsplit;
  const int b = grp / a.Hkv, h = grp % a.Hkv;
  const int i = row / a.G, gg = row % a.G;
  typedef part_t<E> PT;
  combine_vec<PT>(a.nsplit,
                  [&](int s, const float*& ml, const PT*& o) {
                    const size_t base = (item0 + s) * rows_wg + rl;
                    ml = a.part_ml + base * 2;
                    o = reinterpret_cast<const PT*>(a.part_o) + base * 128 + 8 * c;
                  },
                  reinterpret_cast<E*>(a.out) + ((size_t)(b * a.kd + i) * a.Hq + h * a.G + gg) * 128 + 8 * c);
}

// The combine launch for `rows` output rows.
template <class E>
static void launch_spec_combine(const SpecArgs& a, int64_t rows, hipStream_t s) {
  if (rows >= kCombineVecRows)
    hipLaunchKernelGGL(spec_combine_vec_kernel<E>, dim3((unsigned)((rows + 3) / 4)), dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL(spec_combine_kernel<E>, dim3((unsigned)rows), dim3(128), 0, s, a);
}

struct SpecPlan {
  bool rows_mode;
  int WR, WK, nrb, nsplit, chunk;
  size_t po_floats, pml_floats;
};

static SpecPlan spec_plan(int64_t B, int64_t kd, int64_t Hq, int64_t Hkv, int64_t L) {
  SpecPlan p;
  const int64_t G = Hq / Hkv, R = kd * G;
  p.rows_mode = R > 64;
  if (p.rows_mode) { p.WR = R <= 128 ? 4 : 8; p.WK = 1; }   // row-split: WR = waves sharing one ring
  else if (R <= 32) { p.WR = 1; p.WK = 4; }
  else { p.WR = 2; p.WK = 2; }
  const int64_t rows_wg = 32 * p.WR;
  p.nrb = (int)((R + rows_wg - 1) / rows_wg);
  const int64_t base = B * Hkv * p.nrb;
  // The split size depends on the rows of one group (kd * G) only, never on B: a batch entry goes through the same
  // key splits, tile order and merge as the same entry alone, so its rows are bit-equal (batch invariance).  Key
  // split: 2048 keys up to 16 rows (decode: 256 workgroups once B * Hkv * L reaches 2^19), then 128 keys per row
  // (C3: 4096), which keeps the fp32 partials at 1/64 of the K/V bytes.  Row split: 4096 keys, 16 per row beyond.
  const int64_t chunk = p.rows_mode ? std::max<int64_t>(4096, 16 * R)
                                    : std::min<int64_t>(8192, std::max<int64_t>(2048, 128 * R));
  p.chunk = (int)chunk;
  p.nsplit = (int)((L + chunk - 1) / chunk);
  const size_t items = (size_t)base * p.nsplit;
  p.po_floats = items * rows_wg * 128;
  p.pml_floats = items * rows_wg * 2;
  return p;
}

}  // namespace vmk

using namespace vmk;

extern "C" size_t vmk_spec_workspace_size(int64_t B, int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L) {
  if (B <= 0 || kd <= 0 || Hkv <= 0 || Hq % Hkv || D != 128 || L < kd) return 0;
  SpecPlan p = spec_plan(B, kd, Hq, Hkv, L);
  return kWsHead + (p.po_floats + p.pml_floats) * sizeof(float) + 512;   // fits either partial type
}

// Partial launch (key split or row split by the plan) and LSE-combine launch of one spec/decode call; V is the
// operand type of the inputs (half8: fp16, bf16x8: bf16).  `partials` is the 256-byte aligned region of
// spec_partials_bytes<V>(p) bytes that receives the partials: every partial the combine reads is written first, so
// the region needs no initialisation.  Layout: the normalised O rows in the partial type of V's inputs, then the
// (m, l) pairs from the next 256-byte boundary.
template <class V>
static size_t spec_ml_offset(const SpecPlan& p) {
  return (p.po_floats * sizeof(part_t<elem_t<V>>) + 255) / 256 * 256;
}
template <class V>
static size_t spec_partials_bytes(const SpecPlan& p) { return spec_ml_offset<V>(p) + p.pml_floats * sizeof(float); }

template <class V>
static int spec_launch(SpecArgs& a, const SpecPlan& p, void* partials, hipStream_t s) {
  a.part_o = partials;
  a.part_ml = reinterpret_cast<float*>((char*)partials + spec_ml_offset<V>(p));
  a.WR = p.WR; a.WK = p.WK; a.nrb = p.nrb; a.nsplit = p.nsplit; a.chunk = p.chunk;
  a.sl2 = (float)(1.0 / sqrt(128.0)) * kLog2e;
  const unsigned items = (unsigned)(a.B * a.Hkv * p.nrb * p.nsplit);
  prof_before(kKSpecPartial, s);
  if (!p.rows_mode)
    hipLaunchKernelGGL(spec_partial_kernel<V>, dim3(items), dim3(256), 0, s, a);
  else if (p.WR == 4)
    hipLaunchKernelGGL((spec_partial_rows_kernel<4, V>), dim3(items), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((spec_partial_rows_kernel<8, V>), dim3(items), dim3(512), 0, s, a);
  prof_after(kKSpecPartial, s);
  VMK_CHECK_HIP(hipGetLastError());
  prof_before(kKSpecCombine, s);
  launch_spec_combine<elem_t<V>>(a, (int64_t)a.B * a.Hkv * a.kd * a.G, s);
  prof_after(kKSpecCombine, s);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

// Host-side argument checks shared by vmk_spec_verify and vmk_spec_verify_noalloc (no HIP call).
static int spec_check_args(const void* q, const void* k, const void* v, const void* mask_words, void* out,
                           int64_t B, int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W) {
  VMK_CHECK(q && k && v && mask_words && out, "null pointer argument");
  VMK_CHECK(B > 0 && kd > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "bad head/batch sizes");
  VMK_CHECK(D == 128, "only head_dim 128 is supported");
  VMK_CHECK(L >= kd, "L must count the kd drafts (L >= kd)");
  VMK_CHECK(W == (kd + 31) / 32, "mask must hold ceil(kd/32) 32-bit words per draft");
  VMK_CHECK(kd <= 32 * kMaskWords, "at most 256 drafts");
  VMK_CHECK((Hq / Hkv) * kd <= 1 << 20 && B * Hkv * L <= (int64_t)1 << 40, "sizes out of range");
  VMK_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), "tensors must be 16-byte aligned");
  return 0;
}

template <class V>
static int spec_verify(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                       int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W, void* workspace,
                       size_t ws_bytes, void* stream) {
  if (int rc = spec_check_args(q, k, v, mask_words, out, B, kd, Hq, Hkv, D, L, W)) return rc;
  const size_t need = vmk_spec_workspace_size(B, kd, Hq, Hkv, D, L);
  VMK_CHECK(workspace && ws_bytes >= need, "workspace too small (query vmk_spec_workspace_size)");
  SpecPlan p = spec_plan(B, kd, Hq, Hkv, L);
  SpecArgs a;
  a.q = (const f16*)q; a.k = (const f16*)k; a.v = (const f16*)v; a.bits = (const uint32_t*)mask_words;
  a.lens = nullptr;
  a.out = (f16*)out;
  a.B = (int)B; a.kd = (int)kd; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv); a.L = (int)L; a.W = (int)W;
  return spec_launch<V>(a, p, align_up((char*)workspace + kWsHead, 256), (hipStream_t)stream);
}

// Plain single-token decode: the verify path with one query row per request and no mask (the row's own position is
// the last of the cache, visible like every other).
extern "C" size_t vmk_decode_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t L) {
  return vmk_spec_workspace_size(B, 1, Hq, Hkv, D, L);
}

template <class V>
static int decode(const void* q, const void* k, const void* v, const void* lens, void* out, int64_t B, int64_t Hq,
                  int64_t Hkv, int64_t D, int64_t L, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(q && k && v && out, "null pointer argument");
  VMK_CHECK(B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "bad head/batch sizes");
  VMK_CHECK(D == 128, "only head_dim 128 is supported");
  VMK_CHECK(L >= 1, "L must be at least 1");
  VMK_CHECK(Hq / Hkv <= 1 << 20 && B * Hkv * L <= (int64_t)1 << 40, "sizes out of range");
  VMK_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), "tensors must be 16-byte aligned");
  const size_t need = vmk_decode_workspace_size(B, Hq, Hkv, D, L);
  VMK_CHECK(workspace && ws_bytes >= need, "workspace too small (query vmk_decode_workspace_size)");
  SpecPlan p = spec_plan(B, 1, Hq, Hkv, L);
  SpecArgs a;
  a.q = (const f16*)q; a.k = (const f16*)k; a.v = (const f16*)v; a.bits = nullptr;
  a.lens = (const int*)lens;
  a.out = (f16*)out;
  a.B = (int)B; a.kd = 1; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv); a.L = (int)L; a.W = 1;
  return spec_launch<V>(a, p, align_up((char*)workspace + kWsHead, 256), (hipStream_t)stream);
}

extern "C" int vmk_spec_verify(const void* q, const void* k, const void* v, const void* mask_words, void* out,
                               int64_t B, int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W,
                               void* workspace, size_t ws_bytes, void* stream) {
  return spec_verify<half8>(q, k, v, mask_words, out, B, kd, Hq, Hkv, D, L, W, workspace, ws_bytes, stream);
}

extern "C" int vmk_spec_verify_bf16(const void* q, const void* k, const void* v, const void* mask_words, void* out,
                                    int64_t B, int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W,
                                    void* workspace, size_t ws_bytes, void* stream) {
  return spec_verify<bf16x8>(q, k, v, mask_words, out, B, kd, Hq, Hkv, D, L, W, workspace, ws_bytes, stream);
}

extern "C" int vmk_decode(const void* q, const void* k, const void* v, const void* lens, void* out, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t D, int64_t L, void* workspace, size_t ws_bytes,
                          void* stream) {
  return decode<half8>(q, k, v, lens, out, B, Hq, Hkv, D, L, workspace, ws_bytes, stream);
}

extern "C" int vmk_decode_bf16(const void* q, const void* k, const void* v, const void* lens, void* out, int64_t B,
                               int64_t Hq, int64_t Hkv, int64_t D, int64_t L, void* workspace, size_t ws_bytes,
                               void* stream) {
  return decode<bf16x8>(q, k, v, lens, out, B, Hq, Hkv, D, L, workspace, ws_bytes, stream);
}

// Paged single-token decode (HND or NHD page pools).
extern "C" size_t vmk_decode_paged_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                                                  int64_t max_pages) {
  if (page_size < 32 || page_size % 32 || page_size > (1 << 20) || max_pages < 1 || max_pages > (1 << 20)) return 0;
  return vmk_decode_workspace_size(B, Hq, Hkv, D, page_size * max_pages);
}

template <bool kNHD, class V>
static int decode_paged(const void* q, const void* k_pages, const void* v_pages, const void* page_table,
                        const void* lens, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t num_pages,
                        int64_t page_size, int64_t max_pages, void* workspace, size_t ws_bytes, void* stream) {
  VMK_CHECK(q && k_pages && v_pages && page_table && out, "null pointer argument");
  VMK_CHECK(B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "bad head/batch sizes");
  VMK_CHECK(D == 128, "only head_dim 128 is supported");
  VMK_CHECK(Hq / Hkv <= 16, "at most 16 query heads per KV head");
  VMK_CHECK(!kNHD || Hkv <= 4096, "NHD pages: at most 4096 KV heads");
  VMK_CHECK(page_size >= 32 && page_size % 32 == 0 && page_size <= (1 << 20), "page_size must be a multiple of 32");
  VMK_CHECK(max_pages >= 1 && page_size * max_pages < (1 << 30) && B * max_pages < ((int64_t)1 << 31),
            "max_pages out of range");
  VMK_CHECK(num_pages > 0 && num_pages < (1 << 30) && num_pages * Hkv * page_size <= ((int64_t)1 << 34),
            "num_pages out of range");
  VMK_CHECK(B * Hkv * page_size * max_pages <= (int64_t)1 << 40, "sizes out of range");
  VMK_CHECK(aligned16(q) && aligned16(k_pages) && aligned16(v_pages) && aligned16(out),
            "tensors must be 16-byte aligned");
  const int64_t L = page_size * max_pages;
  const size_t need = vmk_decode_paged_workspace_size(B, Hq, Hkv, D, page_size, max_pages);
  VMK_CHECK(workspace && ws_bytes >= need, "workspace too small (query vmk_decode_paged_workspace_size)");
  SpecPlan p = spec_plan(B, 1, Hq, Hkv, L);
  VMK_CHECK(!p.rows_mode && p.WR == 1 && p.WK == 4 && p.nrb == 1 && p.chunk <= 2048, "unsupported decode plan");
  SpecArgs a;
  a.q = (const f16*)q; a.k = (const f16*)k_pages; a.v = (const f16*)v_pages; a.bits = nullptr;
  a.lens = (const int*)lens;
  a.out = (f16*)out;
  a.B = (int)B; a.kd = 1; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv); a.L = (int)L; a.W = 1;
  a.pages = (const int*)page_table;
  a.ps = (int)page_size; a.max_pages = (int)max_pages; a.num_pages = (int)num_pages;
  a.part_o = align_up((char*)workspace + kWsHead, 256);
  a.part_ml = reinterpret_cast<float*>((char*)a.part_o + spec_ml_offset<V>(p));
  a.WR = p.WR; a.WK = p.WK; a.nrb = p.nrb; a.nsplit = p.nsplit; a.chunk = p.chunk;
  a.sl2 = (float)(1.0 / sqrt(128.0)) * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  prof_before(kKSpecPartial, s);
  hipLaunchKernelGGL((decode_paged_kernel<kNHD, V>), dim3((unsigned)(B * Hkv * p.nsplit)), dim3(256), 0, s, a);
  prof_after(kKSpecPartial, s);
  VMK_CHECK_HIP(hipGetLastError());
  prof_before(kKSpecCombine, s);
  launch_spec_combine<elem_t<V>>(a, B * Hq, s);
  prof_after(kKSpecCombine, s);
  VMK_CHECK_HIP(hipGetLastError());
  return 0;
}

#define VMK_DECODE_PAGED_ENTRY(name, nhd, V)                                                                      \
  extern "C" int name(const void* q, const void* k_pages, const void* v_pages, const void* page_table,           \
                      const void* lens, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,               \
                      int64_t num_pages, int64_t page_size, int64_t max_pages, void* workspace, size_t ws_bytes,  \
                      void* stream) {                                                                            \
    return decode_paged<nhd, V>(q, k_pages, v_pages, page_table, lens, out, B, Hq, Hkv, D, num_pages, page_size, \
                                max_pages, workspace, ws_bytes, stream);                                          \
  }
VMK_DECODE_PAGED_ENTRY(vmk_decode_paged, false, half8)
VMK_DECODE_PAGED_ENTRY(vmk_decode_paged_bf16, false, bf16x8)
VMK_DECODE_PAGED_ENTRY(vmk_decode_paged_nhd, true, half8)
VMK_DECODE_PAGED_ENTRY(vmk_decode_paged_nhd_bf16, true, bf16x8)
#undef VMK_DECODE_PAGED_ENTRY

// ---------------------------------------------------------------------------------------------- allocation-free
// The spec half of vmk_spec_verify_noalloc.  The entry point and its static scratch live in vmk_noalloc.hip, a code
// object of their own, which the HIP runtime loads onto a device (and so allocates the scratch on) only when the
// scratch is first looked up there.
namespace vmk {
int spec_noalloc_need(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                      int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W, size_t* need) {
  if (int rc = spec_check_args(q, k, v, mask_words, out, B, kd, Hq, Hkv, D, L, W)) return rc;
  *need = spec_partials_bytes<half8>(spec_plan(B, kd, Hq, Hkv, L));
  return 0;
}

int spec_noalloc_launch(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                        int64_t kd, int64_t Hq, int64_t Hkv, int64_t L, int64_t W, void* partials, hipStream_t s) {
  const SpecPlan p = spec_plan(B, kd, Hq, Hkv, L);
  SpecArgs a;
  a.q = (const f16*)q; a.k = (const f16*)k; a.v = (const f16*)v; a.bits = (const uint32_t*)mask_words;
  a.lens = nullptr;
  a.out = (f16*)out;
  a.B = (int)B; a.kd = (int)kd; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv); a.L = (int)L; a.W = (int)W;
  return spec_launch<half8>(a, p, partials, s);
}
}  // namespace vmk
