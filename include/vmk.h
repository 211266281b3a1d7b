/* libvmk: MI355X (gfx950) kernels for shared-prefix decode, speculative chain/tree verification and DeepSeek Sparse
 * Attention decode, behind a plain C ABI (raw device pointers, sizes, a caller-provided workspace and a HIP stream).
 *
 * Conventions shared by every entry point:
 *   - tensors are dense row-major device buffers, 16-byte aligned; fp16 unless stated otherwise;
 *   - inputs are never written; outputs are fully overwritten;
 *   - `stream` is a hipStream_t (NULL = default stream); the call only enqueues work and returns;
 *   - `workspace` is device memory of at least the size returned by the matching *_workspace_size query.  Its first
 *     VMK_WORKSPACE_HEAD bytes (the head) must be zero before the first call that uses it, and every call leaves the
 *     head zero again (kernels accumulate histograms and counters into it), so zero it once at allocation; the rest
 *     needs no initialisation.  Calls sharing one workspace must be ordered (one stream, or synchronised);
 *   - return 0 on success; 1 = rejected arguments (nothing launched), 2 = HIP launch/runtime error; the message of
 *     the last failure on this host thread is returned by vmk_last_error().
 *
 * Each entry point replaces the `kernel(**inputs)` function of one of the reference's kernel modules, called with
 * the keyword inputs listed in verify.py:35-37; the Python modules verified-metal-kernels_amd/kernels/<op>_mi355x.py
 * keep that signature and call into this ABI.
 */
#ifndef VMK_H
#define VMK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes at the start of every workspace that must be zero before first use (see above). */
#define VMK_WORKSPACE_HEAD ((size_t)4 << 20)

/* Library version (1). */
int vmk_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* vmk_last_error(void);

/* 0 when the current HIP device is a gfx950 (the only architecture this library is built for), else 1. */
int vmk_check_device(void);

/* ---------------------------------------------------------------------------------------------- speculative verify
 * Replaces kernel(q, k, v, bits) of kernels/spec_opus55_v7.py:467-521 (op contract ops/spec.py:1-3, 59-82).
 *   q          (B, kd, Hq, D)        fp16    draft queries
 *   k, v       (B, Hkv, L, D)        fp16    cache; the last kd positions are the drafts themselves
 *   mask_words (B, kd, W)            uint32  W = ceil(kd/32); bit j%32 of word j/32 of draft i: i may attend draft j
 *                                            (the reference's (B, kd) int32 `bits` is the W = 1 case)
 *   out        (B, kd, Hq, D)        fp16
 * D must be 128, Hq a multiple of Hkv, L >= kd.  Context positions (< L-kd) are visible to every draft. */
size_t vmk_spec_workspace_size(int64_t B, int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L);
int vmk_spec_verify(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                    int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W, void* workspace,
                    size_t ws_bytes, void* stream);

/* Allocation-free form of vmk_spec_verify.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same inputs,
 * output and result as vmk_spec_verify (same kernels and plan, so the same bits); the partials go to a static
 * device array of vmk_spec_noalloc_max_bytes() bytes (32 MiB) that each GPU holds from this entry point's first
 * call on it until the process ends (the array has a code object of its own, loaded on that first call), so it
 * calls no hipMalloc/hipFree.  Shapes whose partials exceed it are rejected (return 1, nothing launched).  All calls
 * on one GPU share that GPU's array: calls that overlap on one GPU (two streams or threads) race. */
size_t vmk_spec_noalloc_max_bytes(void);
int vmk_spec_verify_noalloc(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                            int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W, void* stream);

/* ---------------------------------------------------------------------------------------------- single-token decode
 * No kernel module of the reference ships this op: it is the plain decode that the reference benchmarks against
 * llama.cpp (llama_cpp/test-backend-ops.patch:79-83: 32 q / 8 kv heads, D = 128) and reports at parity
 * (POST.md:42-46).  It is the verify path with one query row per request and no mask.
 *   q     (B, Hq, D)       fp16   one token per request
 *   k, v  (B, Hkv, L, D)   fp16   cache; the token's own key/value is its last position in use
 *   lens  (B,)             int32  positions in use per request (clamped to [1, L]), or NULL: all L
 *   out   (B, Hq, D)       fp16
 * D must be 128, Hq a multiple of Hkv, L >= 1. */
size_t vmk_decode_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t L);
int vmk_decode(const void* q, const void* k, const void* v, const void* lens, void* out, int64_t B, int64_t Hq,
               int64_t Hkv, int64_t D, int64_t L, void* workspace, size_t ws_bytes, void* stream);

/* Paged single-token decode: vmk_decode over a page pool, as serving engines keep their caches.  No reference kernel
 * covers it (the reference's paged variant is the shared-prefix one it leaves out, README.md:141-142); it joins this
 * decode op with the page pools of vmk_prefix_decode_paged.
 *   k_pages, v_pages  (num_pages, Hkv, page_size, D)  (HND; _nhd: (num_pages, page_size, Hkv, D))  page pool
 *   page_table        (B, max_pages)  int32   each request's pages, in order; ids outside [0, num_pages) are absent
 *                                             pages, left out of the softmax (no memory is read for them)
 *   lens              (B,)            int32   positions in use (clamped to [1, page_size * max_pages]), or NULL
 * page_size a multiple of 32, Hq / Hkv <= 16.  With every page of the rows in use present, the output is bit-equal to
 * vmk_decode on the gathered cache (L = page_size * max_pages).  _bf16: bf16 q, pages and output. */
size_t vmk_decode_paged_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                                       int64_t max_pages);
int vmk_decode_paged(const void* q, const void* k_pages, const void* v_pages, const void* page_table,
                     const void* lens, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t num_pages,
                     int64_t page_size, int64_t max_pages, void* workspace, size_t ws_bytes, void* stream);
int vmk_decode_paged_bf16(const void* q, const void* k_pages, const void* v_pages, const void* page_table,
                          const void* lens, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                          int64_t num_pages, int64_t page_size, int64_t max_pages, void* workspace, size_t ws_bytes,
                          void* stream);
int vmk_decode_paged_nhd(const void* q, const void* k_pages, const void* v_pages, const void* page_table,
                         const void* lens, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                         int64_t num_pages, int64_t page_size, int64_t max_pages, void* workspace, size_t ws_bytes,
                         void* stream);
int vmk_decode_paged_nhd_bf16(const void* q, const void* k_pages, const void* v_pages, const void* page_table,
                              const void* lens, void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                              int64_t num_pages, int64_t page_size, int64_t max_pages, void* workspace,
                              size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------- shared-prefix decode
 * Replaces kernel(q, kp, vp, ks, vs) of kernels/prefix_opus55_v8.py:282-355 (op contract ops/prefix.py:1-4, 57-70).
 *   q       (N, Hq, D)        fp16   one decode token per request
 *   kp, vp  (Hkv, P, D)       fp16   shared prefix (may be NULL when P == 0)
 *   ks, vs  (N, Hkv, S, D)    fp16   per-request suffixes, padded to S rows (may be NULL when S == 0)
 *   slens   (N,)              int32  rows of each suffix in use when ragged != 0 (clamped to [0, S]); else unused
 *   out     (N, Hq, D)        fp16
 * D must be 128, Hq a multiple of Hkv with at most 32 query heads per KV head. */
size_t vmk_prefix_workspace_size(int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t P, int64_t S,
                                 int64_t ragged);
int vmk_prefix_decode(const void* q, const void* kp, const void* vp, const void* ks, const void* vs,
                      const void* slens, void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t P,
                      int64_t S, int64_t ragged, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------- paged shared prefix
 * No kernel of the reference covers it: README.md:141-142 leaves the paged-cache variant of the shared-prefix kernel
 * out of the package.  Same op as vmk_prefix_decode with the keys and values in a page pool (the layout FlashInfer
 * calls HND):
 *   k_pages, v_pages  (num_pages, Hkv, page_size, D)  fp16   page pool; page_size a multiple of 32
 *   prefix_pages      (P / page_size,)                int32  the shared prefix's pages (P a whole number of pages)
 *   suffix_pages      (N, max_suffix_pages)           int32  each request's suffix pages
 *   slens             (N,)                            int32  suffix rows in use (clamped to [0, max_suffix_pages *
 *                                                            page_size]), or NULL: every suffix is full
 * A page id outside [0, num_pages) is an absent page: its rows are left out of the softmax (no memory is read for
 * it).  With every page present the output is bit-equal to vmk_prefix_decode on the gathered cache with
 * S = max_suffix_pages * page_size. */
size_t vmk_prefix_paged_workspace_size(int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t P, int64_t page_size,
                                       int64_t max_suffix_pages);
int vmk_prefix_decode_paged(const void* q, const void* k_pages, const void* v_pages, const void* prefix_pages,
                            const void* suffix_pages, const void* slens, void* out, int64_t N, int64_t Hq,
                            int64_t Hkv, int64_t D, int64_t num_pages, int64_t page_size, int64_t P,
                            int64_t max_suffix_pages, void* workspace, size_t ws_bytes, void* stream);
/* The same op over a page pool in the layout FlashInfer calls NHD: k_pages, v_pages (num_pages, page_size, Hkv, D),
 * a page's rows of one head Hkv * D elements apart.  Same arguments, limits (also Hkv <= 4096), workspace size and
 * plans as vmk_prefix_decode_paged; the output is bit-equal to it on the same logical cache. */
int vmk_prefix_decode_paged_nhd(const void* q, const void* k_pages, const void* v_pages, const void* prefix_pages,
                                const void* suffix_pages, const void* slens, void* out, int64_t N, int64_t Hq,
                                int64_t Hkv, int64_t D, int64_t num_pages, int64_t page_size, int64_t P,
                                int64_t max_suffix_pages, void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------- bf16 inputs
 * The reference kernels read fp16 only (README.md:140: on bf16 inputs they produce invalid values).  These entry points
 * take bf16 q, keys and values (and write a bf16 output) with the same arguments, workspace sizes, plans and
 * semantics as their fp16 counterparts above: the MFMAs run in bf16 with fp32 accumulation, and P is rounded to bf16
 * before the P.V product.  DSA takes bf16 q, kv, iq and ik (w stays fp32; its scores are fp32 either way). */
int vmk_spec_verify_bf16(const void* q, const void* k, const void* v, const void* mask_words, void* out, int64_t B,
                         int64_t kd, int64_t Hq, int64_t Hkv, int64_t D, int64_t L, int64_t W, void* workspace,
                         size_t ws_bytes, void* stream);
int vmk_decode_bf16(const void* q, const void* k, const void* v, const void* lens, void* out, int64_t B, int64_t Hq,
                    int64_t Hkv, int64_t D, int64_t L, void* workspace, size_t ws_bytes, void* stream);
int vmk_prefix_decode_bf16(const void* q, const void* kp, const void* vp, const void* ks, const void* vs,
                           const void* slens, void* out, int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t P,
                           int64_t S, int64_t ragged, void* workspace, size_t ws_bytes, void* stream);
int vmk_prefix_decode_paged_bf16(const void* q, const void* k_pages, const void* v_pages, const void* prefix_pages,
                                 const void* suffix_pages, const void* slens, void* out, int64_t N, int64_t Hq,
                                 int64_t Hkv, int64_t D, int64_t num_pages, int64_t page_size, int64_t P,
                                 int64_t max_suffix_pages, void* workspace, size_t ws_bytes, void* stream);
int vmk_prefix_decode_paged_nhd_bf16(const void* q, const void* k_pages, const void* v_pages,
                                     const void* prefix_pages, const void* suffix_pages, const void* slens, void* out,
                                     int64_t N, int64_t Hq, int64_t Hkv, int64_t D, int64_t num_pages,
                                     int64_t page_size, int64_t P, int64_t max_suffix_pages, void* workspace,
                                     size_t ws_bytes, void* stream);
int vmk_dsa_indexer_select_bf16(const void* iq, const void* ik, const void* w, const void* lens, void* idx, void* cnt,
                                int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream);
int vmk_dsa_indexer_bf16(const void* iq, const void* ik, const void* w, const void* lens, void* scores, int64_t B,
                         int64_t L, void* workspace, size_t ws_bytes, void* stream);
int vmk_dsa_sparse_mla_bf16(const void* q, const void* kv, const void* idx, const void* cnt, void* out, int64_t B,
                            int64_t L, void* workspace, size_t ws_bytes, void* stream);
int vmk_dsa_decode_bf16(const void* q, const void* kv, const void* iq, const void* ik, const void* w, const void* lens,
                        void* out, void* idx, void* cnt, int64_t B, int64_t L, void* workspace, size_t ws_bytes,
                        void* stream);

/* ---------------------------------------------------------------------------------------------- DSA decode
 * Replaces kernel(q, kv, iq, ik, w, lens) of kernels/dsa_opus55_v7.py:946-977 (op contract ops/dsa.py:1-9, 53-83).
 *   q     (B, 128, 576)  fp16    absorbed queries (512 latent + 64 rope)
 *   kv    (B, L, 576)    fp16    latent cache; the value is the first 512 dims of the same row
 *   iq    (B, 64, 128)   fp16    indexer queries
 *   ik    (B, L, 128)    fp16    indexer keys
 *   w     (B, 64)        fp32    indexer head weights
 *   lens  (B,)           int32   valid positions per request, or NULL for all L
 *   idx   (B, 2048)      int32   selected positions; entries [0, cnt[b]) are valid (out for the select entries,
 *                                in for vmk_dsa_sparse_mla).  Order: positions above the threshold bucket in increasing
 *                                order, then the bucket's picks in increasing order; ties at the threshold are taken in
 *                                increasing position order.  With n <= 2048 valid positions, idx = 0..n-1.
 *   cnt   (B,)           int32   min(n, 2048)
 *   out   (B, 128, 512)  fp16
 * score[l] = sum_h w[h] * max(iq[h] . ik[l], 0) in fp32; attention scale 1/sqrt(192).
 * Limits: L <= 4194304 (indexer/select); the attention entries also need L * 1152 bytes < 2 GiB per request
 * (L <= 1864134), since the row gather addresses a request's cache by 32-bit offsets. */
size_t vmk_dsa_workspace_size(int64_t B, int64_t L);
/* Indexer + exact top-2048 only (the reference's indexer_mpp/indexer_float + select, dsa_opus55_v7.py:963-973). */
int vmk_dsa_indexer_select(const void* iq, const void* ik, const void* w, const void* lens, void* idx, void* cnt,
                           int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream);
/* The two stages of the select on their own, as llama.cpp decomposes DSA decode (LIGHTNING_INDEXER and TOP_K,
 * llama_cpp/test-backend-ops.patch:96-97; the reference's separate dsa_indexer and dsa_select kernels,
 * dsa_opus55_v7.py:27-98, 100-307).  vmk_dsa_indexer writes scores (B, L) fp32, row stride L; positions at or past
 * lens[b] are not written.  vmk_dsa_topk takes such scores and writes idx/cnt exactly as vmk_dsa_indexer_select does
 * (the same picks in the same order for the same scores).  The mask of llama.cpp's TOP_K_MASK step has no
 * counterpart: vmk_dsa_sparse_mla reads the indices directly. */
int vmk_dsa_indexer(const void* iq, const void* ik, const void* w, const void* lens, void* scores, int64_t B, int64_t L,
                    void* workspace, size_t ws_bytes, void* stream);
int vmk_dsa_topk(const void* scores, const void* lens, void* idx, void* cnt, int64_t B, int64_t L, void* workspace,
                 size_t ws_bytes, void* stream);
/* Sparse absorbed-MLA attention over given indices (the reference's attn_mpp/attn_float, dsa_opus55_v7.py:975). */
int vmk_dsa_sparse_mla(const void* q, const void* kv, const void* idx, const void* cnt, void* out, int64_t B,
                       int64_t L, void* workspace, size_t ws_bytes, void* stream);
/* ------------------------------------------------------------------------------------------------ DSA projections
 * The per-token projections that produce the DSA op's inputs from a hidden state.  The reference leaves them outside
 * its op (ops/dsa.py:8-9); this build defines them after DeepSeek-V3.2's attention block (absorbed MLA and the
 * lightning indexer), for one new token per request:
 *   cq   = rmsnorm(x Wq_a^T) * q_norm, rounded to the input type          (B, 1536)
 *   q    = [nope_h W_uk[h]^T | rope(pe_h)] per head h of cq Wq_b^T = [nope (128) | pe (64)]
 *   iq   = [rope_half(pe_j) | nope_j] per head j of cq Wiq_b^T = [pe (64) | nope (64)]
 *   w    = (x Wiw^T) / sqrt(64 * 128)                                     (B, 64) fp32, the op's pre-scaled w
 *   kv[b, pos[b]] = [rmsnorm(kv_c) * kv_norm | rope(k_pe)],  [kv_c (512) | k_pe (64)] = x Wkv_a^T
 *   ik[b, pos[b]] = layernorm(x Wik^T) * ik_norm_w + ik_norm_b, rope_half on its first 64 dims
 * RMSNorm/LayerNorm eps 1e-6.  Both RoPE forms rotate pair i by rope_cos/rope_sin[pos[b], i] (tables of
 * (rope_rows, 32) fp32; pos is clamped into them): MLA's `rope` (q's and kv's rope parts) pairs interleaved
 * neighbours (v[2i], v[2i+1]); the indexer's `rope_half` (iq, ik) pairs the halves (v[i], v[i+32]), as
 * DeepSeek-V3.2's indexer applies it (not interleaved).  The indexer's Hadamard rotation of DeepSeek-V3.2 is
 * orthonormal and leaves every iq . ik unchanged, so it is not applied.
 * Matrices are row-major (out, in), 16-bit like x (fp16; bf16 for the _bf16 entry); W_uk is the absorbed key half of
 * Wkv_b pre-transposed to (128 heads, 512 latent, 128 nope); norm weights are fp32.  The struct is read on the host
 * (its fields are device pointers).
 *   x (B, 7168), pos (B,) int32, q (B, 128, 576), iq (B, 64, 128), w (B, 64) fp32, kv (B, L, 576), ik (B, L, 128)
 * Only row pos[b] of each request's kv and ik is written, and only when 0 <= pos[b] < L. */
typedef struct vmk_dsa_project_weights {
  const void* wq_a;       /* (1536, 7168) */
  const void* q_norm;     /* (1536,) fp32 */
  const void* wq_b;       /* (24576, 1536): head h rows [192 h, 192 h + 128) nope, then 64 pe */
  const void* w_uk;       /* (128, 512, 128) */
  const void* wkv_a;      /* (576, 7168) */
  const void* kv_norm;    /* (512,) fp32 */
  const void* iwq_b;      /* (8192, 1536): head j rows [128 j, 128 j + 64) pe, then 64 nope */
  const void* iwk;        /* (128, 7168) */
  const void* ik_norm_w;  /* (128,) fp32 */
  const void* ik_norm_b;  /* (128,) fp32 */
  const void* iw;         /* (64, 7168) */
} vmk_dsa_project_weights;
size_t vmk_dsa_project_workspace_size(int64_t B);
int vmk_dsa_project(const void* x, const void* pos, const void* rope_cos, const void* rope_sin, int64_t rope_rows,
                    const vmk_dsa_project_weights* weights, void* q, void* iq, void* w, void* kv, void* ik, int64_t B,
                    int64_t L, void* workspace, size_t ws_bytes, void* stream);
int vmk_dsa_project_bf16(const void* x, const void* pos, const void* rope_cos, const void* rope_sin,
                         int64_t rope_rows, const vmk_dsa_project_weights* weights, void* q, void* iq, void* w,
                         void* kv, void* ik, int64_t B, int64_t L, void* workspace, size_t ws_bytes, void* stream);

/* The whole decode step: vmk_dsa_indexer_select followed by vmk_dsa_sparse_mla (idx/cnt are written). */
int vmk_dsa_decode(const void* q, const void* kv, const void* iq, const void* ik, const void* w, const void* lens,
                   void* out, void* idx, void* cnt, int64_t B, int64_t L, void* workspace, size_t ws_bytes,
                   void* stream);
/* The same decode step as ONE kernel launch (the reference's chain of 5-6 launches, dsa_opus55_v7.py:946-977, and
 * vmk_dsa_decode's four, fused): indexer, select, attention and combine run as phases of one grid of at most one
 * co-resident round of workgroups, separated by grid barriers.  Same arguments, workspace size and outputs as
 * vmk_dsa_decode, bit for bit.  Every grid-barrier wait is bounded: if one gives up (workgroups that were not
 * resident together, e.g. beside another kernel on the device), the call still ends, and reports cnt[b] = -1 for
 * every request; the workspace then stays marked (every later call on it reports -1 the same way) until its head
 * is zeroed. */
int vmk_dsa_decode_single(const void* q, const void* kv, const void* iq, const void* ik, const void* w,
                          const void* lens, void* out, void* idx, void* cnt, int64_t B, int64_t L, void* workspace,
                          size_t ws_bytes, void* stream);
int vmk_dsa_decode_single_bf16(const void* q, const void* kv, const void* iq, const void* ik, const void* w,
                               const void* lens, void* out, void* idx, void* cnt, int64_t B, int64_t L,
                               void* workspace, size_t ws_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------- measurement hook
 * No reference counterpart (the reference times whole calls only, bench.py:61-96).  The next launch of kernel
 * `kernel_id` on this host thread is bracketed by hipEventRecord(before) and hipEventRecord(after) on its stream.
 * Ids: 0 spec_partial, 1 spec_combine, 2 prefix_partial, 3 prefix_combine, 4 dsa_indexer, 5 dsa_select (final),
 *      6 dsa_attn, 7 dsa_combine, 8 dsa_select_scan, 9 the heads launch of vmk_dsa_project (its q, iq products and
 *      the absorbed product), 10 the single-launch DSA decode kernel. */
int vmk_profile_next(void* before_event, void* after_event, int kernel_id);

/* ---------------------------------------------------------------------------------------------- test hooks
 * No reference counterpart.  Lane-layout check of the 32x32x16 fp16 MFMA (a, b: 64 lanes x 8 fp16; d: 64 x 16 fp32),
 * and a stage dump of the attention wave pipeline for one 32-key tile (q, k, v: 32 x 128 fp16). */
int vmk_debug_mfma32(const void* a, const void* b, void* d, void* stream);
int vmk_debug_tile(const void* q, const void* k, const void* v, void* s, void* vt, void* o, void* ml, float sl2,
                   void* stream);
/* Host-only replay (no GPU work) of the DSA select's threshold-bucket search, with the kernels' own bin arithmetic:
 * coarse_hist (256) and fine_hist (8192) counts in host memory, need = picks (2048) -> out[0] coarse bin, out[1]
 * picks left in it, out[2] fine bucket.  Every bin it returns is inside the histograms, whatever the counts. */
int vmk_debug_select_threshold(const uint32_t* coarse_hist, const uint32_t* fine_hist, uint32_t need, uint32_t* out);

#ifdef __cplusplus
}
#endif

#endif /* VMK_H */
