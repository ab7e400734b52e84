/* C ABI of the MI355X tiered quantized KV cache (int8ring_int4) -- libkvtier.so.
 *
 * Conventions (every entry point):
 *   - all tensor memory is owned and allocated by the caller (device pointers of torch tensors); the library
 *     keeps no state and allocates nothing -- except the kvt_vmm_* arena entry points at the end, whose purpose
 *     is to reserve device address space and back it with physical memory on demand;
 *   - work is enqueued on `stream` (a hipStream_t, e.g. torch.cuda.current_stream().cuda_stream); no entry point
 *     synchronizes the host, grid sizes depend only on the integer arguments (capture-safe);
 *   - the return value is KVT_OK (0) or a negative status: KVT_EINVAL (-1) unsupported shape / dtype / size,
 *     KVT_ELAUNCH (-2) the launch failed, KVT_ERANGE (-3) a size beyond a documented maximum; the arena entry
 *     points add KVT_ENOTSUP (-4) no virtual memory management on the device, KVT_ENOMEM (-5) no address space
 *     or physical memory, KVT_EHIP (-6) another HIP runtime failure.
 *
 * Layouts (reference: patches/kv_int4.py:57-60, patches/kv_tiers.py:63-67):
 *   INT4 pool   k_buf/v_buf uint8 [rows, H, D/2] (low nibble = even channel, q + 8);
 *               k_scale/v_scale fp16 [rows, H, D/32]
 *   INT8 ring   ring_k/ring_v int8 [R, H, D]; ring_ks/ring_vs fp16 [R, H, D/group8] (group8 = 64, or D for the
 *               per-(token, head) form); owner int32 [R] (slot rings only)
 *   sm_k/sm_v, sm_k_inv/sm_v_inv: fp16 [H, D] smoothing constants (identity in the served setup), may be NULL.
 * Element type codes for K/V inputs: 0 = bf16, 1 = fp16, 2 = fp32.
 */
#ifndef KVTIER_H
#define KVTIER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVT_OK 0
#define KVT_EINVAL -1
#define KVT_ELAUNCH -2
#define KVT_ERANGE -3
#define KVT_ENOTSUP -4
#define KVT_ENOMEM -5
#define KVT_EHIP -6

/* ----------------------------------------------------------------------------------------- write path */

/* Dual write of N tokens: stamps owner[slot & ring_mask] = slot, then writes the INT8 ring row (owner only) and
 * the INT4 pool row (always).  k/v: [N, H, D] with element strides (sk_n, sk_h), unit last stride; loc int32 or
 * int64 [N].  Replaces quant_store_kv_tiered + _stamp_ring_owner + _quant_store_kv_tiered
 * (patches/kv_tiers.py:272-443). */
int kvt_quant_store_tiered(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n,
                           int64_t sv_h, const void* loc, int loc_is_int64, int64_t N, int H, int D, void* k_buf,
                           void* v_buf, void* k_scale, void* v_scale, void* ring_k, void* ring_v, void* ring_ks,
                           void* ring_vs, void* owner, const void* sm_k_inv, const void* sm_v_inv, int64_t ring_mask,
                           int group8, void* stream);

/* INT8-G quantize + scatter into int8 [rows, H, D] + fp16 [rows, H, D/group8] at loc.  Replaces
 * quant_store_kv_int8 / _quant_store_kv_int8 (patches/kv_int8.py:281-362; scale clamped to fp16 max as in the
 * tiered writer, patches/kv_tiers.py:336-337). */
int kvt_quant_store_int8(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n,
                         int64_t sv_h, const void* loc, int loc_is_int64, int64_t N, int H, int D, void* k_buf,
                         void* v_buf, void* k_scale, void* v_scale, const void* sm_k_inv, const void* sm_v_inv,
                         int group8, void* stream);

/* INT4-G32 quantize + nibble pack + scatter at loc.  Replaces quant_store_kv_int4 / _quant_store_kv_int4
 * (patches/kv_int4.py:289-393). */
int kvt_quant_store_int4(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n,
                         int64_t sv_h, const void* loc, int loc_is_int64, int64_t N, int H, int D, void* k_buf,
                         void* v_buf, void* k_scale, void* v_scale, const void* sm_k_inv, const void* sm_v_inv,
                         void* stream);

/* page_table[seq[i] * pt_stride + lpage[i]] = ppage[i] for i < n (int32 arrays on the device).  The page-table
 * update of the evict-mode write path; no reference counterpart (the reference only specifies the compactor's
 * bookkeeping, docs/KV_TIERS_PLAN.md:63-67). */
int kvt_page_table_update(void* page_table, int64_t pt_stride, int64_t n, const void* seq, const void* lpage,
                          const void* ppage, void* stream);

/* Device-side plan of an evicting append, so that a whole append (+ decode) step needs no host work and captures
 * into a HIP graph.  Sequence seqs[j] (j < n, distinct, n <= 1024) appends cu[j+1] - cu[j] tokens (cu int32 [n+1],
 * cu[0] = 0) at positions L0 .. L0 + cnt - 1, L0 = seq_lens[seqs[j]] when the plan runs.  Writes seq_ids int32 [N]
 * and positions int64 [N] (N = cu[n]: the inputs of kvt_append_evict), gives every page that evicted positions enter
 * for the first time (e = p - ring_len >= ring_start, e % 64 == 0) the next entry of free_list (int32 [n_pages], read
 * from *free_head on), in call order -- sequence j before j + 1, positions ascending, the order of a host allocator
 * walking the same plan -- writes it to page_table[s][e / 64], advances *free_head and sets seq_lens[s] = L0 + cnt.
 * A page that cannot be given (free list exhausted: *status |= 1; logical page >= max_pages: |= 2) stays
 * unassigned and kvt_append_evict then skips that token's requantization (no write outside the pool).  No reference
 * counterpart: the reference's slot allocator is host code (the compactor bookkeeping of docs/KV_TIERS_PLAN.md:63-67
 * was never built). */
int kvt_append_plan(int n, const void* seqs, const void* cu, void* seq_lens, const void* ring_len,
                    const void* ring_start, void* page_table, int64_t pt_stride, int max_pages, const void* free_list,
                    int n_pages, void* free_head, void* seq_ids, void* positions, void* status, void* stream);

/* Position-ring append of N tokens (seq_ids int32 [N], positions int64 [N]; per sequence ring_base int64,
 * ring_len int32 (power of two), ring_start int64): if e = p - ring_len >= ring_start, ring row
 * ring_base + (p & (ring_len - 1)) is first requantized (f32(q8) * f32(s8) -> INT4-G32) into pool row
 * page_table[seq][e / 64] * 64 + e % 64, then the token is quantized into that ring row.  Tokens of one call
 * must use distinct ring rows.  Implements the compactor's _requant_kv_int8_to_int4 (docs/KV_TIERS_PLAN.md:53,
 * :82) fused with the ring write of _quant_store_kv_tiered (patches/kv_tiers.py:325-351). */
int kvt_append_evict(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n, int64_t sv_h,
                     const void* seq_ids, const void* positions, int64_t N, int H, int D, void* k_buf, void* v_buf,
                     void* k_scale, void* v_scale, void* ring_k, void* ring_v, void* ring_ks, void* ring_vs,
                     const void* ring_base, const void* ring_len, const void* ring_start, const void* page_table,
                     int64_t pt_stride, const void* sm_k_inv, const void* sm_v_inv, int group8, void* stream);

/* ----------------------------------------------------------------------------------------- gathers */

/* Valid top-k counts and the packing offsets of kvt_compact_gather, in one launch: counts[b] = the number of columns
 * c < topk whose position indices[b * idx_stride + c] lies in [0, seq_lens[b]); cu_k[0] = 0 and cu_k[b + 1] =
 * counts[0] + ... + counts[b] (int32, or int64 if cu_is_int64).  seq_lens, indices and counts are int32; idx_stride
 * >= 0 (0: every request reads row 0).  Replaces the upstream qwen_sparse_fa2_cu_seqlens_triton the reference calls
 * before a compact gather (gemv/test_kv_tiers.py:297-301, gemv/test_kv_int4.py:150). */
int kvt_sparse_cu_seqlens(const void* seq_lens, const void* indices, int64_t idx_stride, void* counts, void* cu_k,
                          int cu_is_int64, int batch, int topk, void* stream);

/* Top-k gather-dequant into a bf16 scratch [*, H, D]: column c of request b is written at row cu_k[b] + c iff
 * c < cu_k[b+1] - cu_k[b] and 0 <= indices[b][c] < seq_lens[b]; nothing else is written.  kind 0 = INT8 pool
 * (k/v are the int8 codes, ring arguments unused), 1 = INT4 pool, 2 = tiered (owner test per row).  Replaces
 * qwen_sparse_kv_extraction_compact_triton's int8 / int4 / tiered branches (_compact_kv_int8
 * patches/kv_int8.py:365-420, _compact_kv_int4 patches/kv_int4.py:396-460, _compact_kv_tiered
 * patches/kv_tiers.py:446-538, wrapper :688-737).  Pointer alignment (else KVT_EINVAL): INT4 codes 4 bytes, INT8
 * codes and ring codes 8 bytes, out_k / out_v 16 bytes (any torch allocation or row slice of one qualifies). */
int kvt_compact_gather(int kind, const void* k, const void* v, const void* k_scale, const void* v_scale,
                       const void* ring_k, const void* ring_v, const void* ring_ks, const void* ring_vs,
                       const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                       const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                       const void* indices, int64_t idx_stride, const void* seq_lens, const void* cu_k,
                       int cu_is_int64, int batch, int topk, int H, int D, int group8, void* out_k, void* out_v,
                       void* stream);

/* Top-k sparse decode attention, fused: for request b (one query row, q bf16 [batch, Hq, D] with batch stride
 * q_stride_b elements, 16-byte aligned), the selected columns c < cu_k[b+1] - cu_k[b] (and < topk) whose position
 * indices[b * idx_stride + c] lies in [0, seq_lens[b]) are resolved through req_to_token[req_indices[b]] and, for
 * kind 2, the owner table, dequantized as kvt_compact_gather writes them (bf16(q * s * sm)) and attended with scale;
 * bf16 matrix-core products, fp32 accumulation.  Split s of a (request, KV head) covers columns [64 T s, 64 T (s + 1))
 * with T = ceil(ceil(topk / 64) / n_splits) (T > 1: each wavefront loops over T 16-column tiles) and writes one
 * unnormalized partial to part_o (fp32 [batch * H * n_splits, Hq / H, D]) and part_ml ([..., 2]); one (request, KV
 * head)'s partials n_splits * Hq / H * D * 4 bytes < 2^31, else KVT_EINVAL.  counters NULL:
 * merge them afterwards with kvt_decode_combine(n_chunks = n_splits, chunk = 0, split_counts = NULL).  counters
 * (int32 [batch * H], zero before the first call; every call leaves them zero): the launch merges them itself -- the
 * block of a (request, KV head) that counts last merges its n_splits partials in split order and writes out_f32 or
 * out_bf16 (exactly one; [batch, Hq, D] rows with batch stride out_stride_b >= Hq * D, a multiple of 8, 16-byte
 * aligned); calls sharing the counters and
 * partials must not overlap.  Faster than the combine launch for few splits (<= 8), slower for many: one block
 * reads all of a (request, KV head)'s partials.  A request with no attended column comes out
 * NaN (0/0).  n_splits >= 1; Hq / H <= 16, D = 256.  Kinds and buffers as kvt_compact_gather; pool_rows = rows of k / v (byte offsets
 * are 32-bit: pool_rows * H * D (INT8) or * D / 2 (INT4) < 2^31, else KVT_ERANGE).  No reference counterpart: it replaces the
 * compact gather + FlashAttention-2 pair of the reference's decode (flat patch
 * sglang/qwen4exp-serving-73a255206f.patch:1832-1882) for top-k selections. */
int kvt_sparse_decode(int kind, const void* q, int64_t q_stride_b, const void* k, const void* v, const void* k_scale,
                      const void* v_scale, int64_t pool_rows, const void* ring_k, const void* ring_v, const void* ring_ks,
                      const void* ring_vs, const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                      const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                      const void* indices, int64_t idx_stride, const void* seq_lens, const void* cu_k,
                      int cu_is_int64, int batch, int topk, int H, int Hq, int D, int group8, float scale,
                      int n_splits, void* part_o, void* part_ml, void* counters, void* out_f32, void* out_bf16,
                      int64_t out_stride_b, void* stream);

/* Prefix-chunk sparse attention read straight from a quantized pool.  Chunk b owns query rows cu_q[b] ..
 * cu_q[b+1] of q (bf16, row r / q head j at q + r sq_n + j sq_h); its context holds kv_lens[b] positions, resolved
 * through req_to_token[req_indices[b]] (and, kind 2, the owner table) and dequantized as kvt_compact_gather writes
 * them.  Query j of the chunk (q_len rows) attends the entries of its index row (int32, row r / KV head h / column c
 * at indices + r si_m + h si_g + c si_n) among the first min(topk, j + kv_len - q_len + 1) that lie in [0, kv_len);
 * the result is written normalized to out (bf16, or fp32 when out_f32; row r / q head j at out + r so_n + j so_h);
 * a row with no attended entry gives NaN (0/0).  bf16 matrix-core products, fp32 accumulation.  Grid: max_q rows per
 * chunk (the longest chunk).  Hq / H <= 16, D = 256; q and out 16-byte aligned with row and head strides multiples of
 * 16 bytes (else KVT_EINVAL); pool_rows and ring sizes as kvt_sparse_decode.  Replaces sparse_gqa_fwd_interface_paged
 * / _sparse_gqa_chunk_prefill_paged (patches/kv_paged_prefix.py:141-365). */
int kvt_sparse_prefill(int kind, const void* q, int64_t sq_n, int64_t sq_h, const void* cu_q, int cu_q_is_int64,
                       const void* kv_lens, int batch, int max_q, const void* indices, int64_t si_m, int64_t si_g,
                       int64_t si_n, int topk, const void* k, const void* v, const void* k_scale, const void* v_scale,
                       int64_t pool_rows, const void* ring_k, const void* ring_v, const void* ring_ks,
                       const void* ring_vs, const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                       const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64, int H,
                       int Hq, int D, int group8, float scale, void* out, int out_f32, int64_t so_n, int64_t so_h,
                       void* stream);

/* Whole-prefix gather-dequant: rows [0, seq_lens[b]) of request req_indices[b] packed at cu_k[b]; rows at or
 * beyond seq_lens[b] are not written.  Replaces qwen_sparse_prefix_gather_dequant_{int8,int4,tiered}
 * (patches/kv_int8.py:469-504, patches/kv_int4.py:519-557, patches/kv_tiers.py:639-683).  Pointer alignment as
 * kvt_compact_gather. */
int kvt_prefix_gather(int kind, const void* k, const void* v, const void* k_scale, const void* v_scale,
                      const void* ring_k, const void* ring_v, const void* ring_ks, const void* ring_vs,
                      const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                      const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                      const void* seq_lens, const void* cu_k, int cu_is_int64, int batch, int64_t max_len, int H,
                      int D, int group8, void* out_k, void* out_v, void* stream);

/* ----------------------------------------------------------------------------------------- decode attention */

/* Split-K GQA decode attention, reference precision (exact bf16 dequant, fp32 softmax).  One query per sequence:
 * q bf16 [batch, Hq, D] (batch stride q_stride_b elements).  mode 0 = position rings (ring_base/ring_len/
 * ring_start per sequence + page_table), mode 1 = slot rings (req_to_token, req_indices int64, owner, ring_mask).
 * Writes per (sequence, KV head, chunk) partials part_o fp32 [batch*H*n_chunks, Hq/H, D] and part_ml fp32
 * [.., Hq/H, 2] (running max, sum of exp).  chunk <= 512.  Stands in for the reference's decode attention
 * (top-k compact gather + flash_attn_varlen_func, flat patch sglang/qwen4exp-serving-73a255206f.patch:1832-1882),
 * dense over the whole context. */
int kvt_decode_ref(int mode, const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int H, int Hq, int D,
                   int group8, const void* k4, const void* v4, const void* ks4, const void* vs4, const void* rk,
                   const void* rv, const void* rks, const void* rvs, const void* sm_k, const void* sm_v,
                   const void* ring_base, const void* ring_len, const void* ring_start, const void* page_table,
                   int64_t pt_stride, const void* req_to_token, int64_t req_stride, const void* req_indices,
                   const void* owner, int64_t ring_mask, float scale, int chunk, int n_chunks, void* part_o,
                   void* part_ml, void* stream);

/* Split-K GQA decode attention on the matrix cores over position rings + page tables (the mode-0 layout of
 * kvt_decode_ref): QK^T with exact fp16 integer codes and the per-group scales folded in fp32; P.V with the raw INT4
 * codes as exact fp16 values and the V scale folded into fp16 P; fp32 accumulation.  Each split is one block of 8
 * wavefronts (one block per CU) over a position range of equal cost; its tiles go to the wavefronts either first come
 * (flags & KVT_DECODE_DYNAMIC: the wavefronts finish together; the fp32 summation order, and so the last bits of the
 * result, then depend on timing) or in a fixed order (bit-reproducible).
 * Two kernels: for H = 2 and Hq / H <= 8 (unless flags & KVT_DECODE_HEADWISE) a block covers both KV heads of its
 * positions and reads whole pool rows (16-position tiles of both heads per wavefront); otherwise a block covers one
 * (sequence, KV head) (32-position tiles).  split_map NULL: every item -- a sequence for the full-row kernel, a
 * (sequence, KV head) for the head-wise one -- gets n_splits splits; otherwise split_map (int32 [n_map][3] =
 * {sequence, split index, splits of that sequence}) lists the splits (per-sequence counts for ragged batches), the
 * grid has n_map blocks (full-row) or n_map x H (head-wise), and n_splits is the partial slot stride.  Partials in the
 * layout of kvt_decode_ref (n_splits slots per (sequence, KV head)); merge them with kvt_decode_combine(chunk = 0,
 * split_counts).  plan (full-row kernel only; NULL or a kvt_decode_plan output for the same grid): each block starts
 * from its plan entry (ranges and first tile rows: one load before the first copies); an entry made for another
 * length or ring placement of its sequence is detected and the block computes its ranges itself.  The plan's tile
 * rows come from the page table at planning time: re-plan after the page table changes.  Hq / H <= 16, D = 256,
 * group8 64 or 256, q and q_stride_b 16-byte aligned (else KVT_EINVAL); pool_rows = rows of the INT4 pool (byte
 * offsets are 32-bit: pool_rows * H * D / 2 < 2^31, else KVT_ERANGE).  No reference counterpart: it replaces the
 * compact gather + FA2 pair (flat patch sglang/qwen4exp-serving-73a255206f.patch:1832-1882) for dense decode. */
#define KVT_DECODE_DYNAMIC 1
#define KVT_DECODE_HEADWISE 2
int kvt_decode_mfma(const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int H, int Hq, int D,
                    int group8, const void* k4, const void* v4, const void* ks4, const void* vs4, const void* rk,
                    const void* rv, const void* rks, const void* rvs, const void* ring_base, const void* ring_len,
                    const void* ring_start, const void* page_table, int64_t pt_stride, int64_t pool_rows,
                    float scale, int n_splits, const void* split_map, int n_map, void* part_o, void* part_ml,
                    int flags, const void* plan, void* stream);

/* The decode plan of one step for the full-row kvt_decode_mfma grid (batch sequences x n_splits splits, or the n_map
 * entries of split_map): per block 64 int32 words -- sequence, split, split count, ring length, length, ring start,
 * ring base, first ring position, range [w0, w1), and the pool rows of the block's first 16 paged tiles -- computed
 * from the device state (one thread per block, one small launch; capturable).  Shared by every layer of the step:
 * a block's first copies then wait for one load instead of the length -> range -> page-table chain.  plan: int32
 * [blocks * 64].  No reference counterpart (the reference's decode is FA2 over a gathered scratch). */
int kvt_decode_plan(const void* seq_lens, const void* ring_len, const void* ring_start, const void* ring_base,
                    const void* page_table, int64_t pt_stride, int batch, int n_splits, const void* split_map,
                    int n_map, void* plan, void* stream);

/* Merge the split-K partials: out[b, hq, :] = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c (fp32 and/or bf16
 * output, either may be NULL; batch stride out_stride_b elements).  chunk > 0: split c covers positions
 * [c chunk, (c + 1) chunk) and splits beyond the length are skipped; chunk = 0: the first split_counts[b] of the
 * n_chunks slots of sequence b hold partials (all n_chunks if split_counts is NULL; an empty one carries
 * m = -inf).  An empty context yields NaN (0/0), as the reference's chunk kernel
 * (gemv/test_kv_paged_prefix.py:524-526). */
int kvt_decode_combine(const void* part_o, const void* part_ml, int batch, int H, int Hq, int D, int n_chunks,
                       int64_t chunk, const void* seq_lens, const void* split_counts, void* out_f32, void* out_bf16,
                       int64_t out_stride_b, void* stream);

/* kvt_decode_mfma followed by kvt_decode_combine(n_chunks = n_splits, chunk = 0, split_counts), with the split
 * partials in a scratch array that the library holds on each GPU (8 MiB, a file-scope device array kept until the
 * process ends) instead of caller-provided part_o / part_ml: the entry point allocates nothing.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The partials need batch * H * n_splits * (Hq / H) * (D + 2) * 4 bytes
 * (the o part rounded up to 256 bytes); more than 8 MiB returns KVT_ERANGE before anything is launched (the
 * 262,144-position headline at 256 splits needs 4.0 MiB).  split_map and split_counts (int32 [batch],
 * the splits of each sequence) go together, as for the pair of calls this replaces; out_f32 and / or out_bf16 as
 * kvt_decode_combine.  Every call on a GPU shares that GPU's scratch: calls that overlap on one GPU (concurrent
 * streams, other threads) race and must be serialized by the caller. */
int kvt_decode_mfma_noalloc(const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int H, int Hq, int D,
                            int group8, const void* k4, const void* v4, const void* ks4, const void* vs4,
                            const void* rk, const void* rv, const void* rks, const void* rvs, const void* ring_base,
                            const void* ring_len, const void* ring_start, const void* page_table, int64_t pt_stride,
                            int64_t pool_rows, float scale, int n_splits, const void* split_map, int n_map,
                            const void* split_counts, int flags, void* out_f32, void* out_bf16, int64_t out_stride_b,
                            void* stream);

/* Causal prefill attention of a chunk of queries over the position-indexed tiered cache on the matrix cores
 * (K/V tiles dequantized once per block into LDS as the exact bf16 rows bf16(code * scale); QK^T on
 * v_mfma_f32_16x16x32_bf16; P.V on v_mfma_f32_16x16x32_f16 with P rounded to fp16 and V = the bf16 rows / 128 in
 * fp16; fp32 softmax and accumulation).  Sequence b's queries are rows
 * cu_q[b] .. cu_q[b+1] of q (bf16 [total_q, Hq, D], strides sq_n / sq_h) at positions kv_lens[b] - q_len .. ;
 * each attends to every position <= its own (patches/kv_paged_prefix.py:200), read from the cache tiers of
 * sequence b, or, when k_bf16 / v_bf16 are given (batch 1, a chunk without a prefix), from those bf16
 * [positions, H, D] rows (the reference attends to fresh bf16 K/V there; |V| <= 128 * 65504).  out: bf16 or fp32
 * (out_f32) with the layout of q.  Replaces sparse_gqa_fwd_interface_paged (patches/kv_paged_prefix.py:267-365) for dense causal
 * chunks.  Hq / H <= 16, D = 256; q 16-byte aligned with sq_n, sq_h multiples of 8 (Q rows are read 16 bytes at a
 * time); pool_rows = rows of the INT4 pool and kb_rows = rows of the bf16 source (byte offsets are 32-bit, else
 * KVT_ERANGE).  A block stages the page ids of its paged positions in LDS: at most 8,192
 * pages (paged positions below 524,288) per sequence; a query tile whose paged key range exceeds it gets NaN outputs
 * (never keys from the wrong pages), and the Python wrapper refuses such a call from its host lengths.
 * spread_blocks > 0: that many blocks share the launch's key tiles equally (query tiles are split where a share
 * ends; of a query tile's pieces, the one that finishes last merges them in piece order), instead of one block
 * per query tile -- the latest query tiles of a causal chunk see up to a chunk length more keys than the earliest,
 * so one block per CU with equal shares ends them all together.  It needs `work`, at least kvt_prefill_work_bytes
 * bytes, whose counter area (its first 16 KB, the same for every call) is zero before the first call -- each call
 * leaves it at zero again;
 * calls that share a workspace must not overlap; at most 4,096 query tiles (batch x H x tiles of 128 rows), else
 * KVT_ERANGE.  The output does not depend on which block merges. */
int kvt_prefill_attn(const void* q, int64_t sq_n, int64_t sq_h, const void* cu_q, int cu_q_is_int64,
                     const void* kv_lens, int batch, int max_q, int H, int Hq, int D, int group8, const void* k4,
                     const void* v4, const void* ks4, const void* vs4, const void* rk, const void* rv,
                     const void* rks, const void* rvs, const void* ring_base, const void* ring_len,
                     const void* ring_start, const void* page_table, int64_t pt_stride, int64_t pool_rows,
                     const void* k_bf16, const void* v_bf16, int64_t kb_rows, int64_t kb_n, int64_t kb_h,
                     int64_t vb_n, int64_t vb_h, float scale, void* out, int out_f32, int64_t so_n, int64_t so_h,
                     int spread_blocks, void* work, int64_t work_bytes, void* stream);

/* Bytes of the kvt_prefill_attn workspace for these shapes and spread_blocks (0 for spread_blocks 0): a zeroed
 * 4-byte counter per (sequence, KV head, query tile of 128 rows), padded to 256 bytes, and a 132,096-byte state
 * slot (O, m, l of 128 rows in fp32) per query tile plus one per block beyond the first.  No counterpart in the
 * reference (its prefill kernel takes one block per query row). */
int kvt_prefill_work_bytes(int batch, int H, int Hq, int max_q, int spread_blocks, int64_t* bytes);

/* ----------------------------------------------------------------------------- lazy backing (HIP VMM) */

/* Lazily backed device memory for the KV pool (reference: patches/kv_lazy.py -- the pool is reserved as address
 * space for the whole context and backed in steps as pages are handed out; beyond a floor the backing goes back to
 * the driver when the pool is idle).  An arena is one reserved range on `device`; its first `backed` bytes are
 * mapped read-write for that device, the rest is address space only -- a kernel must not touch it.  Every call is
 * host-synchronous; calls that unmap wait for the device's queued work first (hipDeviceSynchronize).  A failed
 * runtime call is also reported on stderr (which call, offset, size, the runtime's message). */

/* Mapping granularity of the arenas: 2 MiB (a multiple of the runtime's recommended granularity): every mapping is
 * whole granules at granule-aligned addresses.  KVT_ENOTSUP without VMM. */
int kvt_vmm_granularity(int device, uint64_t* granularity);

/* Reserve `bytes` (rounded up to the granularity) of address space; nothing is backed yet.  Returns the arena
 * handle and its base address.  Replaces the VMM owner's reservation (SGLang's kv_vmm_backing owner, used in
 * lazy mode by patches/kv_lazy.py:100-106). */
int kvt_vmm_reserve(int device, uint64_t bytes, void** arena, void** base);

/* Back the prefix [0, bytes) (rounded up to the granularity) -- one physical allocation per granule not yet
 * backed; a smaller or equal size is a no-op (commits only grow); KVT_ERANGE past the reservation, KVT_ENOMEM when
 * the device has no physical memory (the granules mapped before the failure stay backed).  Replaces ensure_prefix
 * (patches/kv_lazy.py:70-75). */
int kvt_vmm_commit(void* arena, uint64_t bytes);

/* Unmap and free every mapping (granule) that starts at or beyond align_up(keep_bytes, granularity)
 * (patches/kv_lazy.py:39-63 uncommit_beyond: mappings straddling the cut stay; one-granule mappings never do).  *freed (may be NULL) = bytes returned. */
int kvt_vmm_release_beyond(void* arena, uint64_t keep_bytes, uint64_t* freed);

/* Backed bytes, reserved bytes and number of mappings (any pointer may be NULL). */
int kvt_vmm_backed(void* arena, uint64_t* bytes, uint64_t* reserved, uint64_t* n_mappings);

/* Unmap and free everything and give the address space back; NULL is a no-op. */
int kvt_vmm_destroy(void* arena);

#ifdef __cplusplus
}
#endif

#endif /* KVTIER_H */
