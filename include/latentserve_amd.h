/*
 * latentserve_amd — C ABI of the MI355X (gfx950) paged GQA decode-attention
 * library (liblatentserve_hip.so).
 *
 * Plain pointers, sizes and element strides; no framework types.  Every
 * device pointer is a HIP device allocation; `stream` is a hipStream_t (NULL
 * = the default stream).  Calls only enqueue work on `stream`: no host
 * synchronisation, no device-to-host reads, no allocation — every buffer,
 * including scratch, is the caller's, so the calls can be captured in a
 * HIP graph.  Return value: 0 on success, else an LS_ERR_* code with a
 * message from ls_last_error() (thread-local).
 *
 * Layouts (strides in elements, innermost dimension unit-stride):
 *   q           [B, H_kv, n_rep, 128] fp16        strides q_strides[3] = (b, h, r)
 *   k/v pool    [num_blocks, 16, H_kv, 128]       strides kv_strides[3] = (block, token, head)
 *   block_tables[B, max_pages] int32              row stride bt_stride; max_pages <= 2^24
 *   seq_lens    [B] int32
 *   k_scale     [num_blocks, H_kv, 128] fp32      ks_strides[2] = (block, head)
 *   v_scale     [num_blocks, 16, H_kv]  fp32      vs_strides[3] = (block, token, head)
 *   k_zero/v_zero: as k_scale / v_scale (asymmetric INT8 only, else NULL)
 *   k_residual  [R, 16, H_kv, 128] fp16           res_strides[3] = (row, token, head)
 *   res_rows    [B] int32 (row of k_residual holding each sequence's last page)
 *   out         [B, H_kv, n_rep, 128] fp16        out_strides[3] = (b, h, r)
 *   workspace   fp32 scratch of ls_decode_workspace_bytes() bytes, 256-byte
 *               aligned (B * num_splits * H_kv records of acc[n_rep][128],
 *               m[16], l[16]: a split workgroup's partials, indexed by its
 *               slot among its KV head's B * num_splits workgroups, which
 *               the kernel deals to sequences in proportion to their
 *               lengths); needed only when num_splits > 1
 *   counters    int32 [ls_decode_counter_ints(B, H_kv)] (larger is fine), zero
 *               before the first call; every call leaves it zero again (per
 *               (sequence, head), one 128-byte line apart: the count of
 *               split workgroups that have stored their partials).  Calls
 *               that share scratch must be ordered on one stream.
 *   max_seq_len the longest sequence in the call (the caller's bound, e.g.
 *               a graph bucket); it sets the pages per split.  A sequence
 *               longer than it is still handled (its split is re-derived on
 *               the device, as the reference does); 0 = always derive.
 *
 * The reference (Jash-Vora/LatentServe) has no C ABI: its kernels are CuPy
 * launches of extern "C" __global__ functions with positional pointer and
 * stride arguments.  Each entry point below names the reference interface it
 * replaces.
 */
#ifndef LATENTSERVE_AMD_H
#define LATENTSERVE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    LS_OK = 0,
    LS_ERR_INVALID = 1,    /* shape, dtype-size, alignment or pointer check failed */
    LS_ERR_HIP = 2,        /* the HIP runtime rejected the launch */
};

/* Message for the last non-zero return on this thread. */
const char* ls_last_error(void);

/* ABI version (bumped on any signature change or addition). */
int ls_abi_version(void);

/* What the runtime reports of a loaded kernel (hipFuncGetAttributes and
 * hipOccupancyMaxActiveBlocksPerMultiprocessor).  Replaces the reference's
 * kernel_resources (kernels/cuda/paged_decode_cuda.py:163-186, CUDA driver
 * function attributes; kernels/cuda/paged_sparse.py:254-265). */
typedef struct LsKernelResources {
    int regs;           /* vector registers a lane */
    int local_bytes;    /* private (spill) memory a lane: 0 means no spills */
    int shared_bytes;   /* static LDS a workgroup */
    int threads;        /* threads a workgroup of its launches */
    int groups_per_cu;  /* workgroups one CU holds at once */
} LsKernelResources;

/* `kernel`: "paged_decode_fp16", "paged_decode_int8" (asym, has_res: zero
 * points, fp16 last-page K), "paged_sparse_fp16" (a given list),
 * "sparse_attention_fp16" (selecting from given scores),
 * "sparse_attention_bounds_fp16" (one launch), "combine_splits",
 * "page_index", "page_index_heads", "page_mass", "page_select",
 * "page_bounds_update", "page_bounds_rebuild", "int8_decode_write",
 * "int8_finalize_blocks".  kv_heads: decode kernels pair the heads of an
 * even count in one workgroup; n_rep: the index kernels are specialised on
 * it.  Needs a current HIP device. */
int ls_kernel_resources(const char* kernel, int kv_heads, int n_rep, int asym, int has_res,
                        LsKernelResources* out);

/* Bytes of `workspace` a decode call with these sizes needs (0 when
 * num_splits == 1).  No counterpart in the reference, which sizes its
 * partial buffers in Python (kernels/gqa/paged_decode.py:783-787). */
size_t ls_decode_workspace_bytes(int batch, int kv_heads, int n_rep, int num_splits);

/* Length (int32 elements) of the arrival-counter array a decode call takes:
 * 32 per (sequence, KV head), so that no two pairs' counters share a cache
 * line.  No counterpart in the reference, whose split combine is a second
 * launch (paged_decode.py:689-706). */
size_t ls_decode_counter_ints(int batch, int kv_heads);

/* fp16 paged decode.  Replaces paged_decode_fp16 + the Triton combine, i.e.
 * paged_decode_cuda() for an fp16 pool (kernels/cuda/paged_decode_cuda.py:202-252,
 * kernels/cuda/paged_decode_fp16.cu:55-64) behind paged_decode_attention
 * (kernels/gqa/paged_decode.py:709-829).  One launch: the splits are merged
 * by the last workgroup of each (sequence, head) to finish.  Each split is a
 * contiguous page range whose pages the waves of its workgroup claim one by
 * one.  With num_splits == 1 the output is written directly and workspace is
 * not touched (it may be NULL). */
int ls_paged_decode_fp16(const void* q, const int64_t* q_strides, const void* k_pool,
                         const void* v_pool, const int64_t* kv_strides, int num_blocks,
                         const int32_t* block_tables, int64_t bt_stride, int max_pages,
                         const int32_t* seq_lens, void* out, const int64_t* out_strides,
                         float* workspace, int32_t* counters,
                         int batch, int kv_heads, int n_rep, int head_dim, int page,
                         int num_splits, int max_seq_len, float softmax_scale, void* stream);

/* fp16 paged decode that allocates nothing and takes no workspace or
 * counters: the same kernel as ls_paged_decode_fp16, its split records and
 * arrival counters in a fixed device array of the library (16 MiB of records
 * plus 65536 counter ints, held per GPU until the process ends).  No counterpart
 * in the reference: for callers that cannot allocate device memory (code
 * under graph capture, tight serving loops, harnesses that forbid it).
 * Returns LS_ERR_INVALID when ls_decode_workspace_bytes(batch, kv_heads,
 * n_rep, num_splits) exceeds 16 MiB or batch * kv_heads exceeds 2048.  The
 * first call on a device looks the array up and clears its counters on
 * `stream`.  All calls on one GPU share the array: calls that overlap on
 * one GPU (concurrent streams) race. */
int ls_paged_decode_fp16_noalloc(const void* q, const int64_t* q_strides, const void* k_pool,
                                 const void* v_pool, const int64_t* kv_strides, int num_blocks,
                                 const int32_t* block_tables, int64_t bt_stride, int max_pages,
                                 const int32_t* seq_lens, void* out, const int64_t* out_strides,
                                 int batch, int kv_heads, int n_rep, int head_dim, int page,
                                 int num_splits, int max_seq_len, float softmax_scale,
                                 void* stream);

/* INT8 paged decode.  Replaces paged_decode_int8 (kernels/cuda/paged_decode_int8.cu:87-102;
 * launcher kernels/cuda/paged_decode_cuda.py:236-244).  k_scale/v_scale
 * required (fp32); k_zero and v_zero both or neither; k_residual with
 * res_rows (res_capacity = rows in k_residual) or neither. */
int ls_paged_decode_int8(const void* q, const int64_t* q_strides, const void* k_pool,
                         const void* v_pool, const int64_t* kv_strides, int num_blocks,
                         const float* k_scale, const int64_t* ks_strides, const float* v_scale,
                         const int64_t* vs_strides, const float* k_zero, const float* v_zero,
                         const void* k_residual, const int64_t* res_strides, int res_capacity,
                         const int32_t* res_rows, const int32_t* block_tables, int64_t bt_stride,
                         int max_pages, const int32_t* seq_lens, void* out,
                         const int64_t* out_strides, float* workspace,
                         int32_t* counters, int batch, int kv_heads, int n_rep,
                         int head_dim, int page, int num_splits, int max_seq_len, float softmax_scale,
                         void* stream);

/* Page-subset (sparse) decode over sel[b, h, 0:n] logical pages, fp16 pool.
 * Replaces paged_sparse_fp16 (kernels/cuda/paged_sparse_fp16.cu:205-217; launcher
 * sparse_decode, kernels/cuda/paged_sparse.py:185-219).  With ratio > 0 each
 * sequence attends its first max(recent+1, ceilf(ratio*pages)) entries, capped
 * at its pages and num_sel; ratio <= 0 attends all num_sel.  Entries outside
 * [0, pages) are skipped.  The list is split on the device; max_seq_len is
 * not used. */
int ls_paged_sparse_fp16(const void* q, const int64_t* q_strides, const void* k_pool,
                         const void* v_pool, const int64_t* kv_strides, int num_blocks,
                         const int32_t* block_tables, int64_t bt_stride, int max_pages,
                         const int32_t* seq_lens, const int32_t* sel, const int64_t* sel_strides,
                         int num_sel, float ratio, int recent, void* out,
                         const int64_t* out_strides, float* workspace,
                         int32_t* counters, int batch, int kv_heads, int n_rep,
                         int head_dim, int page, int num_splits, int max_seq_len, float softmax_scale,
                         void* stream);

/* Sparse attention in one launch: each workgroup selects its sequence's
 * page lists from scores [B, H_kv, score_pages] fp32 (score_strides[2] =
 * (b, h); ls_page_scores writes them) as ls_page_select does (sorted = 0:
 * the sequence's budget max(recent+1, ceilf(ratio*pages)), capped at its
 * pages and k, of its best pages in page order, ties to the lower page),
 * then attends them as ls_paged_sparse_fp16 attends such a list; the same
 * list and partition, without the list ever leaving the chip.  k <=
 * score_pages <= 8192; ceil(k / num_splits) <= 1024.  Replaces
 * sparse_attention's select + sparse_decode (kernels/cuda/paged_sparse.py:
 * 222-251, select :164-168). */
int ls_sparse_attention_fp16(const void* q, const int64_t* q_strides, const void* k_pool,
                             const void* v_pool, const int64_t* kv_strides, int num_blocks,
                             const int32_t* block_tables, int64_t bt_stride, int max_pages,
                             const int32_t* seq_lens, const float* scores,
                             const int64_t* score_strides, int score_pages, int k, float ratio,
                             int recent, void* out, const int64_t* out_strides, float* workspace,
                             int32_t* counters, int batch, int kv_heads, int n_rep,
                             int head_dim, int page, int num_splits, int max_seq_len,
                             float softmax_scale, void* stream);

/* Merge split partials: combine_splits / _combine_kernel
 * (kernels/gqa/paged_decode.py:689-706, :422-471).  acc [B, H, S, rows, 128]
 * with strides acc_strides[4] = (b, h, s, row); m and l [B, H, S, rows] with
 * ml_strides[3] = (b, h, s), unit row stride, m in natural-log units; out
 * [B, H, n_rep, 128] fp16 (out_fp32 = 0) or fp32 (out_fp32 = 1). */
int ls_combine_splits(const float* part_acc, const int64_t* acc_strides, const float* part_m,
                      const float* part_l, const int64_t* ml_strides, void* out, int out_fp32,
                      const int64_t* out_strides, int batch, int kv_heads, int num_splits,
                      int n_rep, int head_dim, void* stream);

/* ---- page selection for sparse decode -------------------------------- *
 * kmin / kmax  [num_blocks, H_kv, 128] fp16, per-page per-channel min / max
 *              of K; bound_strides[2] = (block, head)
 * scores       [B, H_kv, >= max_pages] fp32; score_strides[2] = (b, h)
 * sel          [B, H_kv, >= k] int32 page indices; sel_strides[2] = (b, h)
 */

/* Quest page scores: for page p < pages(b) of each (sequence, KV head), the
 * max over its n_rep query heads of sum_d max(q_d*kmin_d, q_d*kmax_d); page 0
 * and the last `recent` pages +inf, pages past the sequence (or whose block
 * id lies outside the pool) -inf.  Replaces page_index
 * (kernels/cuda/paged_sparse_fp16.cu:78-130) / page_scores
 * (kernels/cuda/paged_sparse.py:104-123). */
int ls_page_scores(const void* q, const int64_t* q_strides, const void* kmin, const void* kmax,
                   const int64_t* bound_strides, int num_blocks, const int32_t* block_tables,
                   int64_t bt_stride, int max_pages, const int32_t* seq_lens, float* scores,
                   const int64_t* score_strides, int batch, int kv_heads, int n_rep, int head_dim,
                   int page, int recent, void* stream);

/* sparse_attention with bounds scoring in ONE launch: the page scores are
 * computed by the decode's own workgroups (each scores its share of its
 * sequence's pages, Quest bound of kmin/kmax fp16 [num_blocks, H_kv, 128],
 * bound_strides (block, head); page 0 and the last `recent` pages +inf,
 * pages past the end -inf), exchanged through `scores` fp32 [B, H_kv,
 * >= max_pages + 1] (the word after a row counts the workgroups that have
 * stored their share: all ones before the first call, and every call leaves
 * it so; the rows keep the last call's scores), then each workgroup selects
 * and attends as ls_sparse_attention_fp16 does.  A workgroup that does not
 * see every share stored within 50 us computes the scores it needs itself,
 * so no workgroup depends on another being resident.
 * THE COUNT WORDS MUST START AT ALL ONES (0xFFFFFFFF): a word left anywhere
 * in [0, num_splits - 2] (a zero-filled buffer, a launch that was aborted)
 * lets the readers take a row before every share is stored, and the
 * selection is then silently wrong; other values only cost the 50 us
 * fallback.  Fill a new score buffer with 0xFF bytes before its first call.
 * Replaces the index + select + attend steps of sparse_attention
 * (kernels/cuda/paged_sparse.py:222-251; page_index, paged_sparse_fp16.cu:
 * 78-130).  k <= max_pages <= 2048 (COOP_MAX_PAGES), n_rep <= 8
 * (COOP_MAX_NREP), ceil(k / num_splits) <= 1024; longer rows or more query
 * rows a KV head take ls_page_scores + ls_sparse_attention_fp16. */
int ls_sparse_attention_bounds_fp16(const void* q, const int64_t* q_strides,
                                    const void* k_pool, const void* v_pool,
                                    const int64_t* kv_strides, int num_blocks,
                                    const int32_t* block_tables, int64_t bt_stride,
                                    int max_pages, const int32_t* seq_lens, const void* kmin,
                                    const void* kmax, const int64_t* bound_strides,
                                    float* scores, const int64_t* score_strides, int k,
                                    float ratio, int recent, void* out,
                                    const int64_t* out_strides, float* workspace,
                                    int32_t* counters, int batch, int kv_heads, int n_rep,
                                    int head_dim, int page, int num_splits, int max_seq_len,
                                    float softmax_scale, void* stream);

/* Test hook, no counterpart in the reference: how long (ticks of the 100 MHz
 * s_memrealtime clock, 5000 = 50 us by default) a workgroup of
 * ls_sparse_attention_bounds_fp16 waits for the other workgroups' page scores
 * before computing the missing ones itself.  Any value gives the same
 * results (the scores are recomputed bit for bit); 0 forces the fallback.
 * Process-wide; read at each call. */
int ls_set_coop_wait_ticks(uint64_t ticks);

/* Bytes of `workspace` ls_page_scores_mass needs: the per-head logits,
 * fp32 [batch, kv_heads, n_rep, max_pages]. */
size_t ls_page_mass_workspace_bytes(int batch, int kv_heads, int n_rep, int max_pages);

/* Summed-mass page scores [B, H, 0:max_pages] fp32.  Replaces
 * page_scores_mass (kernels/cuda/paged_sparse.py:126-161, with the
 * page_index_heads kernel, kernels/cuda/paged_sparse_fp16.cu:141-190): each
 * query head's Quest bound of a page turned into an estimated attention
 * weight, softmax over the row's pages of bound * softmax_scale +
 * log(tokens in the page), summed over the KV head's query heads; page 0
 * and the last `recent` pages +inf, pages past the end -inf.  Two launches
 * (per-head logits into `workspace`, then the row softmaxes). */
int ls_page_scores_mass(const void* q, const int64_t* q_strides, const void* kmin,
                        const void* kmax, const int64_t* bound_strides, int num_blocks,
                        const int32_t* block_tables, int64_t bt_stride, int max_pages,
                        const int32_t* seq_lens, float* workspace, float* scores,
                        const int64_t* score_strides, int batch, int kv_heads, int n_rep,
                        int head_dim, int page, int recent, float softmax_scale,
                        void* stream);

/* Top-k pages per (sequence, KV head) from scores [.., 0:num_pages].
 * Replaces select (kernels/cuda/paged_sparse.py:164-168, torch.topk).
 * Order of equal scores: lower page first.  sorted = 1: sel[0:k] best
 * first.  sorted = 0: with ratio > 0, sel[0:n_b] holds the n_b =
 * min(max(recent+1, ceilf(ratio*pages_b)), pages_b, k) best pages of
 * sequence b (the entries ls_paged_sparse_fp16 attends with that ratio) and
 * sel[n_b:k] the next ones, each part in page order; ratio <= 0: the k best in
 * page order.  k <= num_pages <= 8192. */
int ls_page_select(const float* scores, const int64_t* score_strides, const int32_t* seq_lens,
                   int batch, int kv_heads, int num_pages, int k, float ratio, int recent,
                   int sorted, int32_t* sel, const int64_t* sel_strides, void* stream);

/* ls_page_scores then ls_page_select (sorted = 0), two launches on the
 * stream: the index and select steps of sparse_attention
 * (kernels/cuda/paged_sparse.py:222-251).  counters is unused (may be NULL;
 * a caller's buffer is left untouched).  k <= max_pages <= 8192.  With
 * sel == NULL this is ls_page_scores. */
int ls_sparse_index(const void* q, const int64_t* q_strides, const void* kmin, const void* kmax,
                    const int64_t* bound_strides, int num_blocks, const int32_t* block_tables,
                    int64_t bt_stride, int max_pages, const int32_t* seq_lens, float* scores,
                    const int64_t* score_strides, int32_t* counters, int k, float ratio,
                    int recent, int32_t* sel, const int64_t* sel_strides, int batch, int kv_heads,
                    int n_rep, int head_dim, int page, void* stream);

/* Page bounds on write: k_new [B, H_kv, 128] fp16 (kn_strides[2] = (b, h))
 * was just written at flat slot slots[b] (int64); a page's first token
 * resets its bounds, later tokens widen them.  Slots outside the pool are
 * skipped.  Replaces page_bounds_update (paged_sparse_fp16.cu:54-72) /
 * update_bounds (kernels/cuda/paged_sparse.py:86-101). */
int ls_page_bounds_update(const void* k_new, const int64_t* kn_strides, const int64_t* slots,
                          void* kmin, void* kmax, const int64_t* bound_strides, int num_blocks,
                          int batch, int kv_heads, int head_dim, int page, void* stream);

/* Every block's bounds over all 16 rows of the K pool (kv_strides as for
 * the decode calls).  Replaces rebuild_bounds (kernels/cuda/paged_sparse.py:81-84). */
int ls_page_bounds_rebuild(const void* k_pool, const int64_t* kv_strides, int num_blocks,
                           void* kmin, void* kmax, const int64_t* bound_strides, int kv_heads,
                           int head_dim, int page, void* stream);

/* ---- INT8 cache write side ------------------------------------------- *
 * Quantizer constants as the reference cache holds them (k_bits / v_bits
 * = 8: qmax 127, levels 255, offset 128; eps 1e-8).  recip = 1 divides by
 * qmax / levels as a multiply by the fp32 reciprocal formed on the host
 * (torch's `t / python_number` on a GPU, and the reference's int8_write.cu);
 * recip = 0 divides exactly (torch on the CPU).  Either way the codes and
 * scales are bit-exact with that form of the reference's torch ops.
 */

/* Decode-step write for one token per sequence: V [B, H_kv, 128] fp16
 * (v_strides[2] = (b, h)) quantized per (token, head) into flat_v int8
 * [num_slots, H_kv, 128] / flat_v_scale (and flat_v_zero when asym) fp32
 * [num_slots, H_kv] at row slots[b]; K [B, H_kv, 128] copied into the fp16
 * residual k_res [num_res, H_kv, 128] at row res_idx[b].  slots / res_idx
 * int64; rows outside [0, num_slots) / [0, num_res) are skipped.  Replaces
 * int8_decode_write (kernels/cuda/int8_write.cu:46-80; decode_write,
 * kernels/cuda/int8_write.py:61-82). */
int ls_int8_decode_write(const void* k, const int64_t* k_strides, const void* v,
                         const int64_t* v_strides, const int64_t* slots, const int64_t* res_idx,
                         void* flat_v, float* flat_v_scale, float* flat_v_zero, void* k_res,
                         int64_t num_slots, int64_t num_res, int batch, int kv_heads,
                         int head_dim, int asym, float eps, float qmax, float levels,
                         float offset, int recip, void* stream);

/* K quantizer of completed pages: data fp16 [n, 16, H_kv, 128]
 * (data_strides[3] = (block, token, head)) -> int8 codes into k_pool block
 * ids[n] (kv_strides[3]), step into k_scale [num_blocks, H_kv, 128]
 * (ks_strides[2] = (block, head)), zero point into k_zero (asym), one step per
 * (block, head, channel) over the 16 tokens.  ids int64; ids outside the
 * pool are skipped.  Replaces Int8PagedKVCache._finalize_blocks
 * (cache/int8_paged_cache.py:670-699). */
int ls_int8_finalize_blocks(const void* data, const int64_t* data_strides, const int64_t* ids,
                            int n, void* k_pool, const int64_t* kv_strides, float* k_scale,
                            float* k_zero, const int64_t* ks_strides, int64_t num_blocks,
                            int kv_heads, int head_dim, int page, int asym, float eps, float qmax,
                            float levels, float offset, int recip, void* stream);

/* Block-table gather (the paged cache's read path): out [B, length, H_kv,
 * head_dim] (out_strides[3] = (b, token, head)) gets, for token p of
 * sequence b, the pool row of flat slot table[b][p / 16] * 16 + p % 16 when
 * p < seq_lens[b], else flat slot 0 (the reference's zero-padded slot
 * table).  pool [num_blocks, 16, H_kv, head_dim] of elem_bytes-byte elements
 * (fp16 2, int8 1, fp32 4).  Bit-exact byte copy.  Replaces read()
 * (cache/paged_cache.py:486-506, slot table :305-323; slot rule
 * cache/block_allocator.py:214-220). */
int ls_paged_gather(const void* pool, int elem_bytes, const int64_t* kv_strides, int num_blocks,
                    const int32_t* block_tables, int64_t bt_stride, int max_pages,
                    const int32_t* seq_lens, void* out, const int64_t* out_strides, int batch,
                    int kv_heads, int head_dim, int page, int length, void* stream);

/* ---- fused elementwise ops of the decode step ----
 *
 * fp16 throughout, each product, sum and cast rounded to fp16 where Hugging
 * Face's Qwen2 computation rounds (kernels/fused_elementwise.py:75-110).
 * Row-major 2-D operands take a row stride in elements and unit inner
 * stride. */

/* y[r] = w * fp16(s * rsqrt(mean(s^2) + eps)) with s = x[r], or, when
 * residual is given, s = fp16(residual[r] + x[r]), also stored to res_out[r]
 * (residual and res_out both NULL or both given).  x, residual, y, res_out
 * [rows, n]; w [n].  Replaces rms_norm (kernels/fused_elementwise.py:194-205)
 * and fused_add_rms_norm (:207-220). */
int ls_rms_norm(const void* x, int64_t x_stride, const void* residual, int64_t res_stride,
                const void* weight, void* y, int64_t y_stride, void* res_out,
                int64_t res_out_stride, int rows, int n, float eps, void* stream);

/* out[r] = fp16(fp16(silu(g)) * u), g = gate_up[r, :inter], u = gate_up[r,
 * inter:2 inter].  Replaces silu_and_mul (kernels/fused_elementwise.py:222-233). */
int ls_silu_and_mul(const void* gate_up, int64_t gu_stride, void* out, int64_t out_stride,
                    int rows, int inter, void* stream);

/* RoPE (rotate-half pairing) on q [rows, hq * head_dim] and k [rows, hk *
 * head_dim] with fp16 cos / sin rows [rows, head_dim] (a table stride of 0
 * uses one row for all): out = fp16(fp16(x * cos) + fp16(rotate_half(x) *
 * sin)).  Replaces rope_qk (kernels/fused_elementwise.py:235-252). */
int ls_rope_qk(const void* q, int64_t q_stride, const void* k, int64_t k_stride, const void* cos,
               int64_t cos_stride, const void* sin, int64_t sin_stride, void* q_out,
               int64_t q_out_stride, void* k_out, int64_t k_out_stride, int rows, int hq, int hk,
               int head_dim, void* stream);

/* One decode token per sequence, straight from the fused q/k/v projection
 * output qkv [batch, (hq + 2 hk) * head_dim] (row stride qkv_stride): RoPE
 * as ls_rope_qk at position positions[b] (int64, clamped into the table of
 * table_rows rows of fp16 cos / sin, row stride table_stride); the rotated
 * query heads folded to q_out [batch, hk, hq / hk, head_dim] (q_strides[3] =
 * (b, kv head, row); query head i goes to kv head i / (hq / hk)); the
 * rotated key and the value stored at flat slot slots[b] (int64, = block *
 * page + offset; negative or past the pool: not stored) of k_pool / v_pool
 * [num_blocks, page, hk, head_dim] (kv_strides[3] = (block, token, head)).
 * With kmin / kmax [num_blocks, hk, head_dim] fp16 (bounds_strides[2] =
 * (block, head); both NULL to skip), the stored key also updates its page's
 * K bounds as ls_page_bounds_update does.  Replaces, in one launch, rope_qk
 * (model/attention/gqa.py:251-253), the paged store of the new rows
 * (cache/paged_cache.py write, bounds :457-460) and the fold of q to
 * [B, H_kv, n_rep, D] (model/attention/gqa.py:290-341). */
int ls_rope_write_decode(const void* qkv, int64_t qkv_stride, const int64_t* positions,
                         const void* cos, const void* sin, int64_t table_stride, int table_rows,
                         const int64_t* slots, void* k_pool, void* v_pool,
                         const int64_t* kv_strides, int num_blocks, int page, void* q_out,
                         const int64_t* q_strides, void* kmin, void* kmax,
                         const int64_t* bounds_strides, int batch, int hq, int hk, int head_dim,
                         void* stream);

/* The fused q/k/v projection of one decode token per sequence with its
 * finish in the epilogue: qkv = fp16(x[batch, K] . w^T + bias) for w
 * [(hq + 2 hk) * head_dim, K] (never stored), then exactly what
 * ls_rope_write_decode does with it (RoPE at positions[b], q folded to
 * q_out, the rotated key and the value stored at slots[b], the page K
 * bounds updated when kmin / kmax are given), bit-equal to ls_decode_gemm
 * followed by ls_rope_write_decode.  Same arguments as those two (x and w
 * as ls_decode_gemm: 16-byte aligned rows, K % 32 == 0, batch <= 64;
 * head_dim % 16 == 0); refused (LS_ERR_INVALID) for sizes at which the
 * GEMM would split K over workgroups.  Replaces the reference's qkv
 * projection + rope_qk + paged cache write of the decode layer
 * (model/attention/gqa.py:251-253, :283-344; cache/paged_cache.py). */
int ls_decode_qkv_rope_write(const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                             int w_packed, const void* bias, int K, const int64_t* positions,
                             const void* cos,
                             const void* sin, int64_t table_stride, int table_rows,
                             const int64_t* slots, void* k_pool, void* v_pool,
                             const int64_t* kv_strides, int num_blocks, int page, void* q_out,
                             const int64_t* q_strides, void* kmin, void* kmax,
                             const int64_t* bounds_strides, int batch, int hq, int hk,
                             int head_dim, const void* res, int64_t res_stride,
                             const void* norm_w, float eps, void* res_out,
                             int64_t res_out_stride, void* stream);

/* y[r] = ls_rms_norm of table row ids[r] (int64, clamped into [0,
 * table_rows)), and rows_out[r] = that table row (NULL to skip): the token
 * embedding lookup and the first layer's input norm in one launch
 * (rows_out is the residual the layer carries).  Replaces the reference's
 * embed_tokens lookup + input_layernorm (model/latentserve_qwen.py decode
 * loop; the norm as kernels/fused_elementwise.py:194-205). */
int ls_embed_rms_norm(const void* table, int64_t table_stride, int64_t table_rows,
                      const int64_t* ids, const void* weight, void* y, int64_t y_stride,
                      void* rows_out, int64_t rows_out_stride, int rows, int n, float eps,
                      void* stream);

/* out[r] = index of the largest value of fp16 row x[r, :n] (int64; the
 * first among equals, NaN above every number): torch.argmax over the last
 * dimension, the greedy choice of the next token from the logits.  Long
 * rows are split over workgroups, which need a device workspace of
 * ls_argmax_workspace_bytes(rows, n) bytes (0: none; else 16-byte aligned,
 * zero-filled before its first use: its counters are left at zero by each
 * call; calls sharing it are ordered on one stream).  Replaces
 * logits.argmax(dim=-1) of the reference's greedy decode loop. */
size_t ls_argmax_workspace_bytes(int rows, int n);
int ls_argmax_rows(const void* x, int64_t x_stride, int64_t* out, int rows, int n,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Weights of the decode GEMMs packed for their launches: the 16-row tiles
 * of the entry point's row order (kind 0: ls_decode_gemm, 1:
 * ls_decode_gate_up_silu, w = [gate; up]; 2: ls_decode_qkv_rope_write,
 * head_dim used), each 32-channel step of a tile 1 KiB in the order the
 * lanes load it, tiles padded with zero rows.  Every weight load of a
 * packed launch then reads 1 KiB contiguous (a row-major weight gives 64
 * bytes of each of 16 rows).  `packed` holds ls_gemm_packed_bytes(N, K,
 * kind, head_dim) bytes, 16-byte aligned; pass it as `w` with w_packed = 1
 * (w_stride ignored) to the entry point of its kind.  No counterpart in
 * the reference (its weights stay torch Linear tensors). */
size_t ls_gemm_packed_bytes(int N, int K, int kind, int head_dim);
int ls_pack_gemm_weight(const void* w, int64_t w_stride, int N, int K, int kind, int head_dim,
                        void* packed, void* stream);

/* The norm prologue of the three decode GEMMs below (ls_decode_gemm,
 * ls_decode_gate_up_silu, ls_decode_qkv_rope_write): with norm_w non-NULL
 * the product's left operand is not x but ls_rms_norm(x + res) (fp16 rows,
 * weight norm_w [K], eps; the decoder layer's residual add and RMSNorm),
 * and res_out receives x + res, as ls_rms_norm with a residual does; the
 * sum of squares is taken in another order, so the normalised row may
 * differ from ls_rms_norm's in the last fp16 bit.  Needs a packed weight,
 * M <= 16 and a width at which K is not split over workgroups
 * (ls_decode_gemm_workspace_bytes == 0); res, res_out (row strides
 * res_stride, res_out_stride) and norm_w 16-byte aligned; res_out may not
 * overlap x or res.  norm_w NULL: x is the operand and res, res_out are
 * ignored.  Replaces the post_attention_layernorm / input_layernorm / final
 * norm launch before each projection (kernels/fused_elementwise.py:194-205,
 * model/latentserve_qwen.py:425-450). */

/* y[M, N] = x[M, K] . w[N, K]^T (+ bias[N]) in fp16 with fp32 sums: the
 * projections of a decode step (torch Linear weight layout), M <= 64 rows.
 * Rows of x, w and y are strided (x_stride, w_stride, y_stride elements);
 * K % 32 == 0 and x, w 16-byte aligned with strides that keep every row so
 * (y is stored 8 bytes at a time when its alignment allows).  Each output is rounded to fp16
 * once, after the bias add (after the sum of the partials where K is split
 * over workgroups: the last workgroup of a tile to finish adds them in split
 * order).  Replaces the torch Linear calls of the
 * reference's decoder layers (model/latentserve_qwen.py, model/fused.py),
 * which run as cuBLAS GEMMs. */
int ls_decode_gemm(const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                   int w_packed, const void* bias, void* y, int64_t y_stride, int M, int N, int K,
                   void* workspace, size_t workspace_bytes, const void* res, int64_t res_stride,
                   const void* norm_w, float eps, void* res_out, int64_t res_out_stride,
                   void* stream);

/* Bytes of device `workspace` ls_decode_gemm needs for these sizes: fp32
 * partial sums and arrival counters when K is split over workgroups (narrow
 * outputs with long K), 0 otherwise (workspace may then be NULL).  The
 * workspace is 256-byte aligned and zero-filled before its first use; its
 * first 64 KiB hold the counters, which each call leaves at zero again.  Calls that share a workspace
 * must be ordered on one stream.  No counterpart in the reference (a cuBLAS
 * call sizes its own). */
size_t ls_decode_gemm_workspace_bytes(int M, int N, int K);

/* y[M, inter] = fp16(fp16(silu(g)) * u) with g = fp16(x . w[:inter]^T +
 * bias[:inter]) and u = fp16(x . w[inter:]^T + bias[inter:]): the MLP's
 * gate/up projection (w [2 inter, K], gate rows first) with the activation
 * in its epilogue, bit-equal to ls_decode_gemm followed by ls_silu_and_mul.
 * Same operand rules as ls_decode_gemm; refused (LS_ERR_INVALID) for sizes
 * at which ls_decode_gemm would split K over workgroups
 * (ls_decode_gemm_workspace_bytes(M, 2 inter, K) != 0).  Replaces the
 * reference's gate_up projection + silu_and_mul
 * (kernels/fused_elementwise.py:222-233, model/fused.py). */
int ls_decode_gate_up_silu(const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                           int w_packed, const void* bias, void* y, int64_t y_stride, int M,
                           int inter, int K, const void* res, int64_t res_stride,
                           const void* norm_w, float eps, void* res_out, int64_t res_out_stride,
                           void* stream);


#ifdef __cplusplus
}
#endif

#endif /* LATENTSERVE_AMD_H */
