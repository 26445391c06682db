// C ABI of liblatentserve_hip.so: argument checks, then one launch on the
// caller's stream.  Declared in include/latentserve_amd.h.
//
// The checks are what the reference's eligible() / paged_decode_cuda() raise
// on (kernels/cuda/paged_decode_cuda.py:105-141, 214-217), plus what a
// gfx950 launch must not violate: 16-byte vector loads need 16-byte aligned
// rows, the lane mapping needs head_dim 128 and 16-token pages, and the grid's
// y dimension is the batch.

#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <string>

#include "../../include/latentserve_amd.h"
#include "ls_common.h"
#include "ls_decode.h"
#include "ls_sparse.h"
#include "ls_int8_write.h"
#include "ls_gather.h"
#include "ls_elementwise.h"
#include "ls_gemm.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(LS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return LS_OK;
}

bool aligned(const void* p, size_t n) { return ((uintptr_t)p % n) == 0; }

// Base pointer and every listed stride (in elements of `elem` bytes) must be
// `n`-byte aligned for the kernels' vector loads.
bool rows_aligned(const void* p, const int64_t* st, int count, size_t elem, size_t n) {
    if (!aligned(p, n)) return false;
    for (int i = 0; i < count; ++i)
        if ((st[i] * (int64_t)elem) % (int64_t)n != 0) return false;
    return true;
}

int check_common(const void* q, const int64_t* q_strides, const void* k_pool, const void* v_pool,
                 const int64_t* kv_strides, int num_blocks, const int32_t* block_tables,
                 int max_pages, const int32_t* seq_lens, void* out, const int64_t* out_strides,
                 float* workspace, int32_t* counters, int batch,
                 int kv_heads, int n_rep, int head_dim, int page, int num_splits, size_t kv_elem) {
    if (!q || !q_strides || !k_pool || !v_pool || !kv_strides || !block_tables || !seq_lens ||
        !out || !out_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (page != ls::PAGE) return fail(LS_ERR_INVALID, "page (block_size) must be 16, got %d", page);
    if (n_rep < 1 || n_rep > ls::MAX_NREP)
        return fail(LS_ERR_INVALID, "n_rep must be in [1, 16], got %d", n_rep);
    if (batch < 0 || batch > 65535) return fail(LS_ERR_INVALID, "batch must be in [0, 65535], got %d", batch);
    if (kv_heads < 1) return fail(LS_ERR_INVALID, "kv_heads must be >= 1, got %d", kv_heads);
    if (num_splits < 1 || (int64_t)num_splits * kv_heads > (1LL << 31) - 1)
        return fail(LS_ERR_INVALID, "num_splits must be >= 1, got %d", num_splits);
    if (num_blocks < 1) return fail(LS_ERR_INVALID, "num_blocks must be >= 1");
    if (max_pages < 1) return fail(LS_ERR_INVALID, "max_pages (block-table width) must be >= 1");
    if (max_pages > (1 << 24))
        return fail(LS_ERR_INVALID, "max_pages (block-table width) must be <= 2^24");
    if (!rows_aligned(q, q_strides, 3, 2, 16))
        return fail(LS_ERR_INVALID, "q rows must be 16-byte aligned");
    if (!rows_aligned(k_pool, kv_strides, 3, kv_elem, kv_elem == 2 ? 16 : 8) ||
        !rows_aligned(v_pool, kv_strides, 3, kv_elem, kv_elem == 2 ? 16 : 8))
        return fail(LS_ERR_INVALID, "K/V pool rows must be %d-byte aligned", kv_elem == 2 ? 16 : 8);
    if (!aligned(out, 2)) return fail(LS_ERR_INVALID, "out must be 2-byte aligned");
    if (!counters) return fail(LS_ERR_INVALID, "counters is required");
    if (num_splits > 1 && !workspace)
        return fail(LS_ERR_INVALID, "num_splits > 1 needs workspace");
    if (num_splits > 1 && !aligned(workspace, 256))
        return fail(LS_ERR_INVALID, "workspace must be 256-byte aligned");
    (void)out_strides;
    return LS_OK;
}

void fill_common(ls::DecodeParams& a, const void* q, const int64_t* q_strides, const void* k_pool,
                 const void* v_pool, const int64_t* kv_strides, int num_blocks,
                 const int32_t* block_tables, int64_t bt_stride, int max_pages,
                 const int32_t* seq_lens, void* out, const int64_t* out_strides, float* workspace,
                 int32_t* counters, int batch, int kv_heads,
                 int n_rep, int num_splits, int max_seq_len, float softmax_scale) {
    memset(&a, 0, sizeof a);
    a.q = (const _Float16*)q;
    a.sq_b = q_strides[0];
    a.sq_h = q_strides[1];
    a.sq_r = q_strides[2];
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.sk_b = kv_strides[0];
    a.sk_p = kv_strides[1];
    a.sk_h = kv_strides[2];
    a.block_tables = block_tables;
    a.sbt_b = bt_stride;
    a.max_pages = max_pages;
    a.num_blocks = num_blocks;
    a.seq_lens = seq_lens;
    a.work = workspace;
    if (max_seq_len > 0) {
        int pages = (max_seq_len + ls::PAGE - 1) / ls::PAGE;
        pages = pages < max_pages ? pages : max_pages;
        a.pages_per_split = (pages + num_splits - 1) / num_splits;
    }
    a.counters = counters;
    a.out = (_Float16*)out;
    a.so_b = out_strides[0];
    a.so_h = out_strides[1];
    a.so_r = out_strides[2];
    a.B = batch;
    a.H = kv_heads;
    a.NR = n_rep;
    a.num_splits = num_splits;
    a.scale = softmax_scale;
}

int make_rope_params(ls::RopeWriteParams& a, const void* qkv, int64_t qkv_stride,
                     const int64_t* positions, const void* cos, const void* sin,
                     int64_t table_stride, int table_rows, const int64_t* slots, void* k_pool,
                     void* v_pool, const int64_t* kv_strides, int num_blocks, int page,
                     void* q_out, const int64_t* q_strides, void* kmin, void* kmax,
                     const int64_t* bounds_strides, int batch, int hq, int hk, int head_dim) {
    if (!qkv || !positions || !cos || !sin || !slots || !k_pool || !v_pool || !kv_strides ||
        !q_out || !q_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim < 2 || head_dim > 1024 || head_dim % 2 != 0)
        return fail(LS_ERR_INVALID, "head_dim must be even and in [2, 1024], got %d", head_dim);
    if (hk < 1 || hq < 1 || hq % hk != 0 || hq + 2 * hk > 65535)
        return fail(LS_ERR_INVALID, "hq must be a positive multiple of hk (hq %d, hk %d)", hq, hk);
    if (batch < 0 || batch > 65535) return fail(LS_ERR_INVALID, "batch must be in [0, 65535]");
    if (table_rows < 1 || num_blocks < 1 || page < 1)
        return fail(LS_ERR_INVALID, "table_rows, num_blocks and page must be >= 1");
    if ((kmin == nullptr) != (kmax == nullptr) || (kmin && !bounds_strides))
        return fail(LS_ERR_INVALID, "kmin, kmax and bounds_strides must be given together");
    a.qkv = qkv;
    a.sqkv = qkv_stride;
    a.pos = positions;
    a.cos = cos;
    a.sin = sin;
    a.st = table_stride;
    a.tab_rows = table_rows;
    a.slots = slots;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.sp_b = kv_strides[0];
    a.sp_t = kv_strides[1];
    a.sp_h = kv_strides[2];
    a.num_blocks = num_blocks;
    a.page = page;
    a.q_out = q_out;
    a.sq_b = q_strides[0];
    a.sq_h = q_strides[1];
    a.sq_r = q_strides[2];
    a.kmin = kmin;
    a.kmax = kmax;
    a.sb_b = kmin ? bounds_strides[0] : 0;
    a.sb_h = kmin ? bounds_strides[1] : 0;
    a.B = batch;
    a.hq = hq;
    a.hk = hk;
    a.d = head_dim;
    return LS_OK;
}

// x rows 16-byte aligned holding K values; w the same, or packed (its
// layout holds every row; only its base alignment matters).
bool weight_ok(const void* x, int64_t x_stride, const void* w, int64_t w_stride, int w_packed,
               int K) {
    if (!aligned(x, 16) || x_stride % 8 != 0 || x_stride < K || !aligned(w, 16)) return false;
    return w_packed || (w_stride % 8 == 0 && w_stride >= K);
}


// The norm prologue of a decode GEMM (norm_w non-null): x is replaced by
// rms_norm(x + res) with weight norm_w, and x + res stored to res_out.
// Needs a packed weight, M <= 16 and K not split over workgroups; res_out
// is written while other workgroups read x and res, so it may alias
// neither.
int set_norm(ls::GemmParams& a, const void* res, int64_t res_stride, const void* norm_w,
             float eps, void* res_out, int64_t res_out_stride, const char* what) {
    if (!norm_w) return LS_OK;
    if (!res || !res_out) return fail(LS_ERR_INVALID, "%s: the norm needs res and res_out", what);
    if (!a.w_packed || a.M > 16)
        return fail(LS_ERR_INVALID, "%s: the norm prologue needs a packed weight and M <= 16",
                    what);
    if (!aligned(res, 16) || !aligned(res_out, 16) || !aligned(norm_w, 16) ||
        res_stride % 8 != 0 || res_out_stride % 8 != 0 ||
        (a.M > 1 && (res_stride < a.K || res_out_stride < a.K)))
        return fail(LS_ERR_INVALID,
                    "%s: res, res_out and norm_w must be 16-byte aligned rows of K values", what);
    const char* ro = (const char*)res_out;
    const int64_t span = ((int64_t)(a.M - 1) * res_out_stride + a.K) * 2;
    auto overlaps = [&](const void* p, int64_t stride) {
        const char* q = (const char*)p;
        const int64_t qspan = ((int64_t)(a.M - 1) * stride + a.K) * 2;
        return q < ro + span && ro < q + qspan;
    };
    if (overlaps(res, res_stride) || overlaps(a.x, a.ldx))
        return fail(LS_ERR_INVALID, "%s: res_out may not overlap x or res", what);
    if (a.M > 0 && a.N > 0 && ls::decode_gemm_splits(a.M, a.N, a.K) != 1)
        return fail(LS_ERR_INVALID, "%s: K %d is too long for the norm prologue", what, a.K);
    a.norm = 1;
    a.nres = res;
    a.ldr = res_stride;
    a.nw = norm_w;
    a.nres_out = res_out;
    a.ldro = res_out_stride;
    a.eps = eps;
    return LS_OK;
}

}  // namespace

extern "C" {

const char* ls_last_error(void) { return g_err.c_str(); }

int ls_abi_version(void) { return 19; }

int ls_kernel_resources(const char* kernel, int kv_heads, int n_rep, int asym, int has_res,
                        LsKernelResources* out) {
    if (!kernel || !out) return fail(LS_ERR_INVALID, "null pointer argument");
    if (kv_heads < 1 || n_rep < 1 || n_rep > ls::MAX_NREP)
        return fail(LS_ERR_INVALID, "bad kv_heads (%d) or n_rep (%d)", kv_heads, n_rep);
    const std::string k = kernel;
    const bool pair = kv_heads % 2 == 0;
    ls::KernelResources r{};
    hipError_t e;
    if (k == "paged_decode_fp16") e = ls::decode_resources(ls::KV_FP16, 0, false, false, pair, &r);
    else if (k == "paged_decode_int8") e = ls::decode_resources(ls::KV_INT8, 0, asym, has_res, pair, &r);
    else if (k == "paged_sparse_fp16") e = ls::decode_resources(ls::KV_FP16, 1, false, false, pair, &r);
    else if (k == "sparse_attention_fp16") e = ls::decode_resources(ls::KV_FP16, 2, false, false, pair, &r);
    else if (k == "sparse_attention_bounds_fp16") e = ls::decode_resources(ls::KV_FP16, 3, false, false, pair, &r);
    else if (k == "combine_splits") e = ls::combine_resources(&r);
    else if (k == "page_index") e = ls::sparse_index_resources(0, n_rep, &r);
    else if (k == "page_index_heads") e = ls::sparse_index_resources(1, n_rep, &r);
    else if (k == "page_mass") e = ls::sparse_index_resources(2, n_rep, &r);
    else if (k == "page_select") e = ls::sparse_index_resources(3, n_rep, &r);
    else if (k == "page_bounds_update") e = ls::sparse_index_resources(4, n_rep, &r);
    else if (k == "page_bounds_rebuild") e = ls::sparse_index_resources(5, n_rep, &r);
    else if (k == "int8_decode_write") e = ls::int8_write_resources(0, &r);
    else if (k == "int8_finalize_blocks") e = ls::int8_write_resources(1, &r);
    else return fail(LS_ERR_INVALID, "unknown kernel '%s'", kernel);
    if (e != hipSuccess) return hip_status(e, "ls_kernel_resources");
    out->regs = r.regs;
    out->local_bytes = r.local_bytes;
    out->shared_bytes = r.shared_bytes;
    out->threads = r.threads;
    out->groups_per_cu = r.groups_per_cu;
    return LS_OK;
}

// The bound on the one-launch bounds path's wait for the other workgroups'
// scores (ls_set_coop_wait_ticks).
static std::atomic<uint64_t> g_coop_wait_ticks{ls::COOP_WAIT_TICKS};

int ls_set_coop_wait_ticks(uint64_t ticks) {
    g_coop_wait_ticks.store(ticks, std::memory_order_relaxed);
    return LS_OK;
}

size_t ls_decode_counter_ints(int batch, int kv_heads) {
    if (batch <= 0 || kv_heads <= 0) return 0;
    return (size_t)batch * (size_t)kv_heads * ls::COUNTER_STRIDE;
}

size_t ls_decode_workspace_bytes(int batch, int kv_heads, int n_rep, int num_splits) {
    if (batch <= 0 || kv_heads <= 0 || n_rep <= 0 || num_splits <= 1) return 0;
    const size_t rec = (size_t)n_rep * ls::HEAD_DIM + 2 * ls::MAX_NREP;
    return (size_t)batch * kv_heads * num_splits * rec * sizeof(float);
}

int ls_paged_decode_fp16(const void* q, const int64_t* q_strides, const void* k_pool,
                         const void* v_pool, const int64_t* kv_strides, int num_blocks,
                         const int32_t* block_tables, int64_t bt_stride, int max_pages,
                         const int32_t* seq_lens, void* out, const int64_t* out_strides,
                         float* workspace, int32_t* counters,
                         int batch, int kv_heads, int n_rep, int head_dim, int page,
                         int num_splits, int max_seq_len, float softmax_scale, void* stream) {
    int rc = check_common(q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables,
                          max_pages, seq_lens, out, out_strides, workspace,
                          counters, batch, kv_heads, n_rep, head_dim, page, num_splits, 2);
    if (rc) return rc;
    if (batch == 0) return LS_OK;
    ls::DecodeParams a;
    fill_common(a, q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables, bt_stride,
                max_pages, seq_lens, out, out_strides, workspace, counters, batch,
                kv_heads, n_rep, num_splits, max_seq_len, softmax_scale);
    a.kind = ls::KV_FP16;
    return hip_status(ls::launch_decode(a, (hipStream_t)stream), "ls_paged_decode_fp16");
}

int ls_paged_decode_fp16_noalloc(const void* q, const int64_t* q_strides, const void* k_pool,
                                 const void* v_pool, const int64_t* kv_strides, int num_blocks,
                                 const int32_t* block_tables, int64_t bt_stride, int max_pages,
                                 const int32_t* seq_lens, void* out, const int64_t* out_strides,
                                 int batch, int kv_heads, int n_rep, int head_dim, int page,
                                 int num_splits, int max_seq_len, float softmax_scale,
                                 void* stream) {
    if (batch > 0 && kv_heads > 0 &&
        (int64_t)batch * kv_heads > ls::NOALLOC_COUNTERS / ls::COUNTER_STRIDE)
        return fail(LS_ERR_INVALID,
                    "ls_paged_decode_fp16_noalloc: batch * kv_heads = %lld exceeds the fixed "
                    "scratch's %d arrival counters",
                    (long long)batch * kv_heads, ls::NOALLOC_COUNTERS / ls::COUNTER_STRIDE);
    const size_t need = ls_decode_workspace_bytes(batch, kv_heads, n_rep, num_splits);
    if (need > ls::NOALLOC_WORK_BYTES)
        return fail(LS_ERR_INVALID,
                    "ls_paged_decode_fp16_noalloc: %zu bytes of split records (batch %d, "
                    "kv_heads %d, n_rep %d, num_splits %d) exceed the fixed scratch's %zu; use "
                    "fewer splits or ls_paged_decode_fp16 with a workspace",
                    need, batch, kv_heads, n_rep, num_splits, ls::NOALLOC_WORK_BYTES);
    float* work = nullptr;
    int32_t* counters = nullptr;
    if (int rc = hip_status(ls::noalloc_scratch((hipStream_t)stream, &work, &counters),
                            "ls_paged_decode_fp16_noalloc (scratch set-up)"))
        return rc;
    return ls_paged_decode_fp16(q, q_strides, k_pool, v_pool, kv_strides, num_blocks,
                                block_tables, bt_stride, max_pages, seq_lens, out, out_strides,
                                work, counters, batch, kv_heads, n_rep, head_dim, page,
                                num_splits, max_seq_len, softmax_scale, stream);
}

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
                         void* stream) {
    int rc = check_common(q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables,
                          max_pages, seq_lens, out, out_strides, workspace,
                          counters, batch, kv_heads, n_rep, head_dim, page, num_splits, 1);
    if (rc) return rc;
    if (!k_scale || !ks_strides || !v_scale || !vs_strides)
        return fail(LS_ERR_INVALID, "INT8 pools need k_scale and v_scale");
    if (!rows_aligned(k_scale, ks_strides, 2, 4, 16))
        return fail(LS_ERR_INVALID, "k_scale rows must be 16-byte aligned");
    if (!aligned(v_scale, 4)) return fail(LS_ERR_INVALID, "v_scale must be 4-byte aligned");
    if ((k_zero == nullptr) != (v_zero == nullptr))
        return fail(LS_ERR_INVALID, "k_zero and v_zero go together");
    if (k_zero && !aligned(k_zero, 16))
        return fail(LS_ERR_INVALID, "k_zero must be 16-byte aligned");
    if (v_zero && !aligned(v_zero, 4)) return fail(LS_ERR_INVALID, "v_zero must be 4-byte aligned");
    if ((k_residual == nullptr) != (res_rows == nullptr))
        return fail(LS_ERR_INVALID, "k_residual and res_rows go together");
    if (k_residual) {
        if (!res_strides) return fail(LS_ERR_INVALID, "k_residual needs res_strides");
        if (!rows_aligned(k_residual, res_strides, 3, 2, 16))
            return fail(LS_ERR_INVALID, "k_residual rows must be 16-byte aligned");
        if (res_capacity < 1) return fail(LS_ERR_INVALID, "res_capacity must be >= 1");
    }
    if (batch == 0) return LS_OK;
    ls::DecodeParams a;
    fill_common(a, q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables, bt_stride,
                max_pages, seq_lens, out, out_strides, workspace, counters, batch,
                kv_heads, n_rep, num_splits, max_seq_len, softmax_scale);
    a.kind = ls::KV_INT8;
    a.k_scale = k_scale;
    a.sks_b = ks_strides[0];
    a.sks_h = ks_strides[1];
    a.v_scale = v_scale;
    a.svs_b = vs_strides[0];
    a.svs_p = vs_strides[1];
    a.svs_h = vs_strides[2];
    a.k_zero = k_zero;
    a.v_zero = v_zero;
    a.k_res = (const _Float16*)k_residual;
    if (k_residual) {
        a.sr_r = res_strides[0];
        a.sr_p = res_strides[1];
        a.sr_h = res_strides[2];
        a.res_cap = res_capacity;
        a.res_rows = res_rows;
    }
    return hip_status(ls::launch_decode(a, (hipStream_t)stream), "ls_paged_decode_int8");
}

int ls_paged_sparse_fp16(const void* q, const int64_t* q_strides, const void* k_pool,
                         const void* v_pool, const int64_t* kv_strides, int num_blocks,
                         const int32_t* block_tables, int64_t bt_stride, int max_pages,
                         const int32_t* seq_lens, const int32_t* sel, const int64_t* sel_strides,
                         int num_sel, float ratio, int recent, void* out,
                         const int64_t* out_strides, float* workspace,
                         int32_t* counters, int batch, int kv_heads, int n_rep,
                         int head_dim, int page, int num_splits, int max_seq_len, float softmax_scale,
                         void* stream) {
    int rc = check_common(q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables,
                          max_pages, seq_lens, out, out_strides, workspace,
                          counters, batch, kv_heads, n_rep, head_dim, page, num_splits, 2);
    if (rc) return rc;
    if (!sel || !sel_strides) return fail(LS_ERR_INVALID, "sparse decode needs sel");
    if (num_sel < 0) return fail(LS_ERR_INVALID, "num_sel must be >= 0");
    if (batch == 0) return LS_OK;
    ls::DecodeParams a;
    fill_common(a, q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables, bt_stride,
                max_pages, seq_lens, out, out_strides, workspace, counters, batch,
                kv_heads, n_rep, num_splits, max_seq_len, softmax_scale);
    a.kind = ls::KV_FP16;
    a.sel = sel;
    a.ssel_b = sel_strides[0];
    a.ssel_h = sel_strides[1];
    a.num_sel = num_sel;
    a.ratio = ratio;
    a.recent = recent;
    return hip_status(ls::launch_decode(a, (hipStream_t)stream), "ls_paged_sparse_fp16");
}

int ls_sparse_attention_fp16(const void* q, const int64_t* q_strides, const void* k_pool,
                             const void* v_pool, const int64_t* kv_strides, int num_blocks,
                             const int32_t* block_tables, int64_t bt_stride, int max_pages,
                             const int32_t* seq_lens, const float* scores,
                             const int64_t* score_strides, int score_pages, int k, float ratio,
                             int recent, void* out, const int64_t* out_strides, float* workspace,
                             int32_t* counters, int batch, int kv_heads, int n_rep,
                             int head_dim, int page, int num_splits, int max_seq_len,
                             float softmax_scale, void* stream) {
    int rc = check_common(q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables,
                          max_pages, seq_lens, out, out_strides, workspace,
                          counters, batch, kv_heads, n_rep, head_dim, page, num_splits, 2);
    if (rc) return rc;
    if (!scores || !score_strides) return fail(LS_ERR_INVALID, "needs page scores");
    if (score_pages < 1 || score_pages > ls::SELECT_MAX_PAGES)
        return fail(LS_ERR_INVALID, "score_pages must be in [1, %d], got %d",
                    ls::SELECT_MAX_PAGES, score_pages);
    if (k < 0 || k > score_pages)
        return fail(LS_ERR_INVALID, "k must be in [0, score_pages], got %d", k);
    // every split's share of a list must fit the group's item table
    if ((k + num_splits - 1) / num_splits > ls::SELECT_SPLIT_ENTRIES)
        return fail(LS_ERR_INVALID,
                    "k / num_splits must be at most %d (k %d, num_splits %d): use more splits",
                    ls::SELECT_SPLIT_ENTRIES, k, num_splits);
    if (batch == 0) return LS_OK;
    ls::DecodeParams a;
    fill_common(a, q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables, bt_stride,
                max_pages, seq_lens, out, out_strides, workspace, counters, batch,
                kv_heads, n_rep, num_splits, max_seq_len, softmax_scale);
    a.kind = ls::KV_FP16;
    a.scores = const_cast<float*>(scores);
    a.ssc_b = score_strides[0];
    a.ssc_h = score_strides[1];
    a.score_pages = score_pages;
    a.num_sel = k;
    a.ratio = ratio;
    a.recent = recent;
    return hip_status(ls::launch_decode(a, (hipStream_t)stream), "ls_sparse_attention_fp16");
}

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
                                    float softmax_scale, void* stream) {
    if (!kmin || !kmax || !bound_strides) return fail(LS_ERR_INVALID, "needs kmin, kmax");
    if (!rows_aligned(kmin, bound_strides, 2, 2, 16) || !rows_aligned(kmax, bound_strides, 2, 2, 16))
        return fail(LS_ERR_INVALID, "kmin/kmax rows must be 16-byte aligned");
    if (recent < 0) return fail(LS_ERR_INVALID, "recent must be >= 0");
    if (!aligned(scores, 4)) return fail(LS_ERR_INVALID, "scores must be 4-byte aligned");
    int rc = check_common(q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables,
                          max_pages, seq_lens, out, out_strides, workspace,
                          counters, batch, kv_heads, n_rep, head_dim, page, num_splits, 2);
    if (rc) return rc;
    if (!scores || !score_strides) return fail(LS_ERR_INVALID, "needs the score buffer");
    if (score_strides[1] < (int64_t)max_pages + 1 || score_strides[0] < kv_heads * score_strides[1])
        return fail(LS_ERR_INVALID, "score rows need max_pages + 1 words (a count after each)");
    if (max_pages > ls::COOP_MAX_PAGES)
        return fail(LS_ERR_INVALID, "max_pages must be at most %d, got %d",
                    ls::COOP_MAX_PAGES, max_pages);
    if (n_rep > ls::COOP_MAX_NREP)
        return fail(LS_ERR_INVALID, "n_rep must be at most %d, got %d", ls::COOP_MAX_NREP, n_rep);
    if (k < 0 || k > max_pages)
        return fail(LS_ERR_INVALID, "k must be in [0, max_pages], got %d", k);
    if ((k + num_splits - 1) / num_splits > ls::SELECT_SPLIT_ENTRIES)
        return fail(LS_ERR_INVALID,
                    "k / num_splits must be at most %d (k %d, num_splits %d): use more splits",
                    ls::SELECT_SPLIT_ENTRIES, k, num_splits);
    if (batch == 0) return LS_OK;
    ls::DecodeParams a;
    fill_common(a, q, q_strides, k_pool, v_pool, kv_strides, num_blocks, block_tables, bt_stride,
                max_pages, seq_lens, out, out_strides, workspace, counters, batch,
                kv_heads, n_rep, num_splits, max_seq_len, softmax_scale);
    a.kind = ls::KV_FP16;
    a.scores = scores;
    a.ssc_b = score_strides[0];
    a.ssc_h = score_strides[1];
    a.score_pages = max_pages;
    a.kmin = kmin;
    a.kmax = kmax;
    a.sb_b = bound_strides[0];
    a.sb_h = bound_strides[1];
    a.coop_wait_ticks = g_coop_wait_ticks.load(std::memory_order_relaxed);
    a.num_sel = k;
    a.ratio = ratio;
    a.recent = recent;
    return hip_status(ls::launch_decode(a, (hipStream_t)stream),
                      "ls_sparse_attention_bounds_fp16");
}

int ls_combine_splits(const float* part_acc, const int64_t* acc_strides, const float* part_m,
                      const float* part_l, const int64_t* ml_strides, void* out, int out_fp32,
                      const int64_t* out_strides, int batch, int kv_heads, int num_splits,
                      int n_rep, int head_dim, void* stream) {
    if (!part_acc || !acc_strides || !part_m || !part_l || !ml_strides || !out || !out_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (n_rep < 1 || num_splits < 1 || kv_heads < 1 || batch < 0)
        return fail(LS_ERR_INVALID, "bad combine shape");
    if ((int64_t)batch * kv_heads > (1LL << 31) - 1) return fail(LS_ERR_INVALID, "grid too large");
    if (batch == 0) return LS_OK;
    ls::CombineParams p;
    p.acc = part_acc;
    p.sa_b = acc_strides[0];
    p.sa_h = acc_strides[1];
    p.sa_s = acc_strides[2];
    p.sa_r = acc_strides[3];
    p.m = part_m;
    p.l = part_l;
    p.sm_b = ml_strides[0];
    p.sm_h = ml_strides[1];
    p.sm_s = ml_strides[2];
    p.out = out;
    p.out_f32 = out_fp32 ? 1 : 0;
    p.so_b = out_strides[0];
    p.so_h = out_strides[1];
    p.so_r = out_strides[2];
    p.B = batch;
    p.H = kv_heads;
    p.S = num_splits;
    p.NR = n_rep;
    return hip_status(ls::launch_combine(p, (hipStream_t)stream), "ls_combine_splits");
}

int ls_page_scores(const void* q, const int64_t* q_strides, const void* kmin, const void* kmax,
                   const int64_t* bound_strides, int num_blocks, const int32_t* block_tables,
                   int64_t bt_stride, int max_pages, const int32_t* seq_lens, float* scores,
                   const int64_t* score_strides, int batch, int kv_heads, int n_rep, int head_dim,
                   int page, int recent, void* stream) {
    return ls_sparse_index(q, q_strides, kmin, kmax, bound_strides, num_blocks, block_tables,
                           bt_stride, max_pages, seq_lens, scores, score_strides, nullptr, 0,
                           0.f, recent, nullptr, nullptr, batch, kv_heads, n_rep, head_dim, page,
                           stream);
}

size_t ls_page_mass_workspace_bytes(int batch, int kv_heads, int n_rep, int max_pages) {
    if (batch <= 0 || kv_heads <= 0 || n_rep <= 0 || max_pages <= 0) return 0;
    return (size_t)batch * kv_heads * n_rep * max_pages * sizeof(float);
}

int ls_page_scores_mass(const void* q, const int64_t* q_strides, const void* kmin,
                        const void* kmax, const int64_t* bound_strides, int num_blocks,
                        const int32_t* block_tables, int64_t bt_stride, int max_pages,
                        const int32_t* seq_lens, float* workspace, float* scores,
                        const int64_t* score_strides, int batch, int kv_heads, int n_rep,
                        int head_dim, int page, int recent, float softmax_scale,
                        void* stream) {
    if (!q || !q_strides || !kmin || !kmax || !bound_strides || !block_tables || !seq_lens ||
        !scores || !score_strides || !workspace)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (page != ls::PAGE) return fail(LS_ERR_INVALID, "page (block_size) must be 16, got %d", page);
    if (n_rep < 1 || n_rep > ls::MAX_NREP)
        return fail(LS_ERR_INVALID, "n_rep must be in [1, %d], got %d", ls::MAX_NREP, n_rep);
    if (batch < 0 || batch > 65535 || kv_heads < 1 || kv_heads > 65535)
        return fail(LS_ERR_INVALID, "bad batch (%d) or kv_heads (%d)", batch, kv_heads);
    if (num_blocks < 0 || max_pages < 0 || recent < 0)
        return fail(LS_ERR_INVALID, "bad num_blocks, max_pages or recent");
    if (!rows_aligned(q, q_strides, 3, 2, 16))
        return fail(LS_ERR_INVALID, "q rows must be 16-byte aligned");
    if (!rows_aligned(kmin, bound_strides, 2, 2, 16) || !rows_aligned(kmax, bound_strides, 2, 2, 16))
        return fail(LS_ERR_INVALID, "kmin/kmax rows must be 16-byte aligned");
    if (!aligned(scores, 4) || !aligned(workspace, 4))
        return fail(LS_ERR_INVALID, "scores and workspace must be 4-byte aligned");
    if (batch == 0 || max_pages == 0) return LS_OK;
    ls::IndexParams a{};
    a.q = q;
    a.sq_b = q_strides[0];
    a.sq_h = q_strides[1];
    a.sq_r = q_strides[2];
    a.kmin = kmin;
    a.kmax = kmax;
    a.sb_b = bound_strides[0];
    a.sb_h = bound_strides[1];
    a.num_blocks = num_blocks;
    a.block_tables = block_tables;
    a.sbt_b = bt_stride;
    a.max_pages = max_pages;
    a.seq_lens = seq_lens;
    a.scores = const_cast<float*>(scores);
    a.ss_b = score_strides[0];
    a.ss_h = score_strides[1];
    a.B = batch;
    a.H = kv_heads;
    a.NR = n_rep;
    a.recent = recent;
    a.heads = workspace;                  // [B, H, NR, max_pages], contiguous
    a.sh_r = max_pages;
    a.sh_h = (int64_t)n_rep * max_pages;
    a.sh_b = (int64_t)kv_heads * a.sh_h;
    a.scale_log2 = softmax_scale * 1.4426950408889634f;
    return hip_status(ls::launch_page_mass(a, (hipStream_t)stream), "ls_page_scores_mass");
}

int ls_sparse_index(const void* q, const int64_t* q_strides, const void* kmin, const void* kmax,
                    const int64_t* bound_strides, int num_blocks, const int32_t* block_tables,
                    int64_t bt_stride, int max_pages, const int32_t* seq_lens, float* scores,
                    const int64_t* score_strides, int32_t* counters, int k, float ratio,
                    int recent, int32_t* sel, const int64_t* sel_strides, int batch, int kv_heads,
                    int n_rep, int head_dim, int page, void* stream) {
    if (!q || !q_strides || !kmin || !kmax || !bound_strides || !block_tables || !seq_lens ||
        !scores || !score_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (page != ls::PAGE) return fail(LS_ERR_INVALID, "page (block_size) must be 16, got %d", page);
    if (n_rep < 1 || n_rep > ls::MAX_NREP)
        return fail(LS_ERR_INVALID, "n_rep must be in [1, %d], got %d", ls::MAX_NREP, n_rep);
    if (batch < 0 || batch > 65535 || kv_heads < 1 || kv_heads > 65535)
        return fail(LS_ERR_INVALID, "bad batch (%d) or kv_heads (%d)", batch, kv_heads);
    if (num_blocks < 0 || max_pages < 0 || recent < 0)
        return fail(LS_ERR_INVALID, "bad num_blocks, max_pages or recent");
    if (!rows_aligned(q, q_strides, 3, 2, 16))
        return fail(LS_ERR_INVALID, "q rows must be 16-byte aligned");
    if (!rows_aligned(kmin, bound_strides, 2, 2, 16) || !rows_aligned(kmax, bound_strides, 2, 2, 16))
        return fail(LS_ERR_INVALID, "kmin/kmax rows must be 16-byte aligned");
    if (!aligned(scores, 4)) return fail(LS_ERR_INVALID, "scores must be 4-byte aligned");
    const bool fused = sel != nullptr;
    (void)counters;   // unused since the selection became its own launch
    if (fused) {
        if (!sel_strides) return fail(LS_ERR_INVALID, "selection needs sel_strides");
        if (k < 1 || k > max_pages)
            return fail(LS_ERR_INVALID, "k must be in [1, max_pages=%d], got %d", max_pages, k);
        if (max_pages > ls::SELECT_MAX_PAGES)
            return fail(LS_ERR_INVALID, "selection supports max_pages <= %d, got %d",
                        ls::SELECT_MAX_PAGES, max_pages);
    }
    if (batch == 0 || max_pages == 0) return LS_OK;
    ls::IndexParams a{};
    a.q = q;
    a.sq_b = q_strides[0];
    a.sq_h = q_strides[1];
    a.sq_r = q_strides[2];
    a.kmin = kmin;
    a.kmax = kmax;
    a.sb_b = bound_strides[0];
    a.sb_h = bound_strides[1];
    a.num_blocks = num_blocks;
    a.block_tables = block_tables;
    a.sbt_b = bt_stride;
    a.max_pages = max_pages;
    a.seq_lens = seq_lens;
    a.scores = const_cast<float*>(scores);
    a.ss_b = score_strides[0];
    a.ss_h = score_strides[1];
    a.B = batch;
    a.H = kv_heads;
    a.NR = n_rep;
    a.recent = recent;
    const int rc = hip_status(ls::launch_page_index(a, (hipStream_t)stream),
                              fused ? "ls_sparse_index" : "ls_page_scores");
    if (rc != LS_OK || !fused) return rc;
    // the selection: one wave a (sequence, head) row, stream-ordered after
    // the scores it reads
    ls::SelectParams s;
    s.scores = scores;
    s.ss_b = score_strides[0];
    s.ss_h = score_strides[1];
    s.seq_lens = seq_lens;
    s.B = batch;
    s.H = kv_heads;
    s.P = max_pages;
    s.k = k;
    s.recent = recent;
    s.sorted = 0;
    s.ratio = ratio;
    s.sel = sel;
    s.sl_b = sel_strides[0];
    s.sl_h = sel_strides[1];
    return hip_status(ls::launch_page_select(s, (hipStream_t)stream), "ls_sparse_index");
}

int ls_page_select(const float* scores, const int64_t* score_strides, const int32_t* seq_lens,
                   int batch, int kv_heads, int num_pages, int k, float ratio, int recent,
                   int sorted, int32_t* sel, const int64_t* sel_strides, void* stream) {
    if (!scores || !score_strides || !sel || !sel_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (ratio > 0.f && !seq_lens) return fail(LS_ERR_INVALID, "a ratio needs seq_lens");
    if (batch < 0 || batch > 65535 || kv_heads < 1 || kv_heads > 65535 || recent < 0)
        return fail(LS_ERR_INVALID, "bad batch, kv_heads or recent");
    if (num_pages < 0 || num_pages > ls::SELECT_MAX_PAGES)
        return fail(LS_ERR_INVALID, "num_pages must be in [0, %d], got %d", ls::SELECT_MAX_PAGES,
                    num_pages);
    if (k < 0 || k > num_pages)
        return fail(LS_ERR_INVALID, "k must be in [0, num_pages=%d], got %d", num_pages, k);
    if (batch == 0 || k == 0) return LS_OK;
    ls::SelectParams a;
    a.scores = const_cast<float*>(scores);
    a.ss_b = score_strides[0];
    a.ss_h = score_strides[1];
    a.seq_lens = seq_lens;
    a.B = batch;
    a.H = kv_heads;
    a.P = num_pages;
    a.k = k;
    a.recent = recent;
    a.sorted = sorted ? 1 : 0;
    a.ratio = sorted ? 0.f : ratio;
    a.sel = sel;
    a.sl_b = sel_strides[0];
    a.sl_h = sel_strides[1];
    return hip_status(ls::launch_page_select(a, (hipStream_t)stream), "ls_page_select");
}

int ls_page_bounds_update(const void* k_new, const int64_t* kn_strides, const int64_t* slots,
                          void* kmin, void* kmax, const int64_t* bound_strides, int num_blocks,
                          int batch, int kv_heads, int head_dim, int page, void* stream) {
    if (!k_new || !kn_strides || !slots || !kmin || !kmax || !bound_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (page != ls::PAGE) return fail(LS_ERR_INVALID, "page (block_size) must be 16, got %d", page);
    if (batch < 0 || batch > (1 << 30) || kv_heads < 1 || kv_heads > 65535 || num_blocks < 0)
        return fail(LS_ERR_INVALID, "bad batch, kv_heads or num_blocks");
    if (!rows_aligned(k_new, kn_strides, 2, 2, 4) || !rows_aligned(kmin, bound_strides, 2, 2, 4) ||
        !rows_aligned(kmax, bound_strides, 2, 2, 4))
        return fail(LS_ERR_INVALID, "k_new, kmin and kmax rows must be 4-byte aligned");
    if (batch == 0) return LS_OK;
    ls::BoundsParams a;
    a.src = k_new;
    a.s0 = kn_strides[0];
    a.s1 = kn_strides[1];
    a.s2 = 0;
    a.slots = slots;
    a.kmin = kmin;
    a.kmax = kmax;
    a.sb_b = bound_strides[0];
    a.sb_h = bound_strides[1];
    a.num_blocks = num_blocks;
    a.B = batch;
    a.H = kv_heads;
    return hip_status(ls::launch_bounds_update(a, (hipStream_t)stream), "ls_page_bounds_update");
}

int ls_page_bounds_rebuild(const void* k_pool, const int64_t* kv_strides, int num_blocks,
                           void* kmin, void* kmax, const int64_t* bound_strides, int kv_heads,
                           int head_dim, int page, void* stream) {
    if (!k_pool || !kv_strides || !kmin || !kmax || !bound_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (page != ls::PAGE) return fail(LS_ERR_INVALID, "page (block_size) must be 16, got %d", page);
    if (kv_heads < 1 || num_blocks < 0) return fail(LS_ERR_INVALID, "bad kv_heads or num_blocks");
    if (!rows_aligned(k_pool, kv_strides, 3, 2, 16) || !rows_aligned(kmin, bound_strides, 2, 2, 16) ||
        !rows_aligned(kmax, bound_strides, 2, 2, 16))
        return fail(LS_ERR_INVALID, "k_pool, kmin and kmax rows must be 16-byte aligned");
    ls::BoundsParams a;
    a.src = k_pool;
    a.s0 = kv_strides[0];
    a.s1 = kv_strides[1];
    a.s2 = kv_strides[2];
    a.slots = nullptr;
    a.kmin = kmin;
    a.kmax = kmax;
    a.sb_b = bound_strides[0];
    a.sb_h = bound_strides[1];
    a.num_blocks = num_blocks;
    a.B = 0;
    a.H = kv_heads;
    return hip_status(ls::launch_bounds_rebuild(a, (hipStream_t)stream), "ls_page_bounds_rebuild");
}

static int quant_args(int asym, float eps, float qmax, float levels, float offset, int recip,
                      ls::QuantArgs& q) {
    if (!(qmax >= 1.f && qmax <= 127.f) || !(levels >= 1.f && levels <= 255.f) ||
        !(offset >= 0.f && offset <= 128.f) || !(eps >= 0.f))
        return fail(LS_ERR_INVALID, "bad quantizer constants (qmax %g, levels %g, offset %g, eps %g)",
                    qmax, levels, offset, eps);
    q.asym = asym ? 1 : 0;
    q.recip = recip ? 1 : 0;
    q.eps = eps;
    q.qmax = qmax;
    q.levels = levels;
    q.offset = offset;
    // the reciprocal as torch forms it for `t / python_number` on a GPU:
    // one fp32 division on the host
    volatile float one = 1.0f;
    q.inv_qmax = one / qmax;
    q.inv_levels = one / levels;
    return LS_OK;
}

int ls_int8_decode_write(const void* k, const int64_t* k_strides, const void* v,
                         const int64_t* v_strides, const int64_t* slots, const int64_t* res_idx,
                         void* flat_v, float* flat_v_scale, float* flat_v_zero, void* k_res,
                         int64_t num_slots, int64_t num_res, int batch, int kv_heads,
                         int head_dim, int asym, float eps, float qmax, float levels,
                         float offset, int recip, void* stream) {
    if (!k || !k_strides || !v || !v_strides || !slots || !res_idx || !flat_v || !flat_v_scale ||
        !k_res)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (asym && !flat_v_zero) return fail(LS_ERR_INVALID, "asymmetric quantization needs flat_v_zero");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (batch < 0 || kv_heads < 1 || num_slots < 0 || num_res < 0)
        return fail(LS_ERR_INVALID, "bad batch, kv_heads, num_slots or num_res");
    if (!rows_aligned(k, k_strides, 2, 2, 4) || !rows_aligned(v, v_strides, 2, 2, 4) ||
        !aligned(flat_v, 2) || !aligned(k_res, 4) || !aligned(flat_v_scale, 4))
        return fail(LS_ERR_INVALID, "k, v, flat_v and k_res rows must be aligned to channel pairs");
    ls::DecodeWriteParams a;
    if (int rc = quant_args(asym, eps, qmax, levels, offset, recip, a.q)) return rc;
    if (batch == 0) return LS_OK;
    a.k = k;
    a.sk_b = k_strides[0];
    a.sk_h = k_strides[1];
    a.v = v;
    a.sv_b = v_strides[0];
    a.sv_h = v_strides[1];
    a.slots = slots;
    a.res_idx = res_idx;
    a.flat_v = flat_v;
    a.flat_v_scale = flat_v_scale;
    a.flat_v_zero = flat_v_zero;
    a.k_res = k_res;
    a.num_slots = num_slots;
    a.num_res = num_res;
    a.B = batch;
    a.H = kv_heads;
    return hip_status(ls::launch_decode_write(a, (hipStream_t)stream), "ls_int8_decode_write");
}

int ls_int8_finalize_blocks(const void* data, const int64_t* data_strides, const int64_t* ids,
                            int n, void* k_pool, const int64_t* kv_strides, float* k_scale,
                            float* k_zero, const int64_t* ks_strides, int64_t num_blocks,
                            int kv_heads, int head_dim, int page, int asym, float eps, float qmax,
                            float levels, float offset, int recip, void* stream) {
    if (!data || !data_strides || !ids || !k_pool || !kv_strides || !k_scale || !ks_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (asym && !k_zero) return fail(LS_ERR_INVALID, "asymmetric quantization needs k_zero");
    if (head_dim != ls::HEAD_DIM) return fail(LS_ERR_INVALID, "head_dim must be 128, got %d", head_dim);
    if (page != ls::PAGE) return fail(LS_ERR_INVALID, "page (block_size) must be 16, got %d", page);
    if (n < 0 || kv_heads < 1 || num_blocks < 0)
        return fail(LS_ERR_INVALID, "bad n, kv_heads or num_blocks");
    if (!rows_aligned(data, data_strides, 3, 2, 4) || !rows_aligned(k_pool, kv_strides, 3, 1, 2) ||
        !aligned(k_scale, 4))
        return fail(LS_ERR_INVALID, "data, k_pool and k_scale rows must be aligned to channel pairs");
    ls::FinalizeParams a;
    if (int rc = quant_args(asym, eps, qmax, levels, offset, recip, a.q)) return rc;
    if (n == 0) return LS_OK;
    a.data = data;
    a.sd_n = data_strides[0];
    a.sd_t = data_strides[1];
    a.sd_h = data_strides[2];
    a.ids = ids;
    a.k_pool = k_pool;
    a.sp_b = kv_strides[0];
    a.sp_t = kv_strides[1];
    a.sp_h = kv_strides[2];
    a.k_scale = k_scale;
    a.k_zero = k_zero;
    a.ss_b = ks_strides[0];
    a.ss_h = ks_strides[1];
    a.num_blocks = num_blocks;
    a.N = n;
    a.H = kv_heads;
    return hip_status(ls::launch_finalize_k(a, (hipStream_t)stream), "ls_int8_finalize_blocks");
}

int ls_paged_gather(const void* pool, int elem_bytes, const int64_t* kv_strides, int num_blocks,
                    const int32_t* block_tables, int64_t bt_stride, int max_pages,
                    const int32_t* seq_lens, void* out, const int64_t* out_strides, int batch,
                    int kv_heads, int head_dim, int page, int length, void* stream) {
    if (!pool || !kv_strides || !block_tables || !seq_lens || !out || !out_strides)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4)
        return fail(LS_ERR_INVALID, "elem_bytes must be 1, 2 or 4, got %d", elem_bytes);
    if (page != ls::PAGE) return fail(LS_ERR_INVALID, "page (block_size) must be 16, got %d", page);
    if (head_dim < 1 || (head_dim * elem_bytes) % 16 != 0)
        return fail(LS_ERR_INVALID, "a head row must be a multiple of 16 bytes (head_dim %d)",
                    head_dim);
    if (batch < 0 || batch > 65535 || kv_heads < 1 || length < 0 || max_pages < 0 ||
        num_blocks < 1)
        return fail(LS_ERR_INVALID, "bad batch, kv_heads, length, max_pages or num_blocks");
    if ((int64_t)length * kv_heads * (head_dim * elem_bytes / 16) > (1LL << 31) - 256)
        return fail(LS_ERR_INVALID, "length x heads too large for one gather");
    if (!rows_aligned(pool, kv_strides, 3, (size_t)elem_bytes, 16) ||
        !rows_aligned(out, out_strides, 3, (size_t)elem_bytes, 16))
        return fail(LS_ERR_INVALID, "pool and out rows must be 16-byte aligned");
    if (batch == 0 || length == 0) return LS_OK;
    ls::GatherParams a;
    a.pool = pool;
    a.sp_b = kv_strides[0];
    a.sp_t = kv_strides[1];
    a.sp_h = kv_strides[2];
    a.num_blocks = num_blocks;
    a.block_tables = block_tables;
    a.sbt_b = bt_stride;
    a.max_pages = max_pages;
    a.seq_lens = seq_lens;
    a.out = out;
    a.so_b = out_strides[0];
    a.so_t = out_strides[1];
    a.so_h = out_strides[2];
    a.elem = elem_bytes;
    a.row_bytes = head_dim * elem_bytes;
    a.B = batch;
    a.L = length;
    a.H = kv_heads;
    return hip_status(ls::launch_gather(a, (hipStream_t)stream), "ls_paged_gather");
}

int ls_rms_norm(const void* x, int64_t x_stride, const void* residual, int64_t res_stride,
                const void* weight, void* y, int64_t y_stride, void* res_out,
                int64_t res_out_stride, int rows, int n, float eps, void* stream) {
    if (!x || !weight || !y) return fail(LS_ERR_INVALID, "null pointer argument");
    if ((residual == nullptr) != (res_out == nullptr))
        return fail(LS_ERR_INVALID, "residual and res_out must be given together");
    if (rows < 0 || rows > 2147483647 || n < 1)
        return fail(LS_ERR_INVALID, "rows must be >= 0 and n >= 1 (rows %d, n %d)", rows, n);
    if (!(eps >= 0.f)) return fail(LS_ERR_INVALID, "eps must be >= 0");
    ls::NormParams a;
    a.x = x;
    a.sx = x_stride;
    a.res = residual;
    a.sr = res_stride;
    a.w = weight;
    a.y = y;
    a.sy = y_stride;
    a.res_out = res_out;
    a.sro = res_out_stride;
    a.ids = nullptr;
    a.id_rows = 0;
    a.rows = rows;
    a.n = n;
    a.eps = eps;
    a.vec = n % 8 == 0 && aligned(x, 16) && aligned(weight, 16) && aligned(y, 16) &&
            x_stride % 8 == 0 && y_stride % 8 == 0 &&
            (!residual || (aligned(residual, 16) && aligned(res_out, 16) && res_stride % 8 == 0 &&
                           res_out_stride % 8 == 0));
    return hip_status(ls::launch_rms_norm(a, (hipStream_t)stream), "ls_rms_norm");
}

int ls_embed_rms_norm(const void* table, int64_t table_stride, int64_t table_rows,
                      const int64_t* ids, const void* weight, void* y, int64_t y_stride,
                      void* rows_out, int64_t rows_out_stride, int rows, int n, float eps,
                      void* stream) {
    if (!table || !ids || !weight || !y) return fail(LS_ERR_INVALID, "null pointer argument");
    if (rows < 0 || n < 1 || table_rows < 1)
        return fail(LS_ERR_INVALID, "rows must be >= 0, n >= 1 and the table non-empty");
    if (!(eps >= 0.f)) return fail(LS_ERR_INVALID, "eps must be >= 0");
    ls::NormParams a;
    a.x = table;
    a.sx = table_stride;
    a.res = nullptr;
    a.sr = 0;
    a.w = weight;
    a.y = y;
    a.sy = y_stride;
    a.res_out = rows_out;
    a.sro = rows_out_stride;
    a.ids = ids;
    a.id_rows = table_rows;
    a.rows = rows;
    a.n = n;
    a.eps = eps;
    a.vec = n % 8 == 0 && aligned(table, 16) && aligned(weight, 16) && aligned(y, 16) &&
            table_stride % 8 == 0 && y_stride % 8 == 0 &&
            (!rows_out || (aligned(rows_out, 16) && rows_out_stride % 8 == 0));
    return hip_status(ls::launch_rms_norm(a, (hipStream_t)stream), "ls_embed_rms_norm");
}

size_t ls_argmax_workspace_bytes(int rows, int n) {
    if (rows <= 0 || n < 1) return 0;
    return ls::argmax_workspace_bytes(rows, n);
}

int ls_argmax_rows(const void* x, int64_t x_stride, int64_t* out, int rows, int n,
                   void* workspace, size_t workspace_bytes, void* stream) {
    if (!x || !out) return fail(LS_ERR_INVALID, "null pointer argument");
    if (rows < 0 || rows > 65535 || n < 1)
        return fail(LS_ERR_INVALID, "rows must be in [0, 65535] and n >= 1");
    ls::ArgmaxParams a;
    a.x = x;
    a.sx = x_stride;
    a.out = out;
    a.parts = ls::argmax_parts(n);
    a.counters = nullptr;
    a.part_v = nullptr;
    a.part_i = nullptr;
    if (a.parts > 1 && rows > 0) {
        const size_t need = ls::argmax_workspace_bytes(rows, n);
        if (!workspace || workspace_bytes < need || !aligned(workspace, 16))
            return fail(LS_ERR_INVALID, "needs a 16-byte aligned workspace of %zu bytes", need);
        a.counters = (unsigned*)workspace;
        a.part_v = (float*)(a.counters + rows);
        a.part_i = (int*)(a.part_v + (size_t)rows * a.parts);
    }
    a.rows = rows;
    a.n = n;
    a.vec = n % 8 == 0 && aligned(x, 16) && x_stride % 8 == 0;
    return hip_status(ls::launch_argmax_rows(a, (hipStream_t)stream), "ls_argmax_rows");
}

int ls_silu_and_mul(const void* gate_up, int64_t gu_stride, void* out, int64_t out_stride,
                    int rows, int inter, void* stream) {
    if (!gate_up || !out) return fail(LS_ERR_INVALID, "null pointer argument");
    if (rows < 0 || rows > 65535 || inter < 1)
        return fail(LS_ERR_INVALID, "rows must be in [0, 65535] and inter >= 1 (rows %d, inter %d)",
                    rows, inter);
    ls::SiluParams a;
    a.gu = gate_up;
    a.sgu = gu_stride;
    a.out = out;
    a.so = out_stride;
    a.rows = rows;
    a.inter = inter;
    a.vec = inter % 8 == 0 && aligned(gate_up, 16) && aligned(out, 16) && gu_stride % 8 == 0 &&
            out_stride % 8 == 0;
    return hip_status(ls::launch_silu_and_mul(a, (hipStream_t)stream), "ls_silu_and_mul");
}

int ls_rope_qk(const void* q, int64_t q_stride, const void* k, int64_t k_stride, const void* cos,
               int64_t cos_stride, const void* sin, int64_t sin_stride, void* q_out,
               int64_t q_out_stride, void* k_out, int64_t k_out_stride, int rows, int hq, int hk,
               int head_dim, void* stream) {
    if (!q || !k || !cos || !sin || !q_out || !k_out)
        return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim < 2 || head_dim > 1024 || head_dim % 2 != 0)
        return fail(LS_ERR_INVALID, "head_dim must be even and in [2, 1024], got %d", head_dim);
    if (rows < 0 || hq < 0 || hk < 0 || hq + hk < 1 || hq + hk > 65535)
        return fail(LS_ERR_INVALID, "bad rows or head counts (rows %d, hq %d, hk %d)", rows, hq,
                    hk);
    ls::RopeParams a;
    a.q = q;
    a.sq = q_stride;
    a.k = k;
    a.sk = k_stride;
    a.cos = cos;
    a.sc = cos_stride;
    a.sin = sin;
    a.ss = sin_stride;
    a.qo = q_out;
    a.sqo = q_out_stride;
    a.ko = k_out;
    a.sko = k_out_stride;
    a.rows = rows;
    a.hq = hq;
    a.hk = hk;
    a.d = head_dim;
    return hip_status(ls::launch_rope_qk(a, (hipStream_t)stream), "ls_rope_qk");
}

int ls_rope_write_decode(const void* qkv, int64_t qkv_stride, const int64_t* positions,
                         const void* cos, const void* sin, int64_t table_stride, int table_rows,
                         const int64_t* slots, void* k_pool, void* v_pool,
                         const int64_t* kv_strides, int num_blocks, int page, void* q_out,
                         const int64_t* q_strides, void* kmin, void* kmax,
                         const int64_t* bounds_strides, int batch, int hq, int hk, int head_dim,
                         void* stream) {
    ls::RopeWriteParams a;
    const int rc = make_rope_params(a, qkv, qkv_stride, positions, cos, sin, table_stride,
                                    table_rows, slots, k_pool, v_pool, kv_strides, num_blocks,
                                    page, q_out, q_strides, kmin, kmax, bounds_strides, batch, hq,
                                    hk, head_dim);
    if (rc) return rc;
    return hip_status(ls::launch_rope_write_decode(a, (hipStream_t)stream), "ls_rope_write_decode");
}

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
                             int64_t res_out_stride, void* stream) {
    ls::GemmParams a;
    const int rc = make_rope_params(a.rope, x, 0, positions, cos, sin, table_stride, table_rows,
                                    slots, k_pool, v_pool, kv_strides, num_blocks, page, q_out,
                                    q_strides, kmin, kmax, bounds_strides, batch, hq, hk,
                                    head_dim);
    if (rc) return rc;
    if (!w) return fail(LS_ERR_INVALID, "null pointer argument");
    if (head_dim % 16 != 0) return fail(LS_ERR_INVALID, "head_dim must be a multiple of 16");
    if (batch > ls::GEMM_MAX_M || K < 32 || K % 32 != 0)
        return fail(LS_ERR_INVALID, "need batch <= %d and K a positive multiple of 32 (K %d)",
                    ls::GEMM_MAX_M, K);
    if (!weight_ok(x, x_stride, w, w_stride, w_packed, K))
        return fail(LS_ERR_INVALID, "x and w rows must be 16-byte aligned and hold K values");
    if (bias && !aligned(bias, 2)) return fail(LS_ERR_INVALID, "bias must be 2-byte aligned");
    const int N = (hq + 2 * hk) * head_dim;
    if (batch > 0 && ls::decode_gemm_splits(batch, N, K) != 1)
        return fail(LS_ERR_INVALID,
                    "K %d is too long to fuse at this width: use ls_decode_gemm, then "
                    "ls_rope_write_decode", K);
    if (batch == 0) return LS_OK;
    a.x = x;
    a.ldx = x_stride;
    a.w = w;
    a.ldw = w_stride;
    a.w_packed = w_packed ? 1 : 0;
    a.bias = bias;
    a.y = nullptr;
    a.ldy = 0;
    a.M = batch;
    a.N = N;
    a.K = K;
    a.vec_y = 0;
    a.part = nullptr;
    a.counters = nullptr;
    a.splits = 1;
    a.epi = ls::GEMM_ROPE;
    if (int nrc = set_norm(a, res, res_stride, norm_w, eps, res_out, res_out_stride,
                           "ls_decode_qkv_rope_write"))
        return nrc;
    return hip_status(ls::launch_decode_gemm(a, (hipStream_t)stream), "ls_decode_qkv_rope_write");
}

size_t ls_decode_gemm_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || M > ls::GEMM_MAX_M || N <= 0 || K < 32 || K % 32 != 0) return 0;
    return ls::decode_gemm_workspace_bytes(M, N, K);
}

int ls_decode_gemm(const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                   int w_packed, const void* bias, void* y, int64_t y_stride, int M, int N, int K,
                   void* workspace, size_t workspace_bytes, const void* res, int64_t res_stride,
                   const void* norm_w, float eps, void* res_out, int64_t res_out_stride,
                   void* stream) {
    if (!x || !w || !y) return fail(LS_ERR_INVALID, "null pointer argument");
    if (M < 0 || M > ls::GEMM_MAX_M || N < 0 || K < 32 || K % 32 != 0)
        return fail(LS_ERR_INVALID,
                    "need 0 <= M <= %d, N >= 0, K a positive multiple of 32 (M %d, N %d, K %d)",
                    ls::GEMM_MAX_M, M, N, K);
    if (!weight_ok(x, x_stride, w, w_stride, w_packed, K))
        return fail(LS_ERR_INVALID, "x and w rows must be 16-byte aligned and hold K values");
    if (!aligned(y, 2) || (M > 1 && y_stride < N))
        return fail(LS_ERR_INVALID, "y must be 2-byte aligned with y_stride >= N");
    if (bias && !aligned(bias, 2)) return fail(LS_ERR_INVALID, "bias must be 2-byte aligned");
    ls::GemmParams a;
    a.x = x;
    a.ldx = x_stride;
    a.w = w;
    a.ldw = w_stride;
    a.w_packed = w_packed ? 1 : 0;
    a.bias = bias;
    a.y = y;
    a.ldy = y_stride;
    a.M = M;
    a.N = N;
    a.K = K;
    a.vec_y = aligned(y, 8) && y_stride % 4 == 0;
    a.splits = M > 0 && N > 0 ? ls::decode_gemm_splits(M, N, K) : 1;
    a.part = (float*)workspace;
    a.counters = nullptr;
    a.epi = ls::GEMM_PLAIN;
    if (a.splits > 1) {
        const size_t need = ls::decode_gemm_workspace_bytes(M, N, K);
        if (!workspace || workspace_bytes < need || !aligned(workspace, 256))
            return fail(LS_ERR_INVALID,
                        "this product needs a 256-byte aligned workspace of %zu bytes (got %zu)",
                        need, workspace ? workspace_bytes : (size_t)0);
        if (ls::decode_gemm_units(M, N, K) > ls::GEMM_COUNTERS)
            return fail(LS_ERR_INVALID, "N %d is too wide for a split product", N);
        a.counters = (unsigned*)workspace;
        a.part = (float*)((char*)workspace + ls::GEMM_PART_OFFSET);
    }
    if (int nrc = set_norm(a, res, res_stride, norm_w, eps, res_out, res_out_stride,
                           "ls_decode_gemm"))
        return nrc;
    return hip_status(ls::launch_decode_gemm(a, (hipStream_t)stream), "ls_decode_gemm");
}

int ls_decode_gate_up_silu(const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                           int w_packed, const void* bias, void* y, int64_t y_stride, int M,
                           int inter, int K, const void* res, int64_t res_stride,
                           const void* norm_w, float eps, void* res_out, int64_t res_out_stride,
                           void* stream) {
    if (!x || !w || !y) return fail(LS_ERR_INVALID, "null pointer argument");
    if (M < 0 || M > ls::GEMM_MAX_M || inter < 0 || inter > (1 << 29) || K < 32 || K % 32 != 0)
        return fail(LS_ERR_INVALID,
                    "need 0 <= M <= %d, inter >= 0, K a positive multiple of 32 (M %d, inter %d, "
                    "K %d)", ls::GEMM_MAX_M, M, inter, K);
    if (!weight_ok(x, x_stride, w, w_stride, w_packed, K))
        return fail(LS_ERR_INVALID, "x and w rows must be 16-byte aligned and hold K values");
    if (!aligned(y, 2) || (M > 1 && y_stride < inter))
        return fail(LS_ERR_INVALID, "y must be 2-byte aligned with y_stride >= inter");
    if (bias && !aligned(bias, 2)) return fail(LS_ERR_INVALID, "bias must be 2-byte aligned");
    if (M > 0 && inter > 0 && ls::decode_gemm_splits(M, 2 * inter, K) != 1)
        return fail(LS_ERR_INVALID,
                    "K %d is too long to fuse at this width: use ls_decode_gemm, then "
                    "ls_silu_and_mul", K);
    ls::GemmParams a;
    a.x = x;
    a.ldx = x_stride;
    a.w = w;
    a.ldw = w_stride;
    a.w_packed = w_packed ? 1 : 0;
    a.bias = bias;
    a.y = y;
    a.ldy = y_stride;
    a.M = M;
    a.N = 2 * inter;
    a.K = K;
    a.vec_y = aligned(y, 8) && y_stride % 4 == 0;
    a.part = nullptr;
    a.counters = nullptr;
    a.splits = 1;
    a.epi = ls::GEMM_GLU;
    if (int nrc = set_norm(a, res, res_stride, norm_w, eps, res_out, res_out_stride,
                           "ls_decode_gate_up_silu"))
        return nrc;
    return hip_status(ls::launch_decode_gemm(a, (hipStream_t)stream), "ls_decode_gate_up_silu");
}

#ifdef LS_DIAGNOSTICS
// Diagnostic builds only: the page compute alone, MFMA (mode 0) against VALU (1).
int ls_compute_probe(int mode, int groups, int items, float scale, float* out, void* stream) {
    if (!out) return fail(LS_ERR_INVALID, "null pointer argument");
    if ((mode != 0 && mode != 1) || groups < 1 || groups > 65535 || items < 1)
        return fail(LS_ERR_INVALID, "mode 0 or 1, groups in [1, 65535], items >= 1");
    return hip_status(ls::launch_compute_probe(mode, groups, items, scale, out, (hipStream_t)stream),
                      "ls_compute_probe");
}
#endif

size_t ls_gemm_packed_bytes(int N, int K, int kind, int head_dim) {
    if (N < 1 || K < 32 || K % 32 != 0 || kind < 0 || kind > 2) return 0;
    return ls::gemm_packed_bytes(N, K, kind, head_dim);
}

int ls_pack_gemm_weight(const void* w, int64_t w_stride, int N, int K, int kind, int head_dim,
                        void* packed, void* stream) {
    if (!w || !packed) return fail(LS_ERR_INVALID, "null pointer argument");
    if (N < 1 || K < 32 || K % 32 != 0)
        return fail(LS_ERR_INVALID, "need N >= 1 and K a positive multiple of 32 (N %d, K %d)", N,
                    K);
    if (kind < 0 || kind > 2) return fail(LS_ERR_INVALID, "kind must be 0, 1 or 2, got %d", kind);
    if (kind == 1 && N % 2 != 0) return fail(LS_ERR_INVALID, "a gate/up weight has 2I rows");
    if (kind == 2 && (head_dim < 16 || head_dim % 16 != 0 || N % head_dim != 0))
        return fail(LS_ERR_INVALID, "a q/k/v weight needs head_dim %% 16 == 0 dividing N");
    if (!aligned(w, 16) || w_stride % 8 != 0 || w_stride < K || !aligned(packed, 16))
        return fail(LS_ERR_INVALID, "w rows and packed must be 16-byte aligned");
    return hip_status(ls::launch_pack_gemm_weight(w, w_stride, N, K, kind, head_dim, packed,
                                                  (hipStream_t)stream),
                      "ls_pack_gemm_weight");
}

}  // extern "C"
