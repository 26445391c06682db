// Page selection for sparse decode on gfx950: the page indexer (Quest upper
// bound per page), top-k selection, and the per-page K bounds it reads.
//
// Reference: kernels/cuda/paged_sparse_fp16.cu:54-72 (page_bounds_update),
// :78-130 (page_index), kernels/cuda/paged_sparse.py:81-123 (rebuild_bounds,
// update_bounds, page_scores), :164-168 (select = torch.topk) and
// :222-251 (sparse_attention: index -> select -> attend).
//
// Design:
//  * Indexer: a wave scores 4 pages at a time, 16 lanes per page, 8 channels
//    per lane (one 16-byte load of kmin and of kmax).  The per-head bound
//    sum_d max(q_d * lo_d, q_d * hi_d) is formed in fp32 (each product of two
//    fp16 values is exact in fp32) and reduced over the 16 lanes with four
//    DPP adds; the page score is the max over the n_rep query heads.  The
//    work is a pass over 2 x 256 bytes per (page, KV head): HBM-bound.
//  * Selection: a 4-pass radix select (8-bit digits, LDS histograms) finds
//    the n-th largest key of a (sequence, KV head) row, and the selected
//    page ids are written in page order.  Ties at the threshold are taken in
//    page order, so the result is deterministic.  With a ratio the first n_b
//    entries are the sequence's own budget (the rule the sparse decode kernel
//    applies to the list), the rest of the k entries follow.  One 256-thread
//    group a row, the row's keys in its registers (up to 32 a thread); the
//    select itself is in ls_select.h, shared with the sparse decode kernel,
//    whose workgroups can run it on the scores in their prologue.
//  * ls_sparse_index (index, then select) is two launches.  A single launch
//    in which the last index group of a row ran its selection was slower
//    than the pair: its arrival count is a device-scope atomic issued while
//    the other groups stream the page bounds, and such atomics take several
//    microseconds to return under that traffic.
#include "ls_common.h"
#include "ls_sparse.h"
#include "ls_select.h"
#include "ls_quest.h"

namespace ls {

namespace {

enum : int { PG_SKIP = 0, PG_SCORE = 1, PG_FORCED = 2, PG_PAST = 3 };

// NR: query rows per KV head (a compile-time count keeps only those rows'
// registers, which sets how many index groups a CU holds at once).
// MASS: instead of the group's max bound, write every query head's bound as
// a log2-domain logit, bound * scale * log2(e) + log2(tokens in the page),
// to heads[b, h, r, p] (sink and recent pages scored like the others, pages
// past the end or with a block id outside the pool -inf); page_mass_kernel
// turns them into the summed-mass scores.
template <int NR, bool MASS = false>
__global__ __launch_bounds__(256) void page_index_kernel(IndexParams a) {
    const int b = blockIdx.z, h = blockIdx.y;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int c0 = (lane & 15) * 8;
    const int L = a.seq_lens[b];
    const int np = L > 0 ? (L + PAGE - 1) / PAGE : 0;

    // the two pages of this lane's row group: state and bounds
    int pg[2], st[2];
    u4 lo[2], hi[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = blockIdx.x * INDEX_PAGES_PER_GROUP + wv * 8 + i * 4 + (lane >> 4);
        pg[i] = p;
        lo[i] = u4{0u, 0u, 0u, 0u};
        hi[i] = u4{0u, 0u, 0u, 0u};
        if (p >= a.max_pages) {
            st[i] = PG_SKIP;
        } else if (p >= np) {
            st[i] = PG_PAST;
        } else if (!MASS && (p == 0 || p >= np - a.recent)) {
            st[i] = PG_FORCED;
        } else {
            const int blk = a.block_tables[(int64_t)b * a.sbt_b + p];
            if ((unsigned)blk >= (unsigned)a.num_blocks) {
                st[i] = PG_PAST;            // a block id outside the pool is never chosen
            } else {
                st[i] = PG_SCORE;
                const int64_t off = (int64_t)blk * a.sb_b + (int64_t)h * a.sb_h + c0;
                lo[i] = stream_load((const u4*)((const half_t*)a.kmin + off));
                hi[i] = stream_load((const u4*)((const half_t*)a.kmax + off));
            }
        }
    }
    const half_t* qb = (const half_t*)a.q + (int64_t)b * a.sq_b + (int64_t)h * a.sq_h + c0;
    u4 qv[NR], qm[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) qv[r] = *(const u4*)(qb + (int64_t)r * a.sq_r);
#pragma unroll
    for (int r = 0; r < NR; ++r) qm[r] = quest_masks(qv[r]);

    float best[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        float bst = neg_inf();
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float s = quest_row16_sum(quest_part(qv[r], qm[r], lo[i], hi[i]));
            if (MASS)
                bst = (lane & 15) == r ? s : bst;    // lane r of the row keeps head r
            else
                bst = fmaxf(bst, s);
        }
        best[i] = bst;
    }
    if constexpr (MASS) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = lane & 15;
            if (r < NR && st[i] != PG_SKIP) {
                float v = neg_inf();
                if (st[i] == PG_SCORE) {
                    const int cnt = min(PAGE, L - pg[i] * PAGE);
                    v = best[i] * a.scale_log2 + __log2f((float)cnt);
                }
                a.heads[(int64_t)b * a.sh_b + (int64_t)h * a.sh_h + (int64_t)r * a.sh_r + pg[i]] = v;
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if ((lane & 15) == 0 && st[i] != PG_SKIP) {
            const float v = st[i] == PG_SCORE ? best[i]
                            : st[i] == PG_FORCED ? __builtin_inff() : neg_inf();
            a.scores[(int64_t)b * a.ss_b + (int64_t)h * a.ss_h + pg[i]] = v;
        }
    }
}

// Summed-mass page scores from the per-head logits (one 256-thread group
// per (sequence, KV head) row): for each query head a softmax over the
// row's pages of its log2-domain logits, the softmaxes summed over the
// group's heads; sink and recent pages +inf, pages past the end -inf
// (kernels/cuda/paged_sparse.py:126-161).  Three passes over the row's
// NR x P logits (just written, cache-resident): maxima, sums, scores.
template <int NR>
__global__ __launch_bounds__(256) void page_mass_kernel(IndexParams a) {
    __shared__ float red[4][NR];
    const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int L = a.seq_lens[b];
    const int np = L > 0 ? (L + PAGE - 1) / PAGE : 0;
    const int P = a.max_pages;
    const float* row = a.heads + (int64_t)b * a.sh_b + (int64_t)h * a.sh_h;
    float* out = a.scores + (int64_t)b * a.ss_b + (int64_t)h * a.ss_h;

    auto group_reduce = [&](float (&v)[NR], bool is_max) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const float o = __shfl_xor(v[r], off);
                v[r] = is_max ? fmaxf(v[r], o) : v[r] + o;
            }
        }
        __syncthreads();                    // red[] free (read by the last reduction)
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < NR; ++r) red[wv][r] = v[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float x0 = red[0][r], x1 = red[1][r], x2 = red[2][r], x3 = red[3][r];
            v[r] = is_max ? fmaxf(fmaxf(x0, x1), fmaxf(x2, x3)) : (x0 + x1) + (x2 + x3);
        }
    };

    float mx[NR], sm[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) mx[r] = neg_inf();
    for (int p = tid; p < P; p += 256)
#pragma unroll
        for (int r = 0; r < NR; ++r) mx[r] = fmaxf(mx[r], row[(int64_t)r * a.sh_r + p]);
    group_reduce(mx, true);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        sm[r] = 0.f;
        mx[r] = mx[r] == neg_inf() ? 0.f : mx[r];   // an empty row: every weight 0
    }
    for (int p = tid; p < P; p += 256)
#pragma unroll
        for (int r = 0; r < NR; ++r) sm[r] += exp2f(row[(int64_t)r * a.sh_r + p] - mx[r]);
    group_reduce(sm, false);
    float inv[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) inv[r] = sm[r] > 0.f ? 1.f / sm[r] : 0.f;
    for (int p = tid; p < P; p += 256) {
        float v;
        if (p >= np) {
            v = neg_inf();
        } else if (p == 0 || p >= np - a.recent) {
            v = __builtin_inff();
        } else {
            v = 0.f;
#pragma unroll
            for (int r = 0; r < NR; ++r) v += exp2f(row[(int64_t)r * a.sh_r + p] - mx[r]) * inv[r];
        }
        out[p] = v;
    }
}

template <bool SORTED>
__global__ __launch_bounds__(256) void page_select_kernel(SelectParams a) {
    __shared__ SelectSmem sm;
    __shared__ uint32_t skeys[SORTED ? SELECT_MAX_PAGES : 1];
    const int h = blockIdx.x, b = blockIdx.y;
    const int L = a.seq_lens ? a.seq_lens[b] : 0;
    const int n1 = SORTED ? a.k : budget_pages(L, a.P, a.ratio, a.recent, a.k);
    int32_t* out = a.sel + (int64_t)b * a.sl_b + (int64_t)h * a.sl_h;
    const float* srow = a.scores + (int64_t)b * a.ss_b + (int64_t)h * a.ss_h;
    // a position outside the row is never stored: a bad scan result (a
    // histogram counted from a lane that held no key) cannot reach memory
    // outside this row of the output
    const int k = a.k;
    auto emit = [&](int pos, int pg) {
        if ((unsigned)pos < (unsigned)k) out[pos] = pg;
    };
    if constexpr (!SORTED) {
        // one threshold (the whole list is the budget): the linear-bin search
        // the selecting decode runs
        __shared__ LinSelectSmem lsm;
        if (n1 == k) {
            select_lin(srow, a.P, n1, (int)threadIdx.x, lsm, emit);
            return;
        }
    }
    select_row<SORTED>(srow, a.P, n1, a.k, (int)threadIdx.x, out, sm, skeys, emit);
}

// grid (B, H), 64 threads: two channels per lane.
__global__ __launch_bounds__(64) void bounds_update_kernel(BoundsParams a) {
    const int b = blockIdx.x, h = blockIdx.y, c = threadIdx.x * 2;
    const int64_t slot = a.slots[b];
    if (slot < 0) return;
    const int64_t blk = slot / PAGE;
    const int off = (int)(slot % PAGE);
    if (blk >= a.num_blocks) return;
    const h2 v = *(const h2*)((const half_t*)a.src + (int64_t)b * a.s0 + (int64_t)h * a.s1 + c);
    const int64_t i = blk * a.sb_b + (int64_t)h * a.sb_h + c;
    h2* mn = (h2*)((half_t*)a.kmin + i);
    h2* mx = (h2*)((half_t*)a.kmax + i);
    if (off == 0) {                     // a page's first token resets its bounds
        *mn = v;
        *mx = v;
        return;
    }
    const h2 m0 = *mn, x0 = *mx;        // fp16 min / max through fp32 are exact
    h2 rn, rx;
    rn.x = (half_t)fminf((float)m0.x, (float)v.x);
    rn.y = (half_t)fminf((float)m0.y, (float)v.y);
    rx.x = (half_t)fmaxf((float)x0.x, (float)v.x);
    rx.y = (half_t)fmaxf((float)x0.y, (float)v.y);
    *mn = rn;
    *mx = rx;
}

// One (block, head) per 16 lanes, 8 channels per lane, all 16 rows.
__global__ __launch_bounds__(256) void bounds_rebuild_kernel(BoundsParams a) {
    const int lane = threadIdx.x & 63;
    const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;
    if (item >= (int64_t)a.num_blocks * a.H) return;
    const int64_t blk = item / a.H;
    const int h = (int)(item % a.H);
    const int c0 = (lane & 15) * 8;
    const half_t* src = (const half_t*)a.src + blk * a.s0 + (int64_t)h * a.s2 + c0;
    u4 rows[PAGE];
#pragma unroll
    for (int t = 0; t < PAGE; ++t) rows[t] = stream_load((const u4*)(src + (int64_t)t * a.s1));
    float mn[8], mx[8];
    quest_h8_to_f8(rows[0], mn);
    quest_h8_to_f8(rows[0], mx);
#pragma unroll
    for (int t = 1; t < PAGE; ++t) {
        float f[8];
        quest_h8_to_f8(rows[t], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            mn[j] = fminf(mn[j], f[j]);
            mx[j] = fmaxf(mx[j], f[j]);
        }
    }
    uint32_t wn[4], wx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2 a2 = {(half_t)mn[2 * i], (half_t)mn[2 * i + 1]};
        h2 b2 = {(half_t)mx[2 * i], (half_t)mx[2 * i + 1]};
        wn[i] = __builtin_bit_cast(uint32_t, a2);
        wx[i] = __builtin_bit_cast(uint32_t, b2);
    }
    const u4 omn = {wn[0], wn[1], wn[2], wn[3]};
    const u4 omx = {wx[0], wx[1], wx[2], wx[3]};
    const int64_t o = blk * a.sb_b + (int64_t)h * a.sb_h + c0;
    *(u4*)((half_t*)a.kmin + o) = omn;
    *(u4*)((half_t*)a.kmax + o) = omx;
}

}  // namespace

hipError_t launch_page_index(const IndexParams& p, hipStream_t stream) {
    if (p.B == 0 || p.max_pages == 0) return hipSuccess;
    const dim3 grid((p.max_pages + INDEX_PAGES_PER_GROUP - 1) / INDEX_PAGES_PER_GROUP, p.H, p.B);
    switch (p.NR) {
#define LS_INDEX_NR(n) \
    case n: hipLaunchKernelGGL(page_index_kernel<n>, grid, dim3(256), 0, stream, p); break;
        LS_INDEX_NR(1) LS_INDEX_NR(2) LS_INDEX_NR(3) LS_INDEX_NR(4) LS_INDEX_NR(5) LS_INDEX_NR(6)
        LS_INDEX_NR(7) LS_INDEX_NR(8) LS_INDEX_NR(9) LS_INDEX_NR(10) LS_INDEX_NR(11)
        LS_INDEX_NR(12) LS_INDEX_NR(13) LS_INDEX_NR(14) LS_INDEX_NR(15) LS_INDEX_NR(16)
#undef LS_INDEX_NR
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_page_mass(const IndexParams& p, hipStream_t stream) {
    if (p.B == 0 || p.max_pages == 0) return hipSuccess;
    const dim3 grid((p.max_pages + INDEX_PAGES_PER_GROUP - 1) / INDEX_PAGES_PER_GROUP, p.H, p.B);
    switch (p.NR) {
#define LS_MASS_NR(n)                                                                      \
    case n:                                                                                \
        hipLaunchKernelGGL((page_index_kernel<n, true>), grid, dim3(256), 0, stream, p);   \
        hipLaunchKernelGGL(page_mass_kernel<n>, dim3(p.H, p.B), dim3(256), 0, stream, p);  \
        break;
        LS_MASS_NR(1) LS_MASS_NR(2) LS_MASS_NR(3) LS_MASS_NR(4) LS_MASS_NR(5) LS_MASS_NR(6)
        LS_MASS_NR(7) LS_MASS_NR(8) LS_MASS_NR(9) LS_MASS_NR(10) LS_MASS_NR(11)
        LS_MASS_NR(12) LS_MASS_NR(13) LS_MASS_NR(14) LS_MASS_NR(15) LS_MASS_NR(16)
#undef LS_MASS_NR
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_page_select(const SelectParams& p, hipStream_t stream) {
    if (p.B == 0 || p.k == 0) return hipSuccess;
    const dim3 grid(p.H, p.B);
    if (p.sorted) {
        hipLaunchKernelGGL(page_select_kernel<true>, grid, dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(page_select_kernel<false>, grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bounds_update(const BoundsParams& p, hipStream_t stream) {
    if (p.B == 0) return hipSuccess;
    hipLaunchKernelGGL(bounds_update_kernel, dim3(p.B, p.H), dim3(64), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bounds_rebuild(const BoundsParams& p, hipStream_t stream) {
    const int64_t items = (int64_t)p.num_blocks * p.H;
    if (items == 0) return hipSuccess;
    const int64_t groups = (items * 16 + 255) / 256;
    hipLaunchKernelGGL(bounds_rebuild_kernel, dim3((unsigned)groups), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t sparse_index_resources(int what, int n_rep, KernelResources* r) {
    switch (what) {
        case 3: return func_resources(page_select_kernel<false>, 256, r);
        case 4: return func_resources(bounds_update_kernel, 64, r);
        case 5: return func_resources(bounds_rebuild_kernel, 256, r);
        default: break;
    }
    switch (n_rep) {
#define LS_RES_NR(n)                                                               \
    case n:                                                                        \
        return what == 0   ? func_resources(page_index_kernel<n>, 256, r)          \
               : what == 1 ? func_resources(page_index_kernel<n, true>, 256, r)    \
               : what == 2 ? func_resources(page_mass_kernel<n>, 256, r)           \
                           : hipErrorInvalidValue;
        LS_RES_NR(1) LS_RES_NR(2) LS_RES_NR(3) LS_RES_NR(4) LS_RES_NR(5) LS_RES_NR(6)
        LS_RES_NR(7) LS_RES_NR(8) LS_RES_NR(9) LS_RES_NR(10) LS_RES_NR(11)
        LS_RES_NR(12) LS_RES_NR(13) LS_RES_NR(14) LS_RES_NR(15) LS_RES_NR(16)
#undef LS_RES_NR
        default: return hipErrorInvalidValue;
    }
}

}  // namespace ls
