// Top-k page selection over a row of page scores, for a group of 256
// threads: the selection kernel (one group a row) and the selecting decodes'
// prologues (one group a head of the workgroup).
//
// Two searches.  select_row_k, a radix select (8-bit digits, LDS
// histograms, up to 4 passes: it stops once the threshold digit's bin is
// taken whole), finds two thresholds at once (a sequence's own budget and
// the list width) and can report the set best first; the selection kernel
// uses it for those.  select_row_lin finds one threshold over linear bins
// (described below it); the selecting decodes and the one-threshold
// selection use it.  Either reports the selected pages in page order, ties
// at the threshold taken in page order (deterministic).  Reference:
// kernels/cuda/paged_sparse.py:164-168 (select = torch.topk) and the budget
// rule of kernels/cuda/paged_sparse_fp16.cu:242-247.
#pragma once

#include "ls_common.h"
#include "ls_sparse.h"

namespace ls {

// Order-preserving map float -> uint32 (larger float, larger key); -0 and
// +0 compare equal, as they do for the reference's torch.topk.
__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u = u == 0x80000000u ? 0u : u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Pages a sequence of length L attends with this ratio: the rule of the
// sparse decode kernel (paged_sparse_fp16.cu:242-247), capped at k.
__device__ __forceinline__ int budget_pages(int L, int P, float ratio, int recent, int k) {
    int pages = L > 0 ? (L + PAGE - 1) / PAGE : 0;
    pages = pages < P ? pages : P;
    if (!(ratio > 0.f)) return k;
    int want;
    if (ratio >= 1.f) {
        want = pages;
    } else {
        want = (int)ceilf(ratio * (float)pages);
        want = want > recent + 1 ? want : recent + 1;
    }
    want = want < pages ? want : pages;
    return want < k ? want : k;
}

constexpr int SEL_THREADS = 256;
constexpr int SEL_KPT = SELECT_MAX_PAGES / SEL_THREADS;   // keys per thread

struct SelectSmem {
    uint32_t hist[2][2][256];          // [pass parity][threshold][digit]
    uint32_t wsum[2][4];               // [scan parity][wave]
    int found[4];
    uint32_t pfx[2][4];                // [and, or][wave]
};

// Inclusive prefix sum over the 256 threads of a group (tid: the thread's
// index in its group of 256, whose four waves are whole hardware waves):
// DPP row shifts within each row of 16 lanes, readlane for the rows, the
// four waves' totals through LDS with one barrier.  `wsum` alternates
// between consecutive calls (a thread may write the next call's totals
// while another still reads this call's).
__device__ __forceinline__ uint32_t group_scan(uint32_t v, uint32_t* wsum, int tid) {
    const int lane = tid & 63, wv = tid >> 6;
    int x = (int)v;
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);   // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31),
              r2 = __builtin_amdgcn_readlane(x, 47), r3 = __builtin_amdgcn_readlane(x, 63);
    const int row = lane >> 4;
    x += (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
    if (lane == 0) wsum[wv] = (uint32_t)(r0 + r1 + r2 + r3);
    __syncthreads();
    uint32_t u = (uint32_t)x;
    for (int w = 0; w < wv; ++w) u += wsum[w];
    return u;
}

// Select from one row of P scores: out[0, n1) = the n1 best pages, out[n1,
// n2) = the next n2 - n1 (n1 <= n2 <= P), each part in page order.  Order
// among equal scores: lower page first.  With SORTED (n1 == n2) the n2 pages
// are written best first instead.
//
// KPT keys per thread (P <= 256 * KPT): the loops over a thread's keys are
// fully unrolled at exactly KPT, so their cost follows the row length.
//
// Every group of a workgroup passes the same barriers (a workgroup may run
// one group a head): three a radix pass, one a scan after them.
//
// COOP: the row is being written by other workgroups of the same launch
// (the selecting decode's own scoring): once `fix.wait()` reports the
// writers' count complete it is read with device-coherent loads; if the
// count does not complete within its time bound, every score the thread
// needs is computed by `fix(page)` instead (the same bits: the writers
// compute them the same way, and the row may still hold an earlier call's
// scores), so no workgroup depends on another being resident.
struct NoFix {
    __device__ float operator()(int) const { return 0.f; }
    __device__ bool wait() const { return true; }
};

// A thread's KPT keys of the row (pages tid * KPT ...), as order keys;
// `cnt` of them are real (the rest are past P).  COOP: the row is being
// written by other workgroups of the same launch (described above).
template <int KPT, int COOP, class Fix>
__device__ __attribute__((always_inline)) void select_keys(const float* srow, int P, int tid,
                                                           int i0, int cnt, uint32_t* key,
                                                           Fix fix) {
    // unconditional loads (clamped index) so they all issue back to back
    float f[KPT];
    const int last = P > 0 ? P - 1 : 0;
    if constexpr (COOP) {
        const bool done = fix.wait();   // the row's writers say they are done
        LS_STAMP(3);
        if (done && ((uintptr_t)srow & 15) == 0) {
            // a 16-byte aligned row: 16-byte device-coherent loads over a
            // resource of the row's P words (lanes past it read zeros);
            // against one 4-byte load a key, B8 x 32K 45.63 -> 45.10 us
            static_assert(KPT % 4 == 0, "keys in 16-byte pieces");
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc((void*)srow, 0, P * 4, 0x00020000);
#pragma unroll
            for (int j = 0; j < KPT; j += 4) {
                const f4 v = load_coherent4(rs, (i0 + j) * 4);
                f[j] = v[0];
                f[j + 1] = v[1];
                f[j + 2] = v[2];
                f[j + 3] = v[3];
            }
        } else if (done) {
#pragma unroll
            for (int j = 0; j < KPT; ++j)
                f[j] = P > 0 ? load_coherent(srow + (i0 + j < last ? i0 + j : last)) : 0.f;
        } else {
            // a writer not seen finishing in time: this thread's scores
            // computed here, none read from the row
#pragma unroll
            for (int j = 0; j < KPT; ++j) f[j] = j < cnt ? fix(i0 + j) : 0.f;
        }
        LS_STAMP(4);
    } else {
#pragma unroll
        for (int j = 0; j < KPT; ++j) f[j] = P > 0 ? srow[i0 + j < last ? i0 + j : last] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < KPT; ++j) key[j] = j < cnt ? order_key(f[j]) : 0u;
}

template <bool SORTED, int KPT, class Emit>
__device__ __attribute__((always_inline)) void select_row_k(const float* srow, int P, int n1,
                                                            int n2, int tid, int32_t* out,
                                                            SelectSmem& sm, uint32_t* skeys,
                                                            Emit emit) {
    const int i0 = tid * KPT;
    int cnt = P - i0;
    cnt = cnt < 0 ? 0 : (cnt > KPT ? KPT : cnt);
    uint32_t key[KPT];
    select_keys<KPT, 0>(srow, P, tid, i0, cnt, key, NoFix());

    // ---- radix select of the n1-th and n2-th largest keys ----
    uint32_t pre0 = 0, pre1 = 0, msk = 0;
    int rem0 = n1, rem1 = n2;
    int nscan = 0;
    sm.hist[0][0][tid] = 0;
    sm.hist[0][1][tid] = 0;
    // The finite scores of a row share their leading bits (one exponent):
    // a pass over them would put every key in one bin.  So the bits common
    // to the finite keys (forced pages +inf and pages past the end -inf
    // excluded) are found first, and when both thresholds fall among the
    // keys with that prefix, the passes start right below it.
    int shift = 24;
    {
        constexpr uint32_t KEY_PINF = 0xFF800000u, KEY_NINF = 0x007FFFFFu;
        uint32_t kand = 0xFFFFFFFFu, kor = 0u;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            if (j < cnt && key[j] != KEY_PINF && key[j] != KEY_NINF) {
                kand &= key[j];
                kor |= key[j];
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            kand &= (uint32_t)__shfl_xor((int)kand, o);
            kor |= (uint32_t)__shfl_xor((int)kor, o);
        }
        if ((tid & 63) == 0) {
            sm.pfx[0][tid >> 6] = kand;
            sm.pfx[1][tid >> 6] = kor;
        }
        __syncthreads();
        kand = sm.pfx[0][0] & sm.pfx[0][1] & sm.pfx[0][2] & sm.pfx[0][3];
        kor = sm.pfx[1][0] | sm.pfx[1][1] | sm.pfx[1][2] | sm.pfx[1][3];
        const bool any = kand <= kor;                    // some finite key
        const uint32_t diff = kand ^ kor;
        const int h = diff ? 31 - __builtin_clz(diff) : 0;   // highest differing bit
        const uint32_t hi = h >= 31 ? 0u : ~((2u << h) - 1u); // the common bits
        const uint32_t p0 = kand & hi;
        uint32_t above = 0, same = 0;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            if (j < cnt) {
                above += (key[j] & hi) > p0 ? 1u : 0u;
                same += (key[j] & hi) == p0 ? 1u : 0u;
            }
        }
        const int par = nscan++ & 1;
        (void)group_scan(above | (same << 16), sm.wsum[par], tid);
        const uint32_t tot = sm.wsum[par][0] + sm.wsum[par][1] + sm.wsum[par][2] + sm.wsum[par][3];
        const int A = (int)(tot & 0xFFFFu), M = (int)(tot >> 16);
        auto inside = [&](int n) { return n == 0 || (A < n && n <= A + M); };
        if (any && hi != 0u && inside(n1) && inside(n2)) {
            pre0 = pre1 = p0;
            msk = hi;
            rem0 = n1 > 0 ? n1 - A : 0;
            rem1 = n2 > 0 ? n2 - A : 0;
            shift = h - 7;
        }
    }
    const bool two = n2 > 0;            // a second threshold to find
    for (int par = 0;; par ^= 1) {
        // (a pass below bit 0 repeats the bits of the last: the keys that
        // still match the prefix agree on them, so such a pass changes
        // nothing; it runs only while another group of the workgroup goes on)
        const int sh = shift > 0 ? shift : 0;
        // A thread's keys are adjacent pages whose leading digits mostly
        // agree (one exponent for the whole row): count runs of equal digits
        // and add each run once, instead of one LDS atomic per key on a
        // handful of hot bins.
        uint32_t d0 = 256u, n0 = 0u, d1 = 256u, n1c = 0u;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            if (j < cnt) {
                const uint32_t d = (key[j] >> sh) & 255u;
                if ((key[j] & msk) == pre0) {
                    if (d != d0) {
                        if (n0) atomicAdd(&sm.hist[par][0][d0], n0);
                        d0 = d;
                        n0 = 0u;
                    }
                    ++n0;
                }
                if (two && (key[j] & msk) == pre1) {
                    if (d != d1) {
                        if (n1c) atomicAdd(&sm.hist[par][1][d1], n1c);
                        d1 = d;
                        n1c = 0u;
                    }
                    ++n1c;
                }
            }
        }
        if (n0) atomicAdd(&sm.hist[par][0][d0], n0);
        if (n1c) atomicAdd(&sm.hist[par][1][d1], n1c);
        // the next pass's histogram (last read two barriers ago)
        sm.hist[par ^ 1][0][tid] = 0;
        sm.hist[par ^ 1][1][tid] = 0;
        __syncthreads();
        const int bin = 255 - tid;   // thread order = descending digit
        const uint32_t c = sm.hist[par][0][bin] | (sm.hist[par][1][bin] << 16);
        const uint32_t incl = group_scan(c, sm.wsum[nscan++ & 1], tid);
        const uint32_t excl = incl - c;
        const int ci0 = (int)(incl & 0xFFFFu), ce0 = (int)(excl & 0xFFFFu);
        const int ci1 = (int)(incl >> 16), ce1 = (int)(excl >> 16);
        // the thread holding a threshold's digit reports it, and whether
        // that digit's bin is taken whole (then no lower digit matters)
        bool open = false;
        if (ce0 < rem0 && ci0 >= rem0) {
            sm.found[0] = bin;
            sm.found[1] = rem0 - ce0;
            open = open || rem0 - ce0 != ci0 - ce0;
        }
        if (ce1 < rem1 && ci1 >= rem1) {
            sm.found[2] = bin;
            sm.found[3] = rem1 - ce1;
            open = open || rem1 - ce1 != ci1 - ce1;
        }
        // the whole workgroup goes on while any of its groups has a side open
        // (after the pass at bit 0 every bit is decided: nothing is open)
        const bool more = __syncthreads_or(open && sh > 0);
        if (rem0 > 0) {
            pre0 |= (uint32_t)sm.found[0] << sh;
            rem0 = sm.found[1];
        }
        if (rem1 > 0) {
            pre1 |= (uint32_t)sm.found[2] << sh;
            rem1 = sm.found[3];
        }
        msk |= 255u << sh;
        if (!more) break;
        shift -= 8;
    }
    // threshold prefixes pre0 / pre1 of the keys under msk; rem0 / rem1 =
    // how many keys with that prefix belong to the set (the lowest pages
    // first; all of them when the passes stopped early)
    const bool want0 = n1 > 0, want1 = n2 > 0;
    uint32_t kp[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) kp[j] = key[j] & msk;

    uint32_t e = 0;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
        if (j < cnt) e += (kp[j] == pre0 ? 1u : 0u) + (kp[j] == pre1 ? 0x10000u : 0u);
    uint32_t incl = group_scan(e, sm.wsum[nscan++ & 1], tid);
    uint32_t excl = incl - e;
    int r0 = (int)(excl & 0xFFFFu), r1 = (int)(excl >> 16);
    uint32_t ma = 0, mb = 0;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        if (j < cnt) {
            bool a0, a1;
            if (kp[j] == pre0) {
                a0 = want0 && r0 < rem0;
                ++r0;
            } else {
                a0 = want0 && kp[j] > pre0;
            }
            if (kp[j] == pre1) {
                a1 = want1 && r1 < rem1;
                ++r1;
            } else {
                a1 = want1 && kp[j] > pre1;
            }
            ma |= (a0 ? 1u : 0u) << j;
            mb |= (a1 && !a0 ? 1u : 0u) << j;
        }
    }
    const uint32_t ab = (uint32_t)__builtin_popcount(ma) | ((uint32_t)__builtin_popcount(mb) << 16);
    incl = group_scan(ab, sm.wsum[nscan++ & 1], tid);
    excl = incl - ab;
    int pa = (int)(excl & 0xFFFFu), pb = n1 + (int)(excl >> 16);
    if constexpr (!SORTED) {
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            if ((ma >> j) & 1u) emit(pa++, i0 + j);
            if ((mb >> j) & 1u) emit(pb++, i0 + j);
        }
    } else {
        // the set, in page order, into LDS; then rank each member against it
        int pos[KPT];
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            pos[j] = pa;
            if (((ma >> j) & 1u) && pa < n1) skeys[pa++] = key[j];
        }
        __syncthreads();
        int rank[KPT];
#pragma unroll
        for (int j = 0; j < KPT; ++j) rank[j] = 0;
        for (int m = 0; m < n1; ++m) {
            const uint32_t km = skeys[m];
#pragma unroll
            for (int j = 0; j < KPT; ++j)
                rank[j] += (km > key[j] || (km == key[j] && m < pos[j])) ? 1 : 0;
        }
#pragma unroll
        for (int j = 0; j < KPT; ++j)
            if (((ma >> j) & 1u) && rank[j] < n1) out[rank[j]] = i0 + j;
    }
}

// ---- one threshold, linear bins ----
//
// The selecting decode needs only the n best pages of a row (no second
// threshold, page order).  Its rows' finite scores span a narrow range, so
// bins laid linearly over [min, max] of the finite candidate keys (order
// keys: linear in the key, monotone in the score) put a handful of keys in
// each: one round of histogram and scan finds the threshold bin, and the
// few keys in it are ranked against each other directly.  A round is four
// barriers (extrema, histogram, scan, threshold) against three a radix pass
// plus the prefix stage, and one round usually decides what took the radix
// select a prefix stage and two passes.  Bins: 0 for -inf (pages past the
// end), 2047 for +inf (forced pages), 1..2046 linear.  A threshold bin that
// is too full to rank directly (keys crowded by an outlier stretching the
// range) gets another round over its own range.
constexpr int LIN_BINS = 2048;
constexpr int LIN_LIST = 64;            // a threshold bin this small is ranked directly

struct LinSelectSmem {
    // [round parity][bin]; past the bins, 32 words that take the adds of
    // non-candidate keys (so every lane adds, without a branch)
    uint32_t hist[2][LIN_BINS + 32];
    uint32_t red[2][2][4];              // [round parity][min, max][wave]
    uint32_t wsum[2][4];                // group_scan's wave totals
    int found[2][4];                    // [round parity] bin, taken, its count, outcome
    int list_n;
    int vote[2];                        // [round parity] some group needs another round
    uint32_t list_key[LIN_LIST];        // (0 past list_n: never ahead of a real key)
    int list_page[LIN_LIST];
};

// Min or max over a wave: within each row of 16 lanes by DPP (quad swaps,
// half-row and row mirrors), then the four rows by readlane.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_extreme(uint32_t v) {
    auto op = [](uint32_t x, uint32_t y) { return MAX ? (x > y ? x : y) : (x < y ? x : y); };
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return op(op(r0, r1), op(r2, r3));
}

// The n best pages of a row (n <= P), reported in page order through
// emit(position, page); among equal scores the lower page first (the set
// select_row_k reports for n1 = n, n2 = 0).  Same contract for the group,
// COOP and `fix` as select_row_k; every group of the workgroup passes the
// same barriers (the rounds go on while any group needs another: `vote`,
// two ints in LDS, is the workgroup's, the same for every group).
template <int KPT, class Emit, int COOP = 0, class Fix = NoFix>
__device__ __attribute__((always_inline)) void select_row_lin(const float* srow, int P, int n,
                                                              int tid, LinSelectSmem& sm,
                                                              int* vote, Emit emit,
                                                              Fix fix = Fix()) {
    // (written without per-key branches: selects and bit masks, one branch
    // for the thread that reports the threshold; branchy forms of the same
    // steps measured several times slower, each phase a chain of short
    // divergent blocks)
    static_assert(KPT <= 32, "a thread's keys fit a 32-bit mask");
    constexpr int BPT = LIN_BINS / SEL_THREADS;           // bins a thread scans
    static_assert(BPT == 8, "two 16-byte reads a thread");
    constexpr uint32_t KEY_PINF = 0xFF800000u, KEY_NINF = 0x007FFFFFu;
    enum { OPEN = 0, ALL = 1, NONE = 2, PAGE = 3, LIST = 4 };
    const int i0 = tid * KPT;
    int cnt = P - i0;
    cnt = cnt < 0 ? 0 : (cnt > KPT ? KPT : cnt);
    const uint32_t real = cnt >= 32 ? 0xFFFFFFFFu : (1u << cnt) - 1u;
    const int wv = tid >> 6;
    if (tid == 0) {
        sm.list_n = 0;
        vote[0] = 0;
    }
    if (tid < LIN_LIST) sm.list_key[tid] = 0u;
    *(u4*)&sm.hist[0][tid * BPT] = u4{0u, 0u, 0u, 0u};
    *(u4*)&sm.hist[0][tid * BPT + 4] = u4{0u, 0u, 0u, 0u};
    uint32_t key[KPT];
    select_keys<KPT, COOP>(srow, P, tid, i0, cnt, key, fix);

    // candidates: the keys in [clo, chi]; keys above chi are taken, keys
    // below clo are not, and `rem` of the candidates are taken
    uint32_t clo = 0u, chi = 0xFFFFFFFFu;
    int rem = n;
    int mode = n > 0 ? OPEN : NONE;
    int nscan = 0;
    for (int par = 0;; par ^= 1) {
        uint32_t cm = 0u;                                  // candidate keys
        uint32_t kmn = 0xFFFFFFFFu, kmx = 0u;              // extrema of the finite ones
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint32_t k = key[j];
            const bool c = k >= clo && k <= chi;
            cm |= (c ? 1u : 0u) << j;
            const bool f = c && k != KEY_PINF && k != KEY_NINF && ((real >> j) & 1u);
            const uint32_t lo = f ? k : 0xFFFFFFFFu, hi = f ? k : 0u;
            kmn = lo < kmn ? lo : kmn;
            kmx = hi > kmx ? hi : kmx;
        }
        cm &= mode == OPEN ? real : 0u;
        kmn = wave_extreme<false>(kmn);
        kmx = wave_extreme<true>(kmx);
        if ((tid & 63) == 0) {
            sm.red[par][0][wv] = kmn;
            sm.red[par][1][wv] = kmx;
        }
        __syncthreads();
        if (par == 0) LS_STAMP(13);
        // (the other parity's histogram and vote were last read before this
        // barrier)
        if (tid == 0) vote[par ^ 1] = 0;
        *(u4*)&sm.hist[par ^ 1][tid * BPT] = u4{0u, 0u, 0u, 0u};
        *(u4*)&sm.hist[par ^ 1][tid * BPT + 4] = u4{0u, 0u, 0u, 0u};
        uint32_t fmin = sm.red[par][0][0], fmax = sm.red[par][1][0];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            fmin = sm.red[par][0][w] < fmin ? sm.red[par][0][w] : fmin;
            fmax = sm.red[par][1][w] > fmax ? sm.red[par][1][w] : fmax;
        }
        if (fmin > fmax) fmin = fmax = 0u;                 // no finite candidate
        const uint32_t q = (fmax - fmin) / (uint32_t)(LIN_BINS - 2);
        const int sh = q ? 32 - __builtin_clz(q) : 0;      // (fmax - fmin) >> sh <= 2045
        const int spare = LIN_BINS + (tid & 31);
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint32_t k = key[j];
            uint32_t b = 1u + ((k - fmin) >> sh);
            b = b < (uint32_t)(LIN_BINS - 2) ? b : (uint32_t)(LIN_BINS - 2);
            b = k == KEY_PINF ? (uint32_t)(LIN_BINS - 1) : b;
            b = k == KEY_NINF ? 0u : b;
            atomicAdd(&sm.hist[par][((cm >> j) & 1u) ? (int)b : spare], 1u);
        }
        __syncthreads();
        if (par == 0) LS_STAMP(14);
        // this thread's bins, highest first: 2047 - 8 tid - j
        const u4 b_lo = *(const u4*)&sm.hist[par][LIN_BINS - 8 - tid * BPT];
        const u4 b_hi = *(const u4*)&sm.hist[par][LIN_BINS - 4 - tid * BPT];
        const uint32_t c[BPT] = {b_hi.w, b_hi.z, b_hi.y, b_hi.x, b_lo.w, b_lo.z, b_lo.y, b_lo.x};
        uint32_t tot = 0;
#pragma unroll
        for (int j = 0; j < BPT; ++j) tot += c[j];
        const int scan_par = nscan++ & 1;
        const uint32_t incl = group_scan(tot, sm.wsum[scan_par], tid);
        const uint32_t total = sm.wsum[scan_par][0] + sm.wsum[scan_par][1] +
                               sm.wsum[scan_par][2] + sm.wsum[scan_par][3];
        const uint32_t r = (uint32_t)rem;
        uint32_t acc = incl - tot;
        int fj = -1;
        uint32_t fbefore = 0;
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            const bool hit = acc < r && acc + c[j] >= r;
            fj = hit ? j : fj;
            fbefore = hit ? acc : fbefore;
            acc += c[j];
        }
        if (mode == OPEN && r < total && fj >= 0) {
            const int T = LIN_BINS - 1 - tid * BPT - fj;
            const uint32_t cT = c[fj];
            const int take = rem - (int)fbefore;
            const int out = take == (int)cT                             ? ALL
                            : (T == 0 || T == LIN_BINS - 1 || sh == 0) ? PAGE
                            : cT <= (uint32_t)LIN_LIST                  ? LIST
                                                                        : OPEN;
            sm.found[par][0] = T;
            sm.found[par][1] = take;
            sm.found[par][2] = (int)cT;
            sm.found[par][3] = out;
            if (out == OPEN) vote[par] = 1;
        }
        // (a plain barrier and a word in LDS: __syncthreads_or measured
        // 0.36-0.4 us against 0.08 us for a barrier)
        __syncthreads();
        const bool more = vote[par] != 0;
        if (mode == OPEN) {
            if (r >= total) {
                mode = ALL;                                // every candidate is taken
            } else {
                const int T = sm.found[par][0];
                rem = sm.found[par][1];
                mode = sm.found[par][3];
                // the threshold bin's keys become the candidates
                if (T == LIN_BINS - 1) {
                    clo = KEY_PINF;
                } else if (T == 0) {
                    chi = KEY_NINF;
                } else {
                    // (within the finite extremes: ±inf keys stay outside)
                    clo = fmin + ((uint32_t)(T - 1) << sh);
                    const uint32_t top = clo + ((1u << sh) - 1u);
                    chi = top < fmax ? top : fmax;
                }
            }
        }
        if (!more) break;
    }
    LS_STAMP(5);
    uint32_t am = 0u, cm = 0u;          // keys above; candidates
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const uint32_t k = key[j];
        am |= (k > chi ? 1u : 0u) << j;
        cm |= (k >= clo && k <= chi ? 1u : 0u) << j;
    }
    am &= real;
    cm &= real;
    // the threshold bin's keys ranked against each other: (key, page) pairs
    // listed, each candidate counting the pairs ahead of it
    if (mode == LIST) {
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            if ((cm >> j) & 1u) {
                const int at = atomicAdd(&sm.list_n, 1);
                if (at < LIN_LIST) {            // (the bin holds at most LIN_LIST)
                    sm.list_key[at] = key[j];
                    sm.list_page[at] = i0 + j;
                }
            }
        }
    }
    __syncthreads();
    uint32_t tm = mode == ALL ? cm : 0u;           // candidates taken (ALL, LIST)
    if (mode == LIST) {
        const int ln = sm.list_n < LIN_LIST ? sm.list_n : LIN_LIST;
        // the first eight entries read once, by every thread, into registers
        // (a bin usually holds a few keys): a per-candidate loop of LDS reads
        // serialised one round trip after another across a wave's keys
        // (entries past ln hold key 0: never ahead)
        const u4 lk0 = *(const u4*)&sm.list_key[0], lk1 = *(const u4*)&sm.list_key[4];
        const u4 lp0 = *(const u4*)&sm.list_page[0], lp1 = *(const u4*)&sm.list_page[4];
        const uint32_t lk[8] = {lk0.x, lk0.y, lk0.z, lk0.w, lk1.x, lk1.y, lk1.z, lk1.w};
        const uint32_t lp[8] = {lp0.x, lp0.y, lp0.z, lp0.w, lp1.x, lp1.y, lp1.z, lp1.w};
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            if ((cm >> j) & 1u) {
                const uint32_t k = key[j];
                const int pg = i0 + j;
                int rank = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    rank += (lk[i] > k || (lk[i] == k && (int)lp[i] < pg)) ? 1 : 0;
                for (int i = 8; i < ln; i += 4) {
                    const u4 qk = *(const u4*)&sm.list_key[i];
                    const u4 qp = *(const u4*)&sm.list_page[i];
                    rank += (qk.x > k || (qk.x == k && (int)qp.x < pg)) ? 1 : 0;
                    rank += (qk.y > k || (qk.y == k && (int)qp.y < pg)) ? 1 : 0;
                    rank += (qk.z > k || (qk.z == k && (int)qp.z < pg)) ? 1 : 0;
                    rank += (qk.w > k || (qk.w == k && (int)qp.w < pg)) ? 1 : 0;
                }
                tm |= (rank < rem ? 1u : 0u) << j;
            }
        }
    }
    // positions in page order: keys above and candidates taken before this
    // thread's (PAGE: the first rem candidates in page order)
    const uint32_t xm = mode == PAGE ? cm : tm;
    const uint32_t v = (uint32_t)__builtin_popcount(am) | ((uint32_t)__builtin_popcount(xm) << 16);
    const uint32_t ex = group_scan(v, sm.wsum[nscan++ & 1], tid) - v;
    const int x_ex = (int)(ex >> 16);
    if (mode == PAGE) {
        // candidate j is taken when fewer than rem come before it
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const int before = x_ex + __builtin_popcount(cm & ((1u << j) - 1u));
            tm |= (((cm >> j) & 1u) && before < rem ? 1u : 0u) << j;
        }
    }
    const uint32_t take = am | tm;
    int pos = (int)(ex & 0xFFFFu) + (mode == PAGE ? (x_ex < rem ? x_ex : rem) : x_ex);
#pragma unroll
    for (int j = 0; j < KPT; ++j)
        if ((take >> j) & 1u) emit(pos++, i0 + j);
    LS_STAMP(6);
}

template <bool SORTED, class Emit>
__device__ __attribute__((always_inline)) void select_row(const float* srow, int P, int n1, int n2,
                                                          int tid, int32_t* out, SelectSmem& sm,
                                                          uint32_t* skeys, Emit emit) {
    const int kpt = (P + SEL_THREADS - 1) / SEL_THREADS;
    if (kpt <= 1)
        select_row_k<SORTED, 1>(srow, P, n1, n2, tid, out, sm, skeys, emit);
    else if (kpt <= 2)
        select_row_k<SORTED, 2>(srow, P, n1, n2, tid, out, sm, skeys, emit);
    else if (kpt <= 4)
        select_row_k<SORTED, 4>(srow, P, n1, n2, tid, out, sm, skeys, emit);
    else if (kpt <= 8)
        select_row_k<SORTED, 8>(srow, P, n1, n2, tid, out, sm, skeys, emit);
    else if (kpt <= 16)
        select_row_k<SORTED, 16>(srow, P, n1, n2, tid, out, sm, skeys, emit);
    else
        select_row_k<SORTED, 32>(srow, P, n1, n2, tid, out, sm, skeys, emit);
}

// select_row_lin with the keys a thread holds fitted to the row length.
template <class Emit>
__device__ __attribute__((always_inline)) void select_lin(const float* srow, int P, int n, int tid,
                                                          LinSelectSmem& sm, Emit emit) {
    const int kpt = (P + SEL_THREADS - 1) / SEL_THREADS;
    if (kpt <= 1)
        select_row_lin<1>(srow, P, n, tid, sm, sm.vote, emit);
    else if (kpt <= 2)
        select_row_lin<2>(srow, P, n, tid, sm, sm.vote, emit);
    else if (kpt <= 4)
        select_row_lin<4>(srow, P, n, tid, sm, sm.vote, emit);
    else if (kpt <= 8)
        select_row_lin<8>(srow, P, n, tid, sm, sm.vote, emit);
    else if (kpt <= 16)
        select_row_lin<16>(srow, P, n, tid, sm, sm.vote, emit);
    else
        select_row_lin<32>(srow, P, n, tid, sm, sm.vote, emit);
}

}  // namespace ls
