// Top-k page selection over a row of page scores, for a group of 256
// threads: shared by the selection kernel (one group a row) and the sparse
// decode kernel's selecting prologue (one group a head of its workgroup).
//
// A radix select (8-bit digits, LDS histograms, up to 4 passes: it stops
// once the threshold digit's bin is taken whole) finds the n-th largest
// key of the row; the selected pages are reported in page order,
// ties at the threshold taken in page order (deterministic).  Reference:
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
template <bool SORTED, int KPT, class Emit>
__device__ __attribute__((always_inline)) void select_row_k(const float* srow, int P, int n1,
                                                            int n2, int tid, int32_t* out,
                                                            SelectSmem& sm, uint32_t* skeys,
                                                            Emit emit) {
    const int i0 = tid * KPT;
    int cnt = P - i0;
    cnt = cnt < 0 ? 0 : (cnt > KPT ? KPT : cnt);
    uint32_t key[KPT];
    {
        // unconditional loads (clamped index) so they all issue back to back
        float f[KPT];
        const int last = P > 0 ? P - 1 : 0;
#pragma unroll
        for (int j = 0; j < KPT; ++j) f[j] = P > 0 ? srow[i0 + j < last ? i0 + j : last] : 0.f;
#pragma unroll
        for (int j = 0; j < KPT; ++j) key[j] = j < cnt ? order_key(f[j]) : 0u;
    }

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
                if ((key[j] & msk) == pre1) {
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

}  // namespace ls
