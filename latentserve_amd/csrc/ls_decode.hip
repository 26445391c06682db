// Paged GQA decode attention for MI355X (gfx950), fp16 and INT8 KV pools,
// dense page walk or a page-subset list.  Replaces the reference's
// kernels/cuda/paged_decode_fp16.cu, paged_decode_int8.cu and
// paged_sparse_fp16.cu:205-364 (one warp per (sequence, split, head), scalar
// FMAs, a separate Triton combine) with one MI355X-shaped kernel:
//
//  * Work unit: a workgroup of NW wavefronts per (sequence, KV head, split).
//    The split owns pages [lo, hi) (pages per split derived on the device
//    from seq_lens, kernels/gqa/paged_decode.py:564-568, so one fixed grid
//    serves a growing sequence under graph replay); wave w of the group
//    walks pages lo+w, lo+w+NW, ...
//  * One page = 16 tokens = the M side of a 16x16x16 f16 MFMA tile.
//      QK:  S^T[16 tok x 16 rows] = K_page[16 x 128] . Q^T[128 x 16], 8 MFMAs.
//           Lane (g = lane>>4, c = lane&15) feeds K row c, channels
//           32j+8g..+8 straight from one 16-byte load; Q^T is the same lanes'
//           channels of query row c, loaded once.
//      PV:  O^T[128 ch x 16 rows] += V^T[128 x 16 tok] . P^T[16 tok x 16 rows],
//           8 MFMAs.  The QK output tile already sits in exactly the layout of
//           P^T's B operand (lane holds row c, tokens 4g..4g+3), so the softmax
//           weights never move between lanes.  V^T's A operand (four tokens of
//           one channel per lane) is assembled from four natural 16-byte row
//           loads with 16 byte-permutes.
//    The 6 query rows of a KV head (GQA 6:1) ride in the N=16 columns: the
//    whole group shares every K/V load, as the reference's fold intends.
//  * Online softmax in the log2 domain: row max over the page = max of a
//    lane's 4 tokens and two cross-group swaps; the running sum l stays
//    lane-partial until the end.  Rescaling the 32 accumulator registers is
//    skipped when no row's max moved (wave-uniform branch).
//  * INT8: K codes become exact fp16 (byte splice, i8x4_to_h4) and K's
//    per-channel scale is folded into the query operand per page; V's
//    per-token scale is folded into the softmax weights (as the reference
//    does, paged_decode_int8.cu:230-242).  The sequence's last page takes K
//    from the fp16 residual (paged_decode.py:213-216).
//  * Page prefetch: the next page's K/V (and scales) are issued before the
//    current page is computed (two register buffers).
//  * Splits: NW waves merge in LDS; with more than one split, every group
//    writes (m, l, acc) partials in the reference's layout ([B,H,S,NR,D],
//    [B,H,S,NR], m in natural-log units) and the last group to finish a
//    (sequence, head) merges them (combine_splits, paged_decode.py:689-706)
//    and resets its arrival counter, so the path is one launch and safe to
//    replay in a captured graph.

#include <stdlib.h>
#include <string.h>

#include "ls_common.h"
#include "ls_decode.h"

namespace ls {

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// LDS scratch of combine_partials.
constexpr int CMB_CHUNK = 64;   // splits whose weights are staged at once
struct CombineSmem {
    float red[16][MAX_NREP];            // per-thread-group partial max / sum
    float mg[MAX_NREP];                 // row max over all splits
    float lt[MAX_NREP];                 // row sum of weighted l
    float w[CMB_CHUNK][MAX_NREP];       // weights of the current chunk of splits
};


template <int NW>
struct DecodeSmem {
    float m[NW][MAX_NREP];
    float l[NW][MAX_NREP];
    union {
        float acc[NW][MAX_NREP][HEAD_DIM];   // wave states, merged once
        CombineSmem cmb;                     // then reused by the split combine
    };
    int is_last;
};

// Registers of one page for one wave.  K/V as raw dwords; INT8 rows are half
// as wide and use the low 2 dwords of each slot.
struct PageBuf {
    u4 k[4];      // K row `c`, channels 32j+8g..+8   (fp16: 16 B, int8: 8 B)
    u4 v[4];      // V row 4g+i, channels 8c..8c+8     (fp16: 16 B, int8: 8 B)
    f4 ks[4][2];  // INT8: K scale of the same channels (32 B per j)
    f4 kz[4][2];  // INT8 asym: K zero points
    float vs[4];  // INT8: V scale of tokens 4g+i
    float vz[4];  // INT8 asym: V zero points
    int res;      // INT8: this page's K comes from the residual
};

template <int KIND, bool ASYM, bool HAS_RES>
__device__ __forceinline__ void load_page(const DecodeParams& a, PageBuf& buf, int blk, int page,
                                          int num_pages, int b, int h, int g, int c) {
    const int64_t base = (int64_t)blk * a.sk_b + (int64_t)h * a.sk_h;
    if (KIND == KV_FP16) {
        const half_t* kp = (const half_t*)a.k_pool + base + (int64_t)c * a.sk_p + 8 * g;
        const half_t* vp = (const half_t*)a.v_pool + base + (int64_t)(4 * g) * a.sk_p + 8 * c;
#pragma unroll
        for (int j = 0; j < 4; ++j) buf.k[j] = *(const u4*)(kp + 32 * j);
#pragma unroll
        for (int i = 0; i < 4; ++i) buf.v[i] = *(const u4*)(vp + (int64_t)i * a.sk_p);
    } else {
        buf.res = HAS_RES && page == num_pages - 1;
        const int8_t* vp = (const int8_t*)a.v_pool + base + (int64_t)(4 * g) * a.sk_p + 8 * c;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u2 t = *(const u2*)(vp + (int64_t)i * a.sk_p);
            buf.v[i].x = t.x;
            buf.v[i].y = t.y;
        }
        const float* vsp = a.v_scale + (int64_t)blk * a.svs_b + (int64_t)(4 * g) * a.svs_p +
                           (int64_t)h * a.svs_h;
#pragma unroll
        for (int i = 0; i < 4; ++i) buf.vs[i] = vsp[(int64_t)i * a.svs_p];
        if (ASYM) {
            const float* vzp = a.v_zero + (int64_t)blk * a.svs_b + (int64_t)(4 * g) * a.svs_p +
                               (int64_t)h * a.svs_h;
#pragma unroll
            for (int i = 0; i < 4; ++i) buf.vz[i] = vzp[(int64_t)i * a.svs_p];
        }
        if (HAS_RES && buf.res) {
            const half_t* kp = a.k_res + (int64_t)a.res_rows[b] * a.sr_r + (int64_t)c * a.sr_p +
                               (int64_t)h * a.sr_h + 8 * g;
#pragma unroll
            for (int j = 0; j < 4; ++j) buf.k[j] = *(const u4*)(kp + 32 * j);
        } else {
            const int8_t* kp = (const int8_t*)a.k_pool + base + (int64_t)c * a.sk_p + 8 * g;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u2 t = *(const u2*)(kp + 32 * j);
                buf.k[j].x = t.x;
                buf.k[j].y = t.y;
            }
            const float* ksp = a.k_scale + (int64_t)blk * a.sks_b + (int64_t)h * a.sks_h + 8 * g;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                buf.ks[j][0] = *(const f4*)(ksp + 32 * j);
                buf.ks[j][1] = *(const f4*)(ksp + 32 * j + 4);
            }
            if (ASYM) {
                const float* kzp = a.k_zero + (int64_t)blk * a.sks_b + (int64_t)h * a.sks_h + 8 * g;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    buf.kz[j][0] = *(const f4*)(kzp + 32 * j);
                    buf.kz[j][1] = *(const f4*)(kzp + 32 * j + 4);
                }
            }
        }
    }
}

struct WaveState {
    f4 acc[8];   // O^T tiles: lane holds row c, channels 32g + 8i + jj (tile jj, element i)
    float m;     // running max of row c, log2 units, identical in the 4 lanes of row c
    float l;     // lane-partial running sum of this lane's tokens' weights
    float z;     // INT8 asym: lane-partial running sum of p * v_zero
};

template <int KIND, bool ASYM>
__device__ __forceinline__ void compute_page(const PageBuf& buf, WaveState& st, const h4 (&qh)[8],
                                             const float (&qf)[4][8], int page, int len,
                                             float scale_log2, int g) {
    // ---- S^T = K . Q^T ----
    f4 s = {0.f, 0.f, 0.f, 0.f};
    float qz = 0.f;
    if (KIND == KV_FP16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s = mfma16(as_h4(buf.k[j].x, buf.k[j].y), qh[2 * j], s);
            s = mfma16(as_h4(buf.k[j].z, buf.k[j].w), qh[2 * j + 1], s);
        }
    } else {
        if (buf.res) {
            // Exact fp16 K from the residual: the unscaled query.
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s = mfma16(as_h4(buf.k[j].x, buf.k[j].y), qh[2 * j], s);
                s = mfma16(as_h4(buf.k[j].z, buf.k[j].w), qh[2 * j + 1], s);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u2 lo = i8x4_to_h4(buf.k[j].x);
                const u2 hi = i8x4_to_h4(buf.k[j].y);
                h4 q0, q1;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    q0[e] = (half_t)(qf[j][e] * buf.ks[j][0][e]);
                    q1[e] = (half_t)(qf[j][4 + e] * buf.ks[j][1][e]);
                    if (ASYM) qz += qf[j][e] * buf.kz[j][0][e] + qf[j][4 + e] * buf.kz[j][1][e];
                }
                s = mfma16(as_h4(lo.x, lo.y), q0, s);
                s = mfma16(as_h4(hi.x, hi.y), q1, s);
            }
            if (ASYM) qz = group4_sum(qz);
        }
    }

    // ---- online softmax over this page (rows = c, tokens 4g+i) ----
    const int tok0 = page * PAGE + 4 * g;
    float x[4];
    float mloc = neg_inf();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[i] = tok0 + i < len ? (s[i] + qz) * scale_log2 : neg_inf();
        mloc = fmaxf(mloc, x[i]);
    }
    const float m_new = fmaxf(st.m, group4_max(mloc));
    const bool dead = m_new == neg_inf();      // nothing valid yet in this row
    const float alpha = dead ? 0.f : fast_exp2(st.m - m_new);
    float p[4];
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        p[i] = dead ? 0.f : fast_exp2(x[i] - m_new);
        psum += p[i];
    }
    st.l = st.l * alpha + psum;
    st.m = m_new;
    if (__any(alpha != 1.f)) {
#pragma unroll
        for (int t = 0; t < 8; ++t) st.acc[t] *= alpha;
        if (ASYM) st.z *= alpha;
    }

    // ---- O^T += V^T . P^T ----
    h4 pb;
    if (KIND == KV_FP16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) pb[i] = (half_t)p[i];
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) pb[i] = (half_t)(p[i] * buf.vs[i]);
        if (ASYM) {
#pragma unroll
            for (int i = 0; i < 4; ++i) st.z += p[i] * buf.vz[i];
        }
    }
    // Rows of V as fp16 pairs: vr[i][kk] = channels (8c+2kk, 8c+2kk+1) of token 4g+i.
    uint32_t vr[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (KIND == KV_FP16) {
            vr[i][0] = buf.v[i].x;
            vr[i][1] = buf.v[i].y;
            vr[i][2] = buf.v[i].z;
            vr[i][3] = buf.v[i].w;
        } else {
            const u2 lo = i8x4_to_h4(buf.v[i].x);
            const u2 hi = i8x4_to_h4(buf.v[i].y);
            vr[i][0] = lo.x;
            vr[i][1] = lo.y;
            vr[i][2] = hi.x;
            vr[i][3] = hi.y;
        }
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        // channel 8c+2kk (low halves) and 8c+2kk+1 (high halves) of tokens 4g..4g+3
        const uint32_t e0 = __builtin_amdgcn_perm(vr[1][kk], vr[0][kk], 0x05040100u);
        const uint32_t e1 = __builtin_amdgcn_perm(vr[3][kk], vr[2][kk], 0x05040100u);
        const uint32_t o0 = __builtin_amdgcn_perm(vr[1][kk], vr[0][kk], 0x07060302u);
        const uint32_t o1 = __builtin_amdgcn_perm(vr[3][kk], vr[2][kk], 0x07060302u);
        st.acc[2 * kk] = mfma16(as_h4(e0, e1), pb, st.acc[2 * kk]);
        st.acc[2 * kk + 1] = mfma16(as_h4(o0, o1), pb, st.acc[2 * kk + 1]);
    }
}

// Merge S partial states of one (b, h) into out: combine_splits
// (kernels/gqa/paged_decode.py:689-706).  256 threads.  Thread t owns row
// r = t & 15 of split group t >> 4 for the weight passes, and float4 columns
// of the output for the accumulation; every global load of a pass is issued
// before any is consumed, so a pass costs one memory round trip rather than
// one per split.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool COH>
__device__ __forceinline__ float load_part(const float* p) {
    if (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *p;
}

template <int VEC, bool COH = false>
__device__ void combine_partials(const float* acc, const float* m, const float* l, int S, int NR,
                                 int64_t sa_s, int64_t sa_r, int64_t sm_s, void* out, int out_f32,
                                 int64_t so_r, int tid, CombineSmem& cs) {
    const int r = tid & 15, grp = tid >> 4;
    const bool row_ok = r < NR;
    // pass 1: row max
    float mx = neg_inf();
    if (row_ok)
        for (int s = grp; s < S; s += 16) mx = fmaxf(mx, load_part<COH>(m + s * sm_s + r));
    cs.red[grp][r] = mx;
    __syncthreads();
    if (tid < MAX_NREP) {
        float v = neg_inf();
#pragma unroll
        for (int i = 0; i < 16; ++i) v = fmaxf(v, cs.red[i][tid]);
        cs.mg[tid] = v;
    }
    __syncthreads();
    const float mgr = cs.mg[r];
    const bool dead = mgr == neg_inf();

    // pass 2: weights chunk by chunk, accumulating the output columns
    constexpr int NV = HEAD_DIM / VEC;                        // vectors per row
    constexpr int MAXO = (MAX_NREP * NV + 255) / 256;         // outputs per thread
    const int n_out = NR * NV;
    f4 accv[MAXO];
#pragma unroll
    for (int i = 0; i < MAXO; ++i) accv[i] = (f4){0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
    for (int s0 = 0; s0 < S; s0 += CMB_CHUNK) {
        const int n = S - s0 < CMB_CHUNK ? S - s0 : CMB_CHUNK;
        for (int i = grp; i < n; i += 16) {
            float w = 0.f;
            if (row_ok && !dead) {
                w = __expf(load_part<COH>(m + (s0 + i) * sm_s + r) - mgr);
                lsum += load_part<COH>(l + (s0 + i) * sm_s + r) * w;
            }
            cs.w[i][r] = w;
        }
        __syncthreads();
#pragma unroll
        for (int oi = 0; oi < MAXO; ++oi) {
            const int o = tid + 256 * oi;
            if (o < n_out) {
                const int orow = o / NV, col = (o % NV) * VEC;
                const float* src = acc + (int64_t)s0 * sa_s + orow * sa_r + col;
                f4 a4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 16
                for (int i = 0; i < n; ++i) {
                    const float w = cs.w[i][orow];
                    if (VEC == 4) {
                        a4 += w * *(const f4*)(src + i * sa_s);
                    } else {
                        a4[0] += w * load_part<COH>(src + i * sa_s);
                    }
                }
                accv[oi] += a4;
            }
        }
        __syncthreads();
    }
    // row sums of the weighted l
    cs.red[grp][r] = lsum;
    __syncthreads();
    if (tid < MAX_NREP) {
        float v = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) v += cs.red[i][tid];
        cs.lt[tid] = v;
    }
    __syncthreads();
#pragma unroll
    for (int oi = 0; oi < MAXO; ++oi) {
        const int o = tid + 256 * oi;
        if (o < n_out) {
            const int orow = o / NV, col = (o % NV) * VEC;
            const float inv = 1.f / fmaxf(cs.lt[orow], 1e-20f);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float v = accv[oi][e] * inv;
                if (out_f32)
                    ((float*)out)[orow * so_r + col + e] = v;
                else
                    ((half_t*)out)[orow * so_r + col + e] = (half_t)v;
            }
        }
    }
}

template <int KIND, bool ASYM, bool HAS_RES, bool SPARSE, int NW>
__global__ __launch_bounds__(WAVE* NW) void paged_decode_kernel(const DecodeParams a) {
    // Pages in flight ahead of the one being computed: the fp16 page buffer
    // is 32 VGPRs, the INT8 one (codes + K scales) as large again.
    constexpr int PF_DEPTH = KIND == KV_FP16 ? 2 : 1;
    __shared__ DecodeSmem<NW> sm;
    const int H = a.H;
    const int h = blockIdx.x % H;
    const int split = blockIdx.x / H;
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const int w = tid / WAVE;
    const int lane = tid % WAVE;
    const int g = lane >> 4, c = lane & 15;
    const int S = a.num_splits;

    const int len = a.seq_lens[b];
    int num_pages = (len + PAGE - 1) / PAGE;
    num_pages = num_pages < a.max_pages ? num_pages : a.max_pages;
    bool res_ok = false;
    if (HAS_RES) {
        const int rr = a.res_rows[b];
        res_ok = rr >= 0 && rr < a.res_cap;
    }

    // This split's slice of the page walk (dense) or of the selection list.
    int n_list = num_pages;
    const int32_t* sel = nullptr;
    if (SPARSE) {
        sel = a.sel + (int64_t)b * a.ssel_b + (int64_t)h * a.ssel_h;
        n_list = a.num_sel;
        if (a.ratio > 0.f) {
            int want;
            if (a.ratio >= 1.f) {
                want = num_pages;
            } else {
                want = (int)ceilf(a.ratio * (float)num_pages);
                want = want > a.recent + 1 ? want : a.recent + 1;
            }
            want = want < num_pages ? want : num_pages;
            n_list = want < a.num_sel ? want : a.num_sel;
        }
    }
    const int per = (n_list + S - 1) / S;
    const int lo = split * per;
    const int hi = lo + per < n_list ? lo + per : n_list;

    // Query operand: row c (zero beyond n_rep), channels 32j+8g..+8.
    h4 qh[8];
    float qf[4][8];
    {
        const bool row_ok = c < a.NR;
        const half_t* qp = a.q + (int64_t)b * a.sq_b + (int64_t)h * a.sq_h + (int64_t)c * a.sq_r + 8 * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u4 t = {0u, 0u, 0u, 0u};
            if (row_ok) t = *(const u4*)(qp + 32 * j);
            qh[2 * j] = as_h4(t.x, t.y);
            qh[2 * j + 1] = as_h4(t.z, t.w);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qf[j][e] = (float)qh[2 * j][e];
                qf[j][4 + e] = (float)qh[2 * j + 1][e];
            }
        }
    }
    const float scale_log2 = a.scale * LOG2E;

    WaveState st;
#pragma unroll
    for (int t = 0; t < 8; ++t) st.acc[t] = (f4){0.f, 0.f, 0.f, 0.f};
    st.m = neg_inf();
    st.l = 0.f;
    st.z = 0.f;

    // Wave w walks entries lo+w, lo+w+NW, ... in chunks of 64: lane i of the
    // chunk resolves entry i to (logical page, physical block) once, and the
    // page loop reads them back with readlane (no per-page table latency).
    const int first = lo + w;
    const int count = first < hi ? (hi - first + NW - 1) / NW : 0;
    for (int base = 0; base < count; base += WAVE) {
        const int n_chunk = count - base < WAVE ? count - base : WAVE;
        int pg = -1, blk = 0;
        if (lane < n_chunk) {
            const int e = first + (base + lane) * NW;
            pg = SPARSE ? sel[e] : e;
            if (pg >= 0 && pg < num_pages) {
                blk = a.block_tables[(int64_t)b * a.sbt_b + pg];
                // Ids outside the pool, and a last page whose residual row is
                // outside the residual, are never dereferenced.
                if (blk < 0 || blk >= a.num_blocks) pg = -1;
                if (HAS_RES && pg == num_pages - 1 && !res_ok) pg = -1;
            } else {
                pg = -1;
            }
        }
        // Compact the valid entries to the front (a page-subset list pads
        // short sequences with pages past their end, paged_sparse_fp16.cu:266).
        const uint64_t mask = __ballot(pg >= 0);
        const int n_valid = __popcll(mask);
        if (mask != ~0ull) {
            const int before = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
            const int dst = pg >= 0 ? before : n_valid + (lane - before);
            pg = __builtin_amdgcn_ds_permute(dst << 2, pg);
            blk = __builtin_amdgcn_ds_permute(dst << 2, blk);
        }
        if (n_valid == 0) continue;

        // Three page buffers in rotation: pages k+1 and k+2 are in flight
        // while page k is computed.  Prefetches past the end re-read the
        // last page (a cache hit) so every iteration waits the same way.
        PageBuf buf[PF_DEPTH + 1];
        const int last = n_valid - 1;
#pragma unroll
        for (int u = 0; u < PF_DEPTH; ++u) {
            const int kk = u < last ? u : last;
            load_page<KIND, ASYM, HAS_RES>(a, buf[u], __builtin_amdgcn_readlane(blk, kk),
                                           __builtin_amdgcn_readlane(pg, kk), num_pages, b, h, g, c);
        }
        for (int k = 0; k < n_valid;) {
#pragma unroll
            for (int u = 0; u <= PF_DEPTH; ++u) {
                const int kn = k + PF_DEPTH < last ? k + PF_DEPTH : last;
                load_page<KIND, ASYM, HAS_RES>(a, buf[(u + PF_DEPTH) % (PF_DEPTH + 1)],
                                               __builtin_amdgcn_readlane(blk, kn),
                                               __builtin_amdgcn_readlane(pg, kn), num_pages, b, h,
                                               g, c);
                compute_page<KIND, ASYM>(buf[u], st, qh, qf, __builtin_amdgcn_readlane(pg, k), len,
                                         scale_log2, g);
                if (++k >= n_valid) break;
            }
        }
    }

    // ---- merge the NW waves in LDS ----
    const float lrow = group4_sum(st.l);
    if (ASYM) {
        const float zrow = group4_sum(st.z);
#pragma unroll
        for (int t = 0; t < 8; ++t) st.acc[t] += zrow;
    }
    if (g == 0) {
        sm.m[w][c] = st.m;
        sm.l[w][c] = lrow;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.acc[w][c][32 * g + 8 * i + t] = st.acc[t][i];
    __syncthreads();

    const int NR = a.NR;
    const bool single = S == 1;
    const int64_t bh = (int64_t)b * H + h;
    float* pacc = a.part_acc + (bh * S + split) * (int64_t)NR * HEAD_DIM;
    float* pm = a.part_m + (bh * S + split) * NR;
    float* pl = a.part_l + (bh * S + split) * NR;
    for (int idx = tid; idx < NR * HEAD_DIM; idx += WAVE * NW) {
        const int r = idx / HEAD_DIM, d = idx % HEAD_DIM;
        float mg = neg_inf();
#pragma unroll
        for (int u = 0; u < NW; ++u) mg = fmaxf(mg, sm.m[u][r]);
        float lt = 0.f, at = 0.f;
#pragma unroll
        for (int u = 0; u < NW; ++u) {
            const float wt = mg == neg_inf() ? 0.f : fast_exp2(sm.m[u][r] - mg);
            lt += sm.l[u][r] * wt;
            at += sm.acc[u][r][d] * wt;
        }
        if (single) {
            a.out[(int64_t)b * a.so_b + (int64_t)h * a.so_h + (int64_t)r * a.so_r + d] =
                (half_t)(at / fmaxf(lt, 1e-20f));
        } else if (a.fuse) {
            // Device-coherent (write-through) stores: the group that merges
            // may run on another XCD, whose L2 does not see this one's.
            store_coherent(pacc + idx, at);
            if (d == 0) {
                store_coherent(pm + r, mg * LN2);   // natural-log units, the reference's format
                store_coherent(pl + r, lt);
            }
        } else {
            pacc[idx] = at;
            if (d == 0) {
                pm[r] = mg * LN2;
                pl[r] = lt;
            }
        }
    }
    if (single || !a.fuse) return;

    // ---- the last group of this (b, h) to arrive merges all splits ----
    // The partials above bypass the non-coherent L2 path, so ordering needs
    // only their completion before the arrival count: no whole-L2 writeback
    // or invalidate (which a device-scope fence would issue in every group).
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
        const int prev = __hip_atomic_fetch_add(a.counters + bh, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        sm.is_last = prev == S - 1;
    }
    __syncthreads();
    if (!sm.is_last) return;
    static_assert(WAVE * NW == 256, "the fused combine is written for 256 threads");
    combine_partials<1, true>(a.part_acc + bh * S * (int64_t)NR * HEAD_DIM, a.part_m + bh * S * NR,
                              a.part_l + bh * S * NR, S, NR, (int64_t)NR * HEAD_DIM, HEAD_DIM, NR,
                              a.out + (int64_t)b * a.so_b + (int64_t)h * a.so_h, 0, a.so_r, tid,
                              sm.cmb);
    if (tid == 0)
        __hip_atomic_store(a.counters + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int VEC>
__global__ __launch_bounds__(256) void combine_kernel(CombineParams p) {
    __shared__ CombineSmem cs;
    const int bh = blockIdx.x;
    const int b = bh / p.H, h = bh % p.H;
    combine_partials<VEC>(p.acc + (int64_t)b * p.sa_b + (int64_t)h * p.sa_h,
                          p.m + (int64_t)b * p.sm_b + (int64_t)h * p.sm_h,
                          p.l + (int64_t)b * p.sm_b + (int64_t)h * p.sm_h, p.S, p.NR, p.sa_s,
                          p.sa_r, p.sm_s,
                          (char*)p.out + ((int64_t)b * p.so_b + (int64_t)h * p.so_h) *
                                             (p.out_f32 ? 4 : 2),
                          p.out_f32, p.so_r, threadIdx.x, cs);
}

// ------------------------------------------------------------- launch ----

constexpr int NWAVES = 4;

template <int KIND, bool ASYM, bool HAS_RES, bool SPARSE>
static hipError_t launch_t(const DecodeParams& a, hipStream_t stream) {
    dim3 grid(a.num_splits * a.H, a.B);
    hipLaunchKernelGGL((paged_decode_kernel<KIND, ASYM, HAS_RES, SPARSE, NWAVES>), grid,
                       dim3(WAVE * NWAVES), 0, stream, a);
    return hipGetLastError();
}

static hipError_t launch_kernel(const DecodeParams& a, hipStream_t stream) {
    if (a.sel) return launch_t<KV_FP16, false, false, true>(a, stream);
    if (a.kind == KV_FP16) return launch_t<KV_FP16, false, false, false>(a, stream);
    const bool asym = a.k_zero != nullptr, res = a.k_res != nullptr;
    if (asym && res) return launch_t<KV_INT8, true, true, false>(a, stream);
    if (asym) return launch_t<KV_INT8, true, false, false>(a, stream);
    if (res) return launch_t<KV_INT8, false, true, false>(a, stream);
    return launch_t<KV_INT8, false, false, false>(a, stream);
}

// LATENTSERVE_HIP_COMBINE=separate merges the splits in a second launch
// instead of in the decode kernel's last-arriving group (for comparison).
static bool fused_combine() {
    static const int fused = [] {
        const char* e = getenv("LATENTSERVE_HIP_COMBINE");
        return (e && strcmp(e, "separate") == 0) ? 0 : 1;
    }();
    return fused != 0;
}

hipError_t launch_decode(const DecodeParams& a_in, hipStream_t stream) {
    DecodeParams a = a_in;
    a.fuse = fused_combine() ? 1 : 0;
    hipError_t e = launch_kernel(a, stream);
    if (e != hipSuccess || a.fuse || a.num_splits == 1) return e;
    CombineParams p;
    p.acc = a.part_acc;
    p.sa_r = HEAD_DIM;
    p.sa_s = (int64_t)a.NR * HEAD_DIM;
    p.sa_h = p.sa_s * a.num_splits;
    p.sa_b = p.sa_h * a.H;
    p.m = a.part_m;
    p.l = a.part_l;
    p.sm_s = a.NR;
    p.sm_h = (int64_t)a.NR * a.num_splits;
    p.sm_b = p.sm_h * a.H;
    p.out = a.out;
    p.out_f32 = 0;
    p.so_b = a.so_b;
    p.so_h = a.so_h;
    p.so_r = a.so_r;
    p.B = a.B;
    p.H = a.H;
    p.S = a.num_splits;
    p.NR = a.NR;
    return launch_combine(p, stream);
}

hipError_t launch_combine(const CombineParams& p, hipStream_t stream) {
    // float4 partial loads when every row and split starts 16-byte aligned
    const bool vec = ((uintptr_t)p.acc % 16 == 0) && p.sa_b % 4 == 0 && p.sa_h % 4 == 0 &&
                     p.sa_s % 4 == 0 && p.sa_r % 4 == 0;
    if (vec)
        hipLaunchKernelGGL(combine_kernel<4>, dim3(p.B * p.H), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(combine_kernel<1>, dim3(p.B * p.H), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace ls
