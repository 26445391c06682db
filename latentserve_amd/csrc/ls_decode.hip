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
//    per-channel scale is folded into the query operand per page (the
//    512-byte scale row is loaded 8 bytes a lane and handed to the 16 lanes
//    that use each channel through a per-wave LDS slot); V's
//    per-token scale is folded into the softmax weights (as the reference
//    does, paged_decode_int8.cu:230-242).  The sequence's last page takes K
//    from the fp16 residual (paged_decode.py:213-216).
//  * Page prefetch: the next page's K/V (and scales) are issued before the
//    current page is computed (two buffers).  fp16 K rows go through LDS
//    (whole-line direct loads into a per-wave slot, read back in the MFMA
//    layout), V and every INT8 row straight to registers.
//  * Splits: NW waves merge in LDS; with more than one split, every group
//    writes its (acc, m, l) record (acc [NR][128] as the reference's
//    partials hold it, then each row's m, in natural-log units as the
//    reference's, beside its l) and the last group to finish a (sequence,
//    head) merges them (combine_splits, paged_decode.py:689-706) and resets
//    its arrival counter, so the path is one launch and safe to replay in a
//    captured graph.

#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "ls_common.h"
#include "ls_decode.h"
#include "ls_select.h"
#include "ls_quest.h"

namespace ls {

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

constexpr int SCALE_ROW = HEAD_DIM + PAGE;

template <int NWT, int HG, bool SCALES>
struct DecodeSmem {
    // During the walk the merge buffer holds the group's item table: the
    // block of every page of its range (dense walk, shared by the heads) or,
    // per head, the block and page of every list entry (page-subset walk).
    // Rows of the wave states are padded by 16 bytes so that the 16 rows a
    // wave writes at once fall in different banks.
    // The table has its own space so that a wave can store its state the
    // moment its walk ends, while the others still resolve items.
    static constexpr int ROW = HEAD_DIM + 4;
    static constexpr int ENT_INTS = 2048 * HG;
    static constexpr int NWH = NWT / HG;     // waves a head
    float m[HG][NWH][MAX_NREP];
    float l[HG][NWH][MAX_NREP];
    // INT8: each wave's K scale (and zero point) row of the page it computes,
    // then its 16 tokens' V scales (and zero points)
    float kscale[SCALES ? NWT : 1][2][SCALE_ROW];
    // 16-byte aligned, so the state rows move as ds_write_b128 / ds_read_b128
    // (at the struct's default 4-byte alignment they split into ds_*2_b32
    // pairs: twice the LDS instructions, in a bank pattern the padding does
    // not spread)
    alignas(16) float acc[HG][NWH][MAX_NREP][ROW];
    int ent[ENT_INTS];
    int is_last[HG];
    int claim[HG];
};

// Registers of one page for one wave.  K/V as raw dwords; INT8 rows are half
// as wide and use the low 2 dwords of each slot.
struct PageBuf {
    u4 k[4];      // K row `c`: fp16 channels 32j+8g..+8 (16 B each); int8 channels
                  // 64j+16g..+16 in k[0..1] (16 B each), the fp16 residual's
                  // the same channels in k[2j], k[2j+1]
    u4 v[4];      // V row 4g+i, channels 8c..8c+8     (fp16: 16 B, int8: 8 B)
    u2 ks;        // INT8: K scales of channels 2*lane, 2*lane+1 (the row is 512 B)
    u2 kz;        // INT8 asym: K zero points, as ks
    float vs;     // INT8: V scale of token c (the lane group g = 0 covers the page)
    float vz;     // INT8 asym: V zero point of token c
    int res;      // INT8: this page's K comes from the residual
};

// An fp16 page's K rows (16 x 256 bytes of one head) are brought to a 4 KB
// LDS slot of the wave by direct loads, each a whole 256-byte row to 16
// lanes (four rows a load instruction), and read back in the MFMA layout
// (row c per lane): loaded straight to registers in that layout, every load
// instruction covers 64 bytes of each of 16 rows, half of each cache line,
// and a read-only probe of the B16 x 16K pages ran 46.5 us that way against
// 42.5 us through LDS.  Within a row the sixteen 16-byte pieces are stored
// XOR-permuted by the row (piece p holds piece p ^ row), so the 16 lanes
// that read one piece of 16 rows hit 16 different bank groups.
constexpr int KSLOT_BYTES = PAGE * HEAD_DIM * 2;
typedef __attribute__((address_space(3))) void* lds_ptr;
// Vector memory instructions of one fp16 page request: 4 direct K loads, 4 V.
constexpr int FP16_PAGE_VM = 8;

template <int KIND, bool ASYM, bool HAS_RES>
__device__ __forceinline__ void load_page(const DecodeParams& a, PageBuf& buf, int blk, int page,
                                          int num_pages, int res_row, int h, int g, int c,
                                          bool fetch = true, char* kslot = nullptr) {
    // (blk and h are the same in every lane: the wave's item)
    const int64_t base = (int64_t)blk * a.sk_b + (int64_t)h * a.sk_h;
    if (KIND == KV_FP16) {
        const __amdgpu_buffer_rsrc_t rk = page_rsrc((const half_t*)a.k_pool + base, fetch);
        const __amdgpu_buffer_rsrc_t rv = page_rsrc((const half_t*)a.v_pool + base, fetch);
        const int vo = (int)(((int64_t)(4 * g) * a.sk_p + 8 * c) * sizeof(half_t));
        const int row = (int)(a.sk_p * sizeof(half_t));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // lanes (g, c): row 4i + g, LDS piece c <- the row's piece c ^ row
            const int r = 4 * i + g;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr)(kslot + 1024 * i), 16,
                                                     r * row + ((c ^ r) << 4), 0, 0, PAGE_POLICY);
            issue_here();
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            buf.v[i] = page_load16(rv, vo + i * row);
            issue_here();
        }
    } else {
        buf.res = HAS_RES && page == num_pages - 1;
        const __amdgpu_buffer_rsrc_t rv = page_rsrc((const int8_t*)a.v_pool + base, fetch);
        const int vo = (int)((int64_t)(4 * g) * a.sk_p + 8 * c);
        const int row = (int)a.sk_p;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u2 t = page_load8(rv, vo + i * row);
            buf.v[i].x = t.x;
            buf.v[i].y = t.y;
        }
        // the page's 16 V scales in one load (lanes of token c share an
        // address), spread to the lanes that need them through LDS
        // (the scale rows as the K/V codes: the page's base in scalar
        // registers, the page policy; plain loads had cost 0.75 us at
        // B16 x 16K)
        const int64_t vsb = (int64_t)blk * a.svs_b + (int64_t)h * a.svs_h;
        const int vso = (int)(c * a.svs_p * (int64_t)sizeof(float));
        buf.vs = page_load4(page_rsrc(a.v_scale + vsb, fetch), vso);
        if (ASYM) buf.vz = page_load4(page_rsrc(a.v_zero + vsb, fetch), vso);
        // K channels in the INT8 order: lane (c, g) takes 16 contiguous
        // channels 64j+16g.. of token c per load, so one load instruction
        // covers 64 bytes of each of 16 token rows (8 bytes a lane would
        // cover 32 and need twice the cache-line requests per byte, which
        // caps the walk below the HBM rate)
        if (HAS_RES && buf.res) {
            const half_t* kp = a.k_res + (int64_t)res_row * a.sr_r + (int64_t)c * a.sr_p +
                               (int64_t)h * a.sr_h + 16 * g;
#pragma unroll
            for (int j = 0; j < 4; ++j) buf.k[j] = *(const u4*)(kp + 64 * (j / 2) + 8 * (j % 2));
        } else {
            const __amdgpu_buffer_rsrc_t rk = page_rsrc((const int8_t*)a.k_pool + base, fetch);
            const int ko = (int)((int64_t)c * a.sk_p + 16 * g);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                buf.k[j] = page_load16(rk, ko + 64 * j);
            }
            // One coalesced 512-byte row per page, 8 bytes a lane; the
            // compute step spreads it through LDS to the lanes that need
            // each channel (16 lanes share every scale).
            const int lane = 16 * g + c;
            const float* ksp = a.k_scale + (int64_t)blk * a.sks_b + (int64_t)h * a.sks_h;
            buf.ks = page_load8(page_rsrc(ksp, fetch), 8 * lane);
            if (ASYM) {
                const float* kzp = a.k_zero + (int64_t)blk * a.sks_b + (int64_t)h * a.sks_h;
                buf.kz = page_load8(page_rsrc(kzp, fetch), 8 * lane);
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
                                             int page, int len, float scale_log2, int g,
                                             float (*kscale)[SCALE_ROW]) {
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
        // the page's V scales through the wave's LDS slot (one wave's LDS
        // accesses stay in order, so the reads below see this page's)
        const int lane = __lane_id();
        kscale[0][HEAD_DIM + (lane & 15)] = buf.vs;
        if (ASYM) kscale[1][HEAD_DIM + (lane & 15)] = buf.vz;
        // MFMA step r takes channels 64(r/4) + 16g + 4(r%4) + [0, 4) of the
        // lane group g (the query is loaded in the same order)
        if (buf.res) {
            // Exact fp16 K from the residual: the unscaled query.
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s = mfma16(as_h4(buf.k[j].x, buf.k[j].y), qh[2 * j], s);
                s = mfma16(as_h4(buf.k[j].z, buf.k[j].w), qh[2 * j + 1], s);
            }
        } else {
            // the K scale row through the same slot
            if (!ASYM) {
                // as fp16 (the row's first 256 bytes), so the query is scaled
                // with two packed fp16 multiplies a step (fp16(q) x fp16(s)
                // rounded to fp16, against fp16(q x s) before: c4 36.1 ->
                // 35.3 us).  Written and read as 32-bit words; the scale pair
                // converted as one vector (converted one component at a
                // time, this compiler packed the first twice).
                typedef float f2 __attribute__((ext_vector_type(2)));
                const h2 ksh = __builtin_convertvector(__builtin_bit_cast(f2, buf.ks), h2);
                uint32_t* krow = (uint32_t*)&kscale[0][0];
                krow[lane] = __builtin_bit_cast(uint32_t, ksh);
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const u4 kw = buf.k[r / 4];
                    const uint32_t w = r % 4 == 0 ? kw.x : r % 4 == 1 ? kw.y : r % 4 == 2 ? kw.z : kw.w;
                    const u2 kh = i8x4_to_h4(w);
                    const int ch = 64 * (r / 4) + 16 * g + 4 * (r % 4);
                    const h4 ks4 = as_h4(krow[ch / 2], krow[ch / 2 + 1]);
                    s = mfma16(as_h4(kh.x, kh.y), qh[r] * ks4, s);
                }
            }
        }
        if (ASYM && !buf.res) {
            *(u2*)&kscale[0][2 * lane] = buf.ks;
            *(u2*)&kscale[1][2 * lane] = buf.kz;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const u4 kw = buf.k[r / 4];
                const uint32_t w = r % 4 == 0 ? kw.x : r % 4 == 1 ? kw.y : r % 4 == 2 ? kw.z : kw.w;
                const u2 kh = i8x4_to_h4(w);
                const int ch = 64 * (r / 4) + 16 * g + 4 * (r % 4);
                const f4 ks = *(const f4*)&kscale[0][ch];
                f4 kz = {0.f, 0.f, 0.f, 0.f};
                if (ASYM) kz = *(const f4*)&kscale[1][ch];
                // q (fp16) x scale (fp32) rounded once to fp16: mixed-precision
                // multiplies straight from the fp16 query registers
                h4 qs;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float qa = (float)qh[r][e];
                    qs[e] = (half_t)(qa * ks[e]);
                    if (ASYM) qz += qa * kz[e];
                }
                s = mfma16(as_h4(kh.x, kh.y), qs, s);
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
        // unsigned: a dead item (page -1, len 0) masks every token
        x[i] = (unsigned)(tok0 + i) < (unsigned)len ? (s[i] + qz) * scale_log2 : neg_inf();
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
        const f4 vs = *(const f4*)&kscale[0][HEAD_DIM + 4 * g];     // tokens 4g..4g+3
#pragma unroll
        for (int i = 0; i < 4; ++i) pb[i] = (half_t)(p[i] * vs[i]);
        if (ASYM) {
            const f4 vz = *(const f4*)&kscale[1][HEAD_DIM + 4 * g];
#pragma unroll
            for (int i = 0; i < 4; ++i) st.z += p[i] * vz[i];
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
// (kernels/gqa/paged_decode.py:689-706).  256 threads; thread t owns four
// adjacent channels of one row.  Splits are taken 16 at a time with every
// load of a chunk issued before any is used (one memory round trip per
// chunk), and the chunks are merged by a running max (the same rescale the
// page loop applies).  VEC 4 reads the channels as one 16-byte load (rows
// and splits 16-byte aligned), VEC 1 as four scalar loads.
constexpr int CMB_CHUNK = 16;

__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sixteen bytes with the same write-through policy (sc1) the compiler gives
// the relaxed agent-scope store above: one vector store a lane, so a wave
// writes whole lines instead of four partial passes over them.
__device__ __forceinline__ void store_coherent4(float* p, f4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// Eight bytes the same way.
__device__ __forceinline__ void store_coherent2(float* p, float x, float y) {
    u2 v;
    v.x = __builtin_bit_cast(uint32_t, x);
    v.y = __builtin_bit_cast(uint32_t, y);
    asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// The standalone split merge (ls_combine_splits): VEC 4, 16-byte loads; 1,
// scalar loads.
template <int VEC>
__device__ void combine_partials(const float* acc, const float* m, const float* l, int S, int NR,
                                 int64_t sa_s, int64_t sa_r, int64_t sm_s, void* out, int out_f32,
                                 int64_t so_r, int tid) {
    for (int o = tid; o < NR * (HEAD_DIM / 4); o += 256) {
        const int r = o / (HEAD_DIM / 4), d0 = (o % (HEAD_DIM / 4)) * 4;
        float mg = neg_inf(), lt = 0.f;
        float at[4] = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < S; s0 += CMB_CHUNK) {
            const int n = S - s0 < CMB_CHUNK ? S - s0 : CMB_CHUNK;
            float mv[CMB_CHUNK], lv[CMB_CHUNK], av[CMB_CHUNK][4];
            // Every slot loads (slots past the last split reread it) and is
            // masked afterwards: loads under a branch would each wait for
            // the one before.
#pragma unroll
            for (int i = 0; i < CMB_CHUNK; ++i) {
                const int64_t sp = s0 + i < S ? s0 + i : S - 1;
                const float* src = acc + sp * sa_s + r * sa_r + d0;
                mv[i] = m[sp * sm_s + r];
                lv[i] = l[sp * sm_s + r];
                if (VEC == 4) {
                    const f4 t = *(const f4*)src;
#pragma unroll
                    for (int e = 0; e < 4; ++e) av[i][e] = t[e];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) av[i][e] = src[e];
                }
            }
#pragma unroll
            for (int i = 0; i < CMB_CHUNK; ++i) {
                if (i >= n) {
                    mv[i] = neg_inf();
                    lv[i] = 0.f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) av[i][e] = 0.f;
                }
            }
            float cm = mg;
#pragma unroll
            for (int i = 0; i < CMB_CHUNK; ++i) cm = fmaxf(cm, mv[i]);
            if (cm == neg_inf()) continue;            // nothing valid yet
            const float sc = __expf(mg - cm);          // 0 while mg is -inf
            lt *= sc;
#pragma unroll
            for (int e = 0; e < 4; ++e) at[e] *= sc;
#pragma unroll
            for (int i = 0; i < CMB_CHUNK; ++i) {
                const float w = __expf(mv[i] - cm);    // 0 for empty splits (m = -inf)
                lt += lv[i] * w;
#pragma unroll
                for (int e = 0; e < 4; ++e) at[e] += av[i][e] * w;
            }
            mg = cm;
        }
        const float inv = 1.f / fmaxf(lt, 1e-20f);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = at[e] * inv;
            if (out_f32)
                ((float*)out)[r * so_r + d0 + e] = v;
            else
                ((half_t*)out)[r * so_r + d0 + e] = (half_t)v;
        }
    }
}

// The fused decode's split merge over its records (write-through, read with
// device-coherent loads): per split s the accumulator rows at
// acc + s * sa_s + r * sa_r, and m (natural-log units) and l of row r side by
// side at m + s * sm_s + 2r.  Lane j of each half-wave takes channels
// 4j..4j+4 of one row r, and loads m and l of split j of the round: the
// round's weights exp(m_s - m_max) are computed once a split and handed to
// the other lanes by readlane, so a lane holds R accumulator records and no
// other, and up to R (16 or 32) splits are merged in one memory round trip.
// 256 threads, fp16 out.
template <int R>
__device__ void combine_records(const float* acc, const float* m, int S, int NR, int64_t sa_s,
                                int64_t sa_r, int64_t sm_s, half_t* out, int64_t so_r, int tid) {
    static_assert(R == 16 || R == 32, "a round is at most a half-wave of splits");
    // (acc and S are the same in every lane of the wave: declared so, the
    // resource and the split offsets are scalar and the loads issue together)
    S = __builtin_amdgcn_readfirstlane(S);
    const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(wave_uniform(acc));
    const int j = tid & 31;
    const bool upper = (tid & 32) != 0;
    for (int o = tid; o < NR * 32; o += 256) {
        const int r = o / 32, d0 = 4 * j;
        float mg = neg_inf(), lt = 0.f;
        f4 at = {0.f, 0.f, 0.f, 0.f};
        const int vo_m = (int)(((m - acc) + 2 * r) * (int64_t)sizeof(float));
        const int vo_a = (int)((r * sa_r + d0) * (int64_t)sizeof(float));
        for (int s0 = 0; s0 < S; s0 += R) {
            const int n = S - s0 < R ? S - s0 : R;      // the same in every lane
            // Every slot loads (slots past the last split reread it) and is
            // weighted 0: loads under a branch would each wait for the one
            // before.  The split's offset is wave-uniform, a scalar operand.
            const int sj = s0 + (j < n ? j : n - 1);     // (lanes j >= R weigh 0)
            const uint64_t ml = load_coherent8(rs, vo_m + (int)(sj * sm_s * (int64_t)sizeof(float)), 0);
            f4 av[R];
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int sp = s0 + (i < n ? i : n - 1);
                av[i] = load_coherent4(rs, vo_a, (int)(sp * sa_s * (int64_t)sizeof(float)));
            }
            const float mj = j < n ? __builtin_bit_cast(float, (uint32_t)ml) : neg_inf();
            float cm = mj;
#pragma unroll
            for (int k = 16; k > 0; k >>= 1) cm = fmaxf(cm, shfl_xor(cm, k));
            cm = fmaxf(cm, mg);                     // the same in the half-wave
            const bool none = cm == neg_inf();      // nothing valid yet
            const float sc = none ? 1.f : __expf(mg - cm);          // 0 while mg is -inf
            const float wj = none || j >= n ? 0.f : __expf(mj - cm);  // 0 for empty splits
            float lj = wj * __builtin_bit_cast(float, (uint32_t)(ml >> 32));
#pragma unroll
            for (int k = 16; k > 0; k >>= 1) lj += shfl_xor(lj, k);
            lt = lt * sc + lj;
            at *= sc;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const float w0 = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wj), i));
                const float w1 = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wj), 32 + i));
                at += av[i] * (upper ? w1 : w0);
            }
            mg = none ? mg : cm;
        }
        const float inv = 1.f / fmaxf(lt, 1e-20f);
        half_t* op = out + r * so_r + d0;
#pragma unroll
        for (int e = 0; e < 4; ++e) op[e] = (half_t)(at[e] * inv);
    }
}

// Diagnostic: the page walk and every load, with the arithmetic replaced by
// a fold of the loaded words (the loads-only ceiling of the access pattern).
template <int KIND>
__device__ __forceinline__ void consume_page(const PageBuf& buf, WaveState& st) {
    uint32_t x = 0;
    if (KIND == KV_FP16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) x ^= buf.k[j].x ^ buf.k[j].y ^ buf.k[j].z ^ buf.k[j].w;
#pragma unroll
        for (int i = 0; i < 4; ++i) x ^= buf.v[i].x ^ buf.v[i].y ^ buf.v[i].z ^ buf.v[i].w;
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) x ^= buf.k[j].x ^ buf.k[j].y ^ buf.k[j].z ^ buf.k[j].w;
#pragma unroll
        for (int i = 0; i < 4; ++i) x ^= buf.v[i].x ^ buf.v[i].y;
        x ^= __builtin_bit_cast(uint32_t, buf.vs);
        x ^= buf.ks.x ^ buf.ks.y;
    }
    st.acc[0][0] += __builtin_bit_cast(float, x & 0x3f8fffffu);
    st.m = 0.f;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ long long wave_sum_l(long long v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ int wave_excl_scan_i(int v, int lane) {
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    return x - v;
}

// Inclusive prefix sum over the wave's lanes in lane order, and the wave's
// total: a scan within each row of 16 lanes by DPP row shifts (a lane whose
// source is outside its row adds 0), then the rows' totals by readlane.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int wave_incl_scan_dpp(int x, int lane, int& total) {
    x += dpp_i<0x111>(x);    // row_shr:1
    x += dpp_i<0x112>(x);    // row_shr:2
    x += dpp_i<0x114>(x);    // row_shr:4
    x += dpp_i<0x118>(x);    // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31),
              r2 = __builtin_amdgcn_readlane(x, 47), r3 = __builtin_amdgcn_readlane(x, 63);
    total = r0 + r1 + r2 + r3;
    const int row = lane >> 4;
    return x + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
}

struct GroupWork {
    int len;      // its length
    int b;        // sequence served
    int s;        // split index within the sequence
    int n;        // groups serving the sequence
    int first;    // index of its first group among the head group's B * S
};

// Deal the B * S groups of a head group over the sequences: one each, the
// rest in proportion to their pages (floor), the few left over to the first
// sequences.  Every wave of every group computes the same deal from
// seq_lens (lanes take contiguous runs of sequences), so no group needs to
// hear from another.  Equal lengths give S groups each: the host's grid.
// lane_len: seq_lens[lane] (lane < B), loaded by the caller ahead of its
// page requests (loads return in order, so a length requested after them
// would wait for the pages).
__device__ GroupWork deal_groups(const DecodeParams& a, int w_id, int lane, int lane_len) {
    const int B = a.B, S = a.num_splits;
    const int W = B * S;
    auto pages_of_len = [&](int len) {
        int p = len > 0 ? (len + PAGE - 1) / PAGE : 0;
        return p < a.max_pages ? p : a.max_pages;
    };
    GroupWork r = {0, 0, 0, 1, 0};
    if (B <= WAVE) {
        // one sequence a lane: each length is read once.  Pages per lane
        // are at most max_pages < 2^24, so every sum fits 32 bits, and the
        // quotient (W - B) * p / T (numerator < 2^40) is taken in double:
        // correctly rounded, it cannot reach the next integer, since a
        // non-integral quotient is at least 1/T below it.
        const int my_len = lane < B ? lane_len : 0;
        const int p = lane < B ? pages_of_len(my_len) : 0;
        int T;
        (void)wave_incl_scan_dpp(p, lane, T);
        int n = 0;
        if (lane < B)
            n = T > 0 ? 1 + (int)((double)(W - B) * (double)p / (double)T) : S;
        int sum_n;
        const int incl = wave_incl_scan_dpp(n, lane, sum_n);
        const int left = W - sum_n;                    // 0 <= left < B when T > 0
        const int pos = incl - n + (lane < left ? lane : left);
        n += lane < left ? 1 : 0;
        const bool mine = lane < B && w_id >= pos && w_id < pos + n;
        const unsigned long long who = __ballot(mine);
        const int src = who ? __builtin_ctzll(who) : 0;
        r.b = src;
        r.len = __builtin_amdgcn_readlane(my_len, src);
        r.n = __builtin_amdgcn_readlane(n, src);
        r.first = __builtin_amdgcn_readlane(pos, src);
        r.s = w_id - r.first;
        return r;
    }
    // longer batches: lanes take contiguous runs of sequences
    const int per_lane = (B + WAVE - 1) / WAVE;
    const int b0 = lane * per_lane < B ? lane * per_lane : B;
    const int b1 = b0 + per_lane < B ? b0 + per_lane : B;
    long long part = 0;
    for (int i = b0; i < b1; ++i) part += pages_of_len(a.seq_lens[i]);
    const long long T = wave_sum_l(part);
    auto base_n = [&](int p) { return T > 0 ? 1 + (int)((long long)(W - B) * p / T) : S; };
    int mine_n = 0;
    for (int i = b0; i < b1; ++i) mine_n += base_n(pages_of_len(a.seq_lens[i]));
    const int left = W - wave_sum_i(mine_n);
    const int run = mine_n + ((b1 < left ? b1 : left) - (b0 < left ? b0 : left));
    int pos = wave_excl_scan_i(run, lane);
    bool found = false;
    if (w_id >= pos && w_id < pos + run) {
        for (int i = b0; i < b1; ++i) {
            const int li = a.seq_lens[i];
            const int n = base_n(pages_of_len(li)) + (i < left ? 1 : 0);
            if (w_id < pos + n) {
                r.len = li;
                r.b = i;
                r.s = w_id - pos;
                r.n = n;
                r.first = pos;
                found = true;
                break;
            }
            pos += n;
        }
    }
    const unsigned long long who = __ballot(found);
    const int src = who ? __builtin_ctzll(who) : 0;
    r.b = __shfl(r.b, src);
    r.s = __shfl(r.s, src);
    r.n = __shfl(r.n, src);
    r.first = __shfl(r.first, src);
    // (the length comes from the lane that found it, not a new load: a load
    // pending here would make the small-batch path, which this one joins,
    // wait for every outstanding load before its first page request)
    r.len = __shfl(r.len, src);
    return r;
}

// Claim the next item of the group for the calling wave: an LDS atomic by
// lane 0.  The result stays in lane 0's register until claimed_item()
// reads it one iteration later, off the critical path.
__device__ __forceinline__ int claim_item(int* counter, int lane) {
    int r = 0;
    if (lane == 0)
        r = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return r;
}
__device__ __forceinline__ int claimed_item(int raw) { return __builtin_amdgcn_readlane(raw, 0); }

// The Quest scores of the pages [p_lo, p_hi) of sequence b's rows for the
// group's HG heads, stored write-through into a.scores (the index kernel's
// rule: page 0 and the last `recent` pages +inf, pages past the end or with
// a block id outside the pool -inf).  Each 16-lane row of a wave takes one
// (page, head) unit a round, 8 channels a lane; the block ids of R rounds
// are requested together, then their bounds (two dependent round trips a
// batch of R rounds: the caller picks R so that its share is one batch).
template <int NWT, int HG, int R>
__device__ void score_slice(const DecodeParams& a, int b, int h0, int len, int p_lo, int p_hi) {
    const int lane = threadIdx.x % WAVE, wv = threadIdx.x / WAVE;
    const int row = lane >> 4, c0 = (lane & 15) * 8;
    const int np = len > 0 ? (len + PAGE - 1) / PAGE : 0;
    constexpr int PPR = 4 / HG;                 // pages a wave takes a round
    const int hh = row % HG;
    const half_t* qb = a.q + (int64_t)b * a.sq_b + (int64_t)(h0 + hh) * a.sq_h + c0;
    float* srow = a.scores + (int64_t)b * a.ssc_b + (int64_t)(h0 + hh) * a.ssc_h;
    // the lane's 8 channels of every query row, loaded once, together
    // (rows past n_rep repeat row 0 and are not used)
    u4 qv[COOP_MAX_NREP];
#pragma unroll
    for (int q = 0; q < COOP_MAX_NREP; ++q) qv[q] = *(const u4*)(qb + (int64_t)(q < a.NR ? q : 0) * a.sq_r);
    u4 qm[COOP_MAX_NREP];
#pragma unroll
    for (int q = 0; q < COOP_MAX_NREP; ++q) qm[q] = quest_masks(qv[q]);
    for (int base = p_lo; base < p_hi; base += R * NWT * PPR) {
        int pg[R], st[R];
        int blk[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int p = base + (r * NWT + wv) * PPR + row / HG;
            pg[r] = p;
            st[r] = p >= p_hi ? 0 : p >= np ? 3 : (p == 0 || p >= np - a.recent) ? 2 : 1;
            const int pc = p < a.max_pages ? p : a.max_pages - 1;
            blk[r] = a.block_tables[(int64_t)b * a.sbt_b + pc];
            issue_here();   // the table and bounds loads go out where written,
                            // in order (B8 x 32K: 45.77 -> 45.44 us)
        }
        u4 lo[R], hi[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (st[r] == 1 && (unsigned)blk[r] >= (unsigned)a.num_blocks) st[r] = 3;
            const int bk = st[r] == 1 ? blk[r] : 0;
            const int64_t off = (int64_t)bk * a.sb_b + (int64_t)(h0 + hh) * a.sb_h + c0;
            // (read once a call: nontemporal, 0.37 us faster at B8 x 32K
            // than plain loads)
            lo[r] = stream_load((const u4*)((const half_t*)a.kmin + off));
            hi[r] = stream_load((const u4*)((const half_t*)a.kmax + off));
            issue_here();
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            // a round past the share in every lane of the wave: nothing to
            // compute or store (its loads went out with the others')
            if (__builtin_amdgcn_ballot_w64(st[r] != 0) == 0) continue;
            float bst = neg_inf();
#pragma unroll
            for (int q = 0; q < COOP_MAX_NREP; ++q) {
                // (a uniform branch, the loop fully unrolled: the rows stay
                // in registers; a `break` here kept them in scratch)
                if (q < a.NR) bst = fmaxf(bst, quest_row16_sum(quest_part(qv[q], qm[q], lo[r], hi[r])));
            }
            if ((lane & 15) == 0 && st[r] != 0) {
                const float v = st[r] == 1 ? bst : st[r] == 2 ? __builtin_inff() : neg_inf();
                __hip_atomic_store(srow + pg[r], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// One page's score computed alone by the calling thread (the same sums in
// the same order as score_slice), for a score that did not arrive in time.
__device__ float score_one(const DecodeParams& a, int b, int h, int len, int p) {
    const int np = len > 0 ? (len + PAGE - 1) / PAGE : 0;
    if (p >= np) return neg_inf();
    if (p == 0 || p >= np - a.recent) return __builtin_inff();
    const int blk = p < a.max_pages ? a.block_tables[(int64_t)b * a.sbt_b + p] : -1;
    if ((unsigned)blk >= (unsigned)a.num_blocks) return neg_inf();
    const half_t* qb = a.q + (int64_t)b * a.sq_b + (int64_t)h * a.sq_h;
    const half_t* lob = (const half_t*)a.kmin + (int64_t)blk * a.sb_b + (int64_t)h * a.sb_h;
    const half_t* hib = (const half_t*)a.kmax + (int64_t)blk * a.sb_b + (int64_t)h * a.sb_h;
    // quest_row16_sum's order as lane 0 sees it: lane pairs (xor 1), pairs
    // of pairs (xor 2), the half-row mirror, the row mirror, i.e. the pairs
    // (0,1) (2,3) | (6,7) (4,5) || (14,15) (12,13) | (8,9) (10,11) combined
    // left to right at each level; taken one pair at a time so only one
    // pair's operands are live
    float bst = neg_inf();
    for (int q = 0; q < a.NR; ++q) {
        const half_t* qr = qb + (int64_t)q * a.sq_r;
        float pa = 0.f, qa = 0.f, ha = 0.f, tot = 0.f;
#pragma unroll 1
        for (int k = 0; k < 8; ++k) {
            const int m = (k & 4 ? 8 : 0) + ((k & 2) ? (k & 1 ? 4 : 6) : (k & 1 ? 2 : 0)) ^
                          (k & 4 ? 6 : 0);
            const float x = quest_part(*(const u4*)(qr + 8 * m), *(const u4*)(lob + 8 * m),
                                       *(const u4*)(hib + 8 * m));
            const float y = quest_part(*(const u4*)(qr + 8 * (m + 1)),
                                       *(const u4*)(lob + 8 * (m + 1)),
                                       *(const u4*)(hib + 8 * (m + 1)));
            const float v = x + y;
            if ((k & 1) == 0) {
                pa = v;
            } else {
                const float qd = pa + v;
                if ((k & 2) == 0) {
                    qa = qd;
                } else {
                    const float hv = qa + qd;
                    if ((k & 4) == 0) ha = hv;
                    else tot = ha + hv;
                }
            }
        }
        bst = fmaxf(bst, tot);
    }
    return bst;
}

// SPARSE: 0 the dense walk; 1 a page-subset walk over the caller's lists;
// 2 a page-subset walk whose lists the group selects from page scores;
// 3 the same with the scores computed by the launch itself, each group
// scoring its share of its sequence's pages (score_slice).
template <int KIND, bool ASYM, bool HAS_RES, int SPARSE, int NWT, int HG, int ABL = 0>
// (two waves a SIMD also for the 4-wave groups of odd head counts: the
// register budget of the 8-wave groups, 256)
__global__ __launch_bounds__(WAVE* NWT) __attribute__((amdgpu_waves_per_eu(2)))
void paged_decode_kernel(const DecodeParams a) {
    // Pages in flight ahead of the one being computed: one.  INT8: a second
    // buffer measured slower (c4 35.3 -> 39.1 us; with the page loads as
    // inline asm and the walk's own waits, 37.5 us at one head a group,
    // spills at two), and a third takes the kernel to one wave a SIMD.
    // fp16 with K through LDS: the read-only probe of the B16 x 16K pages
    // ran 42.5 us with one page in flight, 43.7 us with two.
    constexpr int PF_DEPTH = 1;
    constexpr int NB = PF_DEPTH + 1;
    __shared__ DecodeSmem<NWT, HG, KIND == KV_INT8> sm;
    // fp16: the waves' K slots, one array a buffer: the compiler holds an
    // LDS access back until every direct load that may write its object is
    // done, so the slots are objects apart from each other and from the
    // item claims and the table
    __shared__ __attribute__((aligned(16))) char kstage0[KIND == KV_FP16 ? NWT * KSLOT_BYTES : 16];
    __shared__ __attribute__((aligned(16))) char kstage1[KIND == KV_FP16 ? NWT * KSLOT_BYTES : 16];

    LS_STAMP(0);
#ifdef LS_STAMPS
    if (threadIdx.x == 0)           // stamp 15: the XCD this group runs on
        g_ls_stamps[(blockIdx.x + gridDim.x * blockIdx.y) * LS_NSTAMP + 15] =
            (uint64_t)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15) | (1ull << 40);
#endif
    const int H = a.H;
    // A group serves HG adjacent KV heads of one (sequence, split) with NWT
    // waves.  Its work items are (page, head) pairs, claimed one at a time
    // from an LDS counter by whichever wave is ready: the oldest waves win
    // memory arbitration and would otherwise finish a static share early
    // and idle while the youngest finish theirs.
    const int n_hg = H / HG;
    // A page-subset walk takes its wave index through readfirstlane, so the
    // compiler knows it wave-uniform (c5 48.6 -> 48.4 us); the dense walks
    // measured no gain from it (c2, c3 +0.05 us).
    const int wv = SPARSE ? __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE)
                          : (int)(threadIdx.x / WAVE);
    const int lane = threadIdx.x % WAVE;
    // the host grid (split * n_hg + head group, sequence); a dense walk's
    // numbered XCD-major so the groups of a sequence share an XCD (c2
    // 50.3 -> 49.8 us; the page-subset walks measured slower so, c5 50.0 ->
    // 51.2 us, and keep the dispatch order)
    const int L = blockIdx.x + gridDim.x * blockIdx.y;
    const int wg = SPARSE ? L : xcd_major(L, gridDim.x * gridDim.y);
    const int h0 = (wg % gridDim.x % n_hg) * HG;
    const int split = wg % gridDim.x / n_hg;
    const int hb = wg / gridDim.x;      // the host grid's sequence (speculation)
    const int g = lane >> 4, c = lane & 15;
    const int S = a.num_splits;
    // Each head of the group has its own NWH waves (wave wv serves head hw
    // of the pair as its wl-th wave): a wave holds one head's state and
    // query, and both heads' waves walk the same pages at about the same
    // time, so the two halves of a token row are still read together.  The
    // heads alternate over the waves: the older waves win memory
    // arbitration, and with the first half of the waves on one head that
    // head ran ahead and its waves idled while the other's finished (c4
    // 32.60 -> 32.30, c2 46.15 -> 45.89, s8k 27.14 -> 26.97 us).
    constexpr int NWH = NWT / HG;
    const int hw = wv % HG, wl = wv / HG;
    if (threadIdx.x < (unsigned)HG) sm.claim[threadIdx.x] = NB * NWH;   // below: fixed items

    // Dense walk with pages-per-split given by the host (from the caller's
    // max_seq_len): the group's block ids are requested before the sequence
    // length arrives.  Any partition of the pages gives the same result
    // (split-K is exact), so the host's only affects speed.
    const bool host_split = !SPARSE && a.pages_per_split > 0;
    // The loads are unconditional (clamped to a valid entry, the value
    // discarded when out of range): predicated loads split the control flow,
    // and the compiler then waits for every outstanding load where the
    // paths join, which would serialise the first page loads behind each
    // other.
    int spec_blk = -1;
    const int spec_lo = host_split ? split * a.pages_per_split : 0;
    int first_blk = -1;
    if (host_split && a.max_pages > 0) {
        const int32_t* row = a.block_tables + (int64_t)hb * a.sbt_b;
        const int last = a.max_pages - 1;
        const int te = spec_lo + (int)threadIdx.x;
        const int tv = row[te < last ? te : last];
        spec_blk = (int)threadIdx.x < a.pages_per_split && te <= last ? tv : -1;
        // ... and lane u < NB of each wave fetches the block of the wave's
        // own fixed item u, so its first page loads need neither the table
        // nor the barrier.
        const int e = wl + (lane < NB ? lane : 0) * NWH;
        const int fe = spec_lo + e;
        const int fv = row[fe < last ? fe : last];
        first_blk = lane < NB && e < a.pages_per_split && fe <= last ? fv : -1;
    }

    // The lengths the deal reads (one a lane for batches up to 64).
    int lane_len = 0;
    if (!SPARSE && a.B <= WAVE) lane_len = a.seq_lens[lane < a.B ? lane : 0];

    // Query operands of the group's heads: row c, channels 32j+8g..+8.
    // Rows past n_rep repeat row 0: their (finite) scores fill MFMA columns
    // whose results are never stored, and not masking them keeps the loads
    // free of any use before the first pages are requested.
    // (The host grid's sequence, which the deal keeps for equal lengths, so
    // the loads need not wait for the deal; reloaded below if it moved.)
    h4 qh[8];
    // (INT8: the channel order of its K loads, 64(r/4) + 16g + 4(r%4) for
    // MFMA step r.)
    auto load_q = [&](int bq) {
        const half_t* qrow = a.q + (int64_t)bq * a.sq_b + (int64_t)(h0 + hw) * a.sq_h +
                             (int64_t)(c < a.NR ? c : 0) * a.sq_r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u4 t = KIND == KV_FP16 ? *(const u4*)(qrow + 8 * g + 32 * j)
                                         : *(const u4*)(qrow + 16 * g + 64 * (j / 2) + 8 * (j % 2));
            qh[2 * j] = as_h4(t.x, t.y);
            qh[2 * j + 1] = as_h4(t.z, t.w);
        }
    };
    load_q(hb);

    // Page buffers in rotation: item k+1 is in flight while item k is
    // computed, and the item after is being claimed.
    PageBuf buf[NB];
    auto kslot = [&](int slot) { return (slot == 0 ? kstage0 : kstage1) + wv * KSLOT_BYTES; };
    static_assert(NB == 2, "one K slot array a page buffer");
    int item[NB], pgs[NB], blks[NB];
    auto issue_raw = [&](int slot, int it, int blk, int pg) {
        item[slot] = it;
        blks[slot] = blk;
        pgs[slot] = pg;
        // A request needs only a block id that is safe to read: the item is
        // checked against the sequence when it is computed (and the walk
        // never holds an INT8 sequence's residual page: it is computed apart)
        // (an item with no block, past the end included, is requested from a
        // resource of no bytes at block 0's address: zeros, no memory
        // request)
        const bool valid = (unsigned)blk < (unsigned)a.num_blocks;
        const int safe_blk = valid ? blk : 0;
        const bool fetch = valid;
        load_page<KIND, ASYM, KIND == KV_FP16 && HAS_RES>(a, buf[slot], safe_blk, -1, 0, 0,
                                                          h0 + hw, g, c, fetch, kslot(slot));
    };
    // fp16: the K rows of the page in buffer `slot`, from its LDS slot into
    // the MFMA layout (row c; pieces 4j + g, stored at (4j + g) ^ c)
    auto k_from_lds = [&](int slot) {
        if constexpr (KIND == KV_FP16) {
            // that page's direct loads are done once no more than its own V
            // loads and the PF_DEPTH later pages' requests are outstanding
            wait_vm_lds<4 + FP16_PAGE_VM * PF_DEPTH>();
            const char* rowp = kslot(slot) + c * 256;
#pragma unroll
            for (int j = 0; j < 4; ++j) buf[slot].k[j] = *(const u4*)(rowp + (((4 * j + g) ^ c) << 4));
        }
    };
    // Which sequence and split this group serves: the host grid's for a
    // page-subset walk, else the length-proportional deal.
    GroupWork gw;
    if (SPARSE) {
        gw.b = hb;
        gw.s = split;
        gw.n = S;
        gw.first = hb * S;
        gw.len = a.seq_lens[hb];
    } else {
        gw = deal_groups(a, hb * S + split, lane, lane_len);
    }
    const int b = gw.b;
    const int Sb = gw.n;
    const int len = gw.len;
    if (b != hb) load_q(b);
    int num_pages = (len + PAGE - 1) / PAGE;
    num_pages = num_pages < a.max_pages ? num_pages : a.max_pages;
    // the sequence's residual row, read once (the page loads take it as a
    // value: a load of it per page would make every page request wait)
    bool res_ok = false;
    int res_row = 0;
    if (HAS_RES) {
        const int rr = a.res_rows[b];
        res_ok = rr >= 0 && rr < a.res_cap;
        res_row = res_ok ? rr : 0;
    }

    // The walk: the sequence's pages (dense) or its selection list (page
    // subset, one list per head, all of the same length).
    int n_list = num_pages;
    if (SPARSE) {
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
    // Pages of this split: the host's partition when the deal kept the host
    // grid for this group and the host's split covers the sequence (its
    // speculative table loads are then the group's own); else S_b even
    // shares of the length (kernels/gqa/paged_decode.py:564-568 derives the
    // split on the device the same way).
    const bool spec_ok = host_split && b == hb && Sb == S && gw.s == split &&
                         num_pages <= S * a.pages_per_split;
    int lo, hi;
    if (spec_ok) {
        lo = spec_lo;
        hi = lo + a.pages_per_split < n_list ? lo + a.pages_per_split : n_list;
    } else if (SPARSE || Sb == S) {
        const int per = (n_list + S - 1) / S;
        lo = gw.s * per;
        hi = lo + per < n_list ? lo + per : n_list;
    } else {
        lo = (int)((long long)gw.s * n_list / Sb);
        hi = (int)((long long)(gw.s + 1) * n_list / Sb);
    }
    const int n_ent = hi > lo ? hi - lo : 0;
    // INT8 with a residual: the sequence's last page (K from the fp16
    // residual) is not a walk item; one wave of the group whose range ends
    // the sequence computes it apart, so the walk's page buffers and compute
    // carry INT8 pages only (their residual branch cost 3 us at c4).
    const bool ends_seq = HAS_RES && n_ent > 0 && hi == num_pages;
    const int n_items = n_ent - (ends_seq ? 1 : 0);     // a head's items

    // Resolve the group's entries to (block, page) once, into LDS (the merge
    // buffer, idle until the walk ends).  Block ids outside the pool, list
    // entries outside the sequence and a last page whose residual row is
    // outside the residual become -1 and are never dereferenced.  A range
    // longer than the table resolves each claimed item from global memory.
    constexpr int ENT_INTS = DecodeSmem<NWT, HG, KIND == KV_INT8>::ENT_INTS;
    constexpr int CAP = SPARSE ? ENT_INTS / (2 * HG) : ENT_INTS;
    const bool cached = n_ent <= CAP;
    // (an item's block and page, returned by value: resolvers writing
    // through references put the pair in a stack slot of the general walk)
    struct ItemRef {
        int blk, pg;
    };
    auto resolve_global = [&](int e, int hh) -> ItemRef {
        const int pg =
            SPARSE ? a.sel[(int64_t)b * a.ssel_b + (int64_t)(h0 + hh) * a.ssel_h + lo + e] : lo + e;
        int blk = -1;
        if (pg >= 0 && pg < num_pages) {
            const int t = a.block_tables[(int64_t)b * a.sbt_b + pg];
            blk = t < 0 || t >= a.num_blocks || (HAS_RES && pg == num_pages - 1 && !res_ok) ? -1 : t;
        }
        return {blk, pg};
    };
    auto fill_table = [&]() {
        if (!cached) return;
        if constexpr (SPARSE >= 2) {
            // Each 256-thread half selects its head's list from the page
            // scores (the selection kernel's radix select; in LDS the merge
            // buffer holds only after the walk) and keeps the entries of
            // this split's range, resolved to blocks.  (A threshold
            // bisection without LDS atomics measured slower, 25 against 10
            // us for the selection alone: at one wave a SIMD the select is
            // bound by its dependent instruction latency, and the bisection
            // has the longer chain.)
            static_assert(WAVE * NWT == 256 * HG, "one 256-thread group a head");
            static_assert(CAP >= SELECT_SPLIT_ENTRIES, "a split's entries fit the table");
            const int hh = threadIdx.x / 256, tid = threadIdx.x % 256;
            static_assert(sizeof(LinSelectSmem) * HG <= sizeof(sm.acc), "selection fits the merge buffer");
            LinSelectSmem* ssm = reinterpret_cast<LinSelectSmem*>(&sm.acc[0][0][0][0]);
            const float* row = a.scores + (int64_t)b * a.ssc_b + (int64_t)(h0 + hh) * a.ssc_h;
            // the selection reports pages only; their blocks are looked up
            // below, one independent load a thread (a load per reported page
            // would chain a thread's round trips)
            auto emit = [&](int pos, int pg) {
                if (pos >= lo && pos < hi) sm.ent[(hh * 2 + 1) * CAP + pos - lo] = pg;
            };
            if constexpr (SPARSE == 3) {
                // this group's share of the sequence's pages scored, then the
                // whole rows read as the other groups' shares land
                const int per = (a.score_pages + Sb - 1) / Sb;
                const int p_lo = gw.s * per;
                const int p_hi = p_lo + per < a.score_pages ? p_lo + per : a.score_pages;
                // (batches of 5 rounds: a share of up to 80 pages in one,
                // the 74-page shares of 14 and 28 splits included, which
                // batches of 4 had taken in two; one variant only: with
                // batches of 4, 5 and 8 compiled in, the larger kernel ran
                // B8 x 32K 0.3 us slower)
                score_slice<NWT, HG, 5>(a, b, h0, len, p_lo, p_hi);
                LS_STAMP(1);
                // the group's score stores complete, then it counts itself in
                // the word after row (b, h0) (all ones at rest, so the count
                // reaches Sb - 1 when every group of the sequence is done)
                int* done = (int*)(a.scores + (int64_t)b * a.ssc_b + (int64_t)h0 * a.ssc_h +
                                   a.score_pages);
                handoff_release();
                __syncthreads();
                if (threadIdx.x == 0)
                    __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                LS_STAMP(2);
                struct Coop {
                    const DecodeParams& a;
                    int b, h, len, Sb;
                    const int* done;
                    __device__ float operator()(int p) const { return score_one(a, b, h, len, p); }
                    // true once every group of the sequence has counted itself
                    // (one word polled: every thread of a wave reads the same
                    // line), false if that does not happen within the bound
                    __device__ bool wait() const {
                        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                        while (true) {
                            if (load_coherent(done) == Sb - 1) return true;
                            if (__builtin_amdgcn_s_memrealtime() - t0 >= a.coop_wait_ticks)
                                return false;
                            // (16 x 64 cycles between polls: 8, 4 and 2 measured
                            // 0.07-0.25 us slower at B8 x 32K, 32 as slow as 8)
                            __builtin_amdgcn_s_sleep(16);
                        }
                    }
                };
                const Coop fix{a, b, h0 + hh, len, Sb, done};
                // (rows of up to COOP_MAX_PAGES pages: eight keys a thread;
                // up to 1024, four, half the work a thread: B16 x 16K 40.6 ->
                // 39.5 us.  In this order: with the four-key branch first,
                // the eight-key rows ran 0.45 us slower, B8 x 32K 42.7 ->
                // 43.1 us)
                if (a.score_pages > 4 * 256)
                    select_row_lin<8, decltype(emit), 1>(row, a.score_pages, n_list, tid, ssm[hh],
                                                         ssm[0].vote, emit, fix);
                else
                    select_row_lin<4, decltype(emit), 1>(row, a.score_pages, n_list, tid, ssm[hh],
                                                         ssm[0].vote, emit, fix);
            } else {
                if (a.score_pages <= 8 * 256)
                    select_row_lin<8>(row, a.score_pages, n_list, tid, ssm[hh], ssm[0].vote, emit);
                else
                    select_row_lin<32>(row, a.score_pages, n_list, tid, ssm[hh], ssm[0].vote,
                                       emit);
            }
            __syncthreads();
            if (SPARSE == 3 && Sb == 1 && threadIdx.x == 0) {
                // the only reader of its rows: the count after row (b, h0)
                // back to all ones (the rows keep their scores: a call reads
                // them only after its writers counted themselves)
                __hip_atomic_store((uint32_t*)(a.scores + (int64_t)b * a.ssc_b +
                                               (int64_t)h0 * a.ssc_h + a.score_pages),
                                   EMPTY_WORD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            const int32_t* trow = a.block_tables + (int64_t)b * a.sbt_b;
            for (int i = threadIdx.x; i < n_ent * HG; i += WAVE * NWT) {
                const int hs = i / n_ent, e = i % n_ent;
                const int pg = sm.ent[(hs * 2 + 1) * CAP + e];
                int blk = -1;
                if (pg >= 0 && pg < num_pages) {
                    blk = trow[pg];
                    if (blk < 0 || blk >= a.num_blocks) blk = -1;
                }
                sm.ent[(hs * 2) * CAP + e] = blk;
            }
        } else if (SPARSE) {
            for (int i = threadIdx.x; i < n_ent * HG; i += WAVE * NWT) {
                const int hh = i / n_ent, e = i % n_ent;
                const ItemRef r = resolve_global(e, hh);
                sm.ent[(hh * 2) * CAP + e] = r.blk;
                sm.ent[(hh * 2 + 1) * CAP + e] = r.pg;
            }
        } else {
            for (int e = threadIdx.x; e < n_ent; e += WAVE * NWT) {
                // this thread's speculative load covered entry threadIdx.x only
                int blk = e == (int)threadIdx.x && spec_ok ? spec_blk : -2;
                const int pg = lo + e;
                if (blk == -2 || !(pg >= 0 && pg < num_pages)) {
                    blk = resolve_global(e, 0).blk;
                } else {
                    if (blk < 0 || blk >= a.num_blocks) blk = -1;
                    if (HAS_RES && pg == num_pages - 1 && !res_ok) blk = -1;
                }
                sm.ent[e] = blk;
            }
        }
    };

    const float scale_log2 = a.scale * LOG2E;

    WaveState st;
#pragma unroll
    for (int t = 0; t < 8; ++t) st.acc[t] = (f4){0.f, 0.f, 0.f, 0.f};
    st.m = neg_inf();
    st.l = 0.f;
    st.z = 0.f;

    // Item i of the wave's head: entry i.  Items past the end or
    // unresolvable come back with blk -1: their buffer is filled from block 0
    // (any valid address: it keeps every iteration's loads and waits
    // identical) and computed with every token masked.
    auto resolve_lds = [&](int i) -> ItemRef {
        if (i >= n_items) return {-1, -1};
        if (SPARSE) return {sm.ent[(hw * 2) * CAP + i], sm.ent[(hw * 2 + 1) * CAP + i]};
        return {sm.ent[i], lo + i};
    };
    // The wave's fixed item u (dense walk with the host's split): its block
    // is in lane u of first_blk.  Returned unchecked: the sequence length is
    // not needed to request the page (issue_with checks the item afterwards).
    auto resolve_first = [&](int u, int i) -> ItemRef {
        return {__builtin_amdgcn_readlane(first_blk, u), spec_lo + i};
    };
    auto resolve_mem = [&](int i) -> ItemRef {
        if (i >= n_items) return {-1, -1};
        return resolve_global(i, hw);
    };

    auto live = [&](int slot) {
        const int it = item[slot], blk = blks[slot], pg = pgs[slot];
        return it < n_items && blk >= 0 && blk < a.num_blocks && pg >= 0 && pg < num_pages &&
               !(HAS_RES && pg == num_pages - 1 && !res_ok);
    };
#ifdef LS_STAMPS
    int n_done = 0;     // items this wave computed live
#endif
    auto walk = [&](auto resolve, auto first) {
        if constexpr (HAS_RES) {
            // the last wave of each head computes that head's last page
            const int hr = hw;
            if (ends_seq && res_ok && wl == NWH - 1) {
                const int lp = num_pages - 1;
                const int blk = a.block_tables[(int64_t)b * a.sbt_b + lp];
                const bool okb = blk >= 0 && blk < a.num_blocks;
                PageBuf rb;
                load_page<KIND, ASYM, true>(a, rb, okb ? blk : 0, lp, num_pages, res_row, h0 + hr,
                                            g, c);
                compute_page<KIND, ASYM>(rb, st, qh, okb ? lp : -1, okb ? len : 0, scale_log2, g,
                                         sm.kscale[wv]);
            }
        }
        auto issue_with = [&](auto res, int slot, int it) {
            const ItemRef r = res(it);
            issue_raw(slot, it, r.blk, r.pg);
        };
        auto issue = [&](int slot, int it) { issue_with(resolve, slot, it); };
        // The first items are fixed (wave wl of a head takes wl, wl + NWH, ...): their
        // loads are in flight while the group fills the item table and meets
        // at the barrier (a selecting group knows its items only after).
        if (SPARSE >= 2) {
            fill_table();
            __syncthreads();
            LS_STAMP(7);
        }
#pragma unroll
        for (int u = 0; u < PF_DEPTH; ++u)
            issue_with([&](int i) { return first(u, i); }, u, wl + u * NWH);
        if (SPARSE < 2) {
            fill_table();
            __syncthreads();
        }
        int it_n = wl + PF_DEPTH * NWH;
        if (item[0] >= n_items) return;
        while (true) {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                // claim an item (read next iteration), then load the item
                // claimed last iteration into the free buffer
                const int raw_new = claim_item(&sm.claim[hw], lane);
                issue((u + PF_DEPTH) % NB, it_n);
                it_n = claimed_item(raw_new);
                // computed even when dead (every token masked, a no-op on the
                // state): a skipped buffer would leave its loads unwaited and
                // force conservative waits on the next reuse of its registers
                const bool ok_u = live(u);
                const int live_len = ok_u ? len : 0;
#ifdef LS_STAMPS
                n_done += ok_u ? 1 : 0;
#endif
                k_from_lds(u);
                if (ABL == 1 || ABL == 2)
                    consume_page<KIND>(buf[u], st);
                else
                    compute_page<KIND, ASYM>(buf[u], st, qh, ok_u ? pgs[u] : -1, live_len,
                                             scale_log2, g, sm.kscale[wv]);
                // items arrive in increasing order: past the end, all later are too
                if (item[(u + 1) % NB] >= n_items) return;
            }
        }
    };
    // Separate instantiations for the fast path (the host's split covers the
    // sequence and the item table fits in LDS) and the general ones, so no
    // fallback load shares the fast path's control flow.
    auto first_fixed = [&](int u, int i) { return resolve_first(u, i); };
    auto first_mem = [&](int, int i) { return resolve_mem(i); };
    auto first_lds = [&](int, int i) { return resolve_lds(i); };
    if (SPARSE >= 2)
        walk(resolve_lds, first_lds);      // the host keeps every range within the table
    else if (cached && spec_ok)
        walk(resolve_lds, first_fixed);
    else if (cached)
        walk(resolve_lds, first_mem);
    else
        walk(resolve_mem, first_mem);
    // (fp16: the direct K loads of items past the end may still be writing
    // the wave's slots; none may land after the group ends)
    if constexpr (KIND == KV_FP16) wait_vm_lds<0>();
    LS_STAMP(8);
#ifdef LS_STAMPS
    // (dense walks: the first and the last of the group's waves to end their
    // walks, stamps 1 and 2, recorded after the merge's barrier)
    __shared__ uint64_t wave_end[NWT];
    if (lane == 0) {
        wave_end[wv] = __builtin_amdgcn_s_memrealtime();
        // per wave (up to 8): walk end, and items computed | head << 16
        if (wv < 8) {
            uint64_t* ws = g_ls_stamps + (blockIdx.x + gridDim.x * blockIdx.y) * LS_NSTAMP + 16;
            ws[wv] = wave_end[wv];
            ws[8 + wv] = (uint64_t)(n_done | (hw << 16));
        }
    }
#endif

    const int NR = a.NR;
    const bool single = Sb == 1;
    const int w_rec = gw.first + gw.s;   // this group's record slot among the head group's B * S
    if (ABL >= 2) {                      // diagnostic: no merge, no partials
        if (st.acc[0][0] == 12345.f && st.l == 1.f) a.out[threadIdx.x] = (half_t)st.m;
        __syncthreads();
        if (!single && threadIdx.x < (unsigned)HG) {
            const int64_t bh = (int64_t)b * H + h0 + threadIdx.x;
            if (__hip_atomic_fetch_add(a.counters + bh * COUNTER_STRIDE, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == Sb - 1)
                __hip_atomic_store(a.counters + bh * COUNTER_STRIDE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }

    // ---- merge the waves' states in LDS (all heads at once); each wave
    // stores its state as soon as its walk ends ----
    // One record per (group, head): acc[NR][128], m[16], l[16], at slot
    // (w_rec * H + h); the groups of a sequence have adjacent slots.  Every
    // cache line of a record is written by this group alone.
    const int64_t rec = (int64_t)NR * HEAD_DIM + 2 * MAX_NREP;
    const float lrow = group4_sum(st.l);
    if (ASYM) {
        const float zrow = group4_sum(st.z);
#pragma unroll
        for (int t = 0; t < 8; ++t) st.acc[t] += zrow;
    }
    if (c < NR) {                        // rows past n_rep hold nothing
        if (g == 0) {
            sm.m[hw][wl][c] = st.m;
            sm.l[hw][wl][c] = lrow;
        }
        // the lane's 32 channels 32g..32g+31 (channel 32g + 8i + t is
        // element i of tile t) as eight 16-byte stores
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            f4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = st.acc[4 * (j % 2) + e][j / 2];
            *(f4*)&sm.acc[hw][wl][c][32 * g + 4 * j] = v;
        }
    }
    __syncthreads();

    // 256 threads a head; a thread merges four channels of one row, with
    // all of its loads issued together (rows 8 apart share a thread).
    // TPH threads a head (a multiple of 32: rows TPH / 32 apart share a thread)
    constexpr int TPH = WAVE * NWH;
    {
        const int hh = threadIdx.x / TPH, t256 = threadIdx.x % TPH;
        const int d0 = (t256 % 32) * 4;
        float* pacc = a.work + ((int64_t)w_rec * H + h0 + hh) * rec;
        float* pm = pacc + NR * HEAD_DIM;       // (m, l) of each row
        for (int r = t256 / 32; r < NR; r += TPH / 32) {
            float mv[NWH], lv[NWH];
            f4 av[NWH];
#pragma unroll
            for (int u = 0; u < NWH; ++u) {
                mv[u] = sm.m[hh][u][r];
                lv[u] = sm.l[hh][u][r];
                av[u] = *(const f4*)&sm.acc[hh][u][r][d0];
            }
            float mg = neg_inf();
#pragma unroll
            for (int u = 0; u < NWH; ++u) mg = fmaxf(mg, mv[u]);
            float lt = 0.f;
            f4 at = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < NWH; ++u) {
                const float wt = mg == neg_inf() ? 0.f : fast_exp2(mv[u] - mg);
                lt += lv[u] * wt;
#pragma unroll
                for (int e = 0; e < 4; ++e) at[e] += av[u][e] * wt;
            }
            if (single) {
                half_t* o = a.out + (int64_t)b * a.so_b + (int64_t)(h0 + hh) * a.so_h +
                            (int64_t)r * a.so_r + d0;
                const float inv = 1.f / fmaxf(lt, 1e-20f);
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = (half_t)(at[e] * inv);
            } else {
                // Device-coherent (write-through) stores: the group that
                // merges may run on another XCD, whose L2 does not see this
                // one's.
                store_coherent4(pacc + r * HEAD_DIM + d0, at);
                if (d0 == 0) {
                    // (m in natural-log units, the reference's format; m and l
                    // of a row side by side: the combining group reads them
                    // as one 8-byte load)
                    store_coherent2(pm + 2 * r, mg * LN2, lt);
                }
            }
        }
    }
    LS_STAMP(9);
#ifdef LS_STAMPS
    if (!SPARSE && threadIdx.x == 0) {
        uint64_t lo = wave_end[0], hi = wave_end[0];
        for (int w = 1; w < NWT; ++w) {
            lo = wave_end[w] < lo ? wave_end[w] : lo;
            hi = wave_end[w] > hi ? wave_end[w] : hi;
        }
        g_ls_stamps[(blockIdx.x + gridDim.x * blockIdx.y) * LS_NSTAMP + 1] = lo;
        g_ls_stamps[(blockIdx.x + gridDim.x * blockIdx.y) * LS_NSTAMP + 2] = hi;
    }
#endif
    if (single) return;

    // ---- the last group of each (b, h) to arrive merges all splits ----
    // Every wave's write-through record stores complete before the group's
    // arrival; the last arriver acquires before reading them.
    handoff_release();
    __syncthreads();
    LS_STAMP(10);
    if (threadIdx.x < (unsigned)HG) {
        const int64_t bh = (int64_t)b * H + h0 + threadIdx.x;
        const int prev = __hip_atomic_fetch_add(a.counters + bh * COUNTER_STRIDE, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        sm.is_last[threadIdx.x] = prev == Sb - 1;
    }
    __syncthreads();
    LS_STAMP(11);
    // a group of HG heads merges each head it closed, 256 threads a head
    const int hh = threadIdx.x / TPH, t256 = threadIdx.x % TPH;
    if (!sm.is_last[hh] || t256 >= 256) return;
    const int64_t bh = (int64_t)b * H + h0 + hh;
    {
        // device-coherent loads: the records of groups on other XCDs
        const float* recs = a.work + ((int64_t)gw.first * H + h0 + hh) * rec;
        // (a round of 32 slots for 16 splits or fewer would reread the
        // last split's record 16 times and more: c2 +1.6 us)
        half_t* o = a.out + (int64_t)b * a.so_b + (int64_t)(h0 + hh) * a.so_h;
        if (Sb <= 16)
            combine_records<16>(recs, recs + NR * HEAD_DIM, Sb, NR, (int64_t)H * rec, HEAD_DIM,
                                (int64_t)H * rec, o, a.so_r, t256);
        else
            combine_records<32>(recs, recs + NR * HEAD_DIM, Sb, NR, (int64_t)H * rec, HEAD_DIM,
                                (int64_t)H * rec, o, a.so_r, t256);
    }
    LS_STAMP(12);
    // every group of this (b, h) has arrived: back to zero for the next launch
    if (t256 == 0)
        __hip_atomic_store(a.counters + bh * COUNTER_STRIDE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (SPARSE == 3) {
        // and every group has read the count after row (b, h0) (a group
        // counts itself before it selects, and arrives here after): back to
        // all ones.  Every group serves all HG heads and arrives for them
        // together, so head h0's last arriver comes after all of them.
        if (t256 == 0 && hh == 0)
            __hip_atomic_store((uint32_t*)(a.scores + (int64_t)b * a.ssc_b +
                                           (int64_t)h0 * a.ssc_h + a.score_pages),
                               EMPTY_WORD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int VEC>
__global__ __launch_bounds__(256) void combine_kernel(CombineParams p) {
    const int bh = blockIdx.x;
    const int b = bh / p.H, h = bh % p.H;
    combine_partials<VEC>(p.acc + (int64_t)b * p.sa_b + (int64_t)h * p.sa_h,
                            p.m + (int64_t)b * p.sm_b + (int64_t)h * p.sm_h,
                            p.l + (int64_t)b * p.sm_b + (int64_t)h * p.sm_h, p.S, p.NR, p.sa_s,
                            p.sa_r, p.sm_s,
                            (char*)p.out + ((int64_t)b * p.so_b + (int64_t)h * p.so_h) *
                                               (p.out_f32 ? 4 : 2),
                            p.out_f32, p.so_r, threadIdx.x);
}

#ifdef LS_STAMPS
// Measurement build: the stamps of the last launch, copied to the host.
extern "C" int ls_diag_read_stamps(void* host, size_t bytes) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_ls_stamps), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

// ------------------------------------------------------------- launch ----

constexpr int NWAVES = 4;

template <int KIND, bool ASYM, bool HAS_RES, int SPARSE, int ABL = 0>
static hipError_t launch_t(const DecodeParams& a, hipStream_t stream) {
    // Heads in pairs when the head count allows: both halves of every token
    // row are then read together (INT8 too: c4 37.0 -> 35.8 us).  Each wave
    // holds one head's state, so asymmetric INT8's zero points fit as well.
    if (a.H % 2 == 0) {
        dim3 grid(a.num_splits * (a.H / 2), a.B);
        hipLaunchKernelGGL((paged_decode_kernel<KIND, ASYM, HAS_RES, SPARSE, 2 * NWAVES, 2, ABL>),
                           grid, dim3(WAVE * NWAVES * 2), 0, stream, a);
        return hipGetLastError();
    }
    {
        dim3 grid(a.num_splits * a.H, a.B);
        hipLaunchKernelGGL((paged_decode_kernel<KIND, ASYM, HAS_RES, SPARSE, NWAVES, 1, ABL>),
                           grid, dim3(WAVE * NWAVES), 0, stream, a);
    }
    return hipGetLastError();
}

#ifdef LS_DIAGNOSTICS
// Diagnostic builds only (-DLS_DIAGNOSTICS; never the shipped library):
// LATENTSERVE_HIP_ABLATION selects, for the fp16 dense walk and the
// symmetric INT8 walk without a residual, a variant whose output is
// meaningless:
//   loads        the walk with the arithmetic removed
//   loads_noepi  ... and without the wave merge / partials / split merge
//   noepi        the full arithmetic without the merge stages
static int ablation() {
    static const int v = [] {
        const char* e = getenv("LATENTSERVE_HIP_ABLATION");
        if (!e) return 0;
        if (strcmp(e, "loads") == 0) return 1;
        if (strcmp(e, "loads_noepi") == 0) return 2;
        if (strcmp(e, "noepi") == 0) return 3;
        return 0;
    }();
    if (v) fprintf(stderr, "latentserve_amd: LATENTSERVE_HIP_ABLATION active, output invalid\n");
    return v;
}
#endif

static hipError_t launch_kernel(const DecodeParams& a, hipStream_t stream) {
    if (a.scores && a.kmin) return launch_t<KV_FP16, false, false, 3>(a, stream);
    if (a.scores) return launch_t<KV_FP16, false, false, 2>(a, stream);
    if (a.sel) return launch_t<KV_FP16, false, false, 1>(a, stream);
#ifdef LS_DIAGNOSTICS
    if (a.kind == KV_FP16 && ablation() != 0) {
        const int abl = ablation();
        if (abl == 1) return launch_t<KV_FP16, false, false, 0, 1>(a, stream);
        if (abl == 2) return launch_t<KV_FP16, false, false, 0, 2>(a, stream);
        return launch_t<KV_FP16, false, false, 0, 3>(a, stream);
    }
#endif
    if (a.kind == KV_FP16) return launch_t<KV_FP16, false, false, 0>(a, stream);
    const bool asym = a.k_zero != nullptr, res = a.k_res != nullptr;
#ifdef LS_DIAGNOSTICS
    if (ablation() != 0 && !asym && !res) {
        const int abl = ablation();
        if (abl == 1) return launch_t<KV_INT8, false, false, 0, 1>(a, stream);
        if (abl == 2) return launch_t<KV_INT8, false, false, 0, 2>(a, stream);
        return launch_t<KV_INT8, false, false, 0, 3>(a, stream);
    }
#endif
    if (asym && res) return launch_t<KV_INT8, true, true, 0>(a, stream);
    if (asym) return launch_t<KV_INT8, true, false, 0>(a, stream);
    if (res) return launch_t<KV_INT8, false, true, 0>(a, stream);
    return launch_t<KV_INT8, false, false, 0>(a, stream);
}

template <int KIND, bool ASYM, bool HAS_RES, int SPARSE>
static hipError_t resources_t(bool pair_heads, KernelResources* r) {
    if (pair_heads)
        return func_resources(paged_decode_kernel<KIND, ASYM, HAS_RES, SPARSE, 2 * NWAVES, 2>,
                              WAVE * NWAVES * 2, r);
    return func_resources(paged_decode_kernel<KIND, ASYM, HAS_RES, SPARSE, NWAVES, 1>,
                          WAVE * NWAVES, r);
}

hipError_t decode_resources(int kind, int walk, bool asym, bool has_res, bool pair_heads,
                            KernelResources* r) {
    if (kind == KV_FP16) {
        switch (walk) {
            case 0: return resources_t<KV_FP16, false, false, 0>(pair_heads, r);
            case 1: return resources_t<KV_FP16, false, false, 1>(pair_heads, r);
            case 2: return resources_t<KV_FP16, false, false, 2>(pair_heads, r);
            case 3: return resources_t<KV_FP16, false, false, 3>(pair_heads, r);
            default: return hipErrorInvalidValue;
        }
    }
    if (walk != 0) return hipErrorInvalidValue;
    if (asym && has_res) return resources_t<KV_INT8, true, true, 0>(pair_heads, r);
    if (asym) return resources_t<KV_INT8, true, false, 0>(pair_heads, r);
    if (has_res) return resources_t<KV_INT8, false, true, 0>(pair_heads, r);
    return resources_t<KV_INT8, false, false, 0>(pair_heads, r);
}

hipError_t combine_resources(KernelResources* r) { return func_resources(combine_kernel<4>, 256, r); }

hipError_t launch_decode(const DecodeParams& a, hipStream_t stream) {
    return launch_kernel(a, stream);
}

hipError_t launch_combine(const CombineParams& p, hipStream_t stream) {
    const bool vec = (uintptr_t)p.acc % 16 == 0 && p.sa_b % 4 == 0 && p.sa_h % 4 == 0 &&
                     p.sa_s % 4 == 0 && p.sa_r % 4 == 0;
    if (vec)
        hipLaunchKernelGGL(combine_kernel<4>, dim3(p.B * p.H), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(combine_kernel<1>, dim3(p.B * p.H), dim3(256), 0, stream, p);
    return hipGetLastError();
}

#ifdef LS_DIAGNOSTICS
// ---- compute probe: the page compute alone, MFMA against VALU ----
//
// Measurement only (no counterpart in the reference).  Every wave applies
// one page (16 tokens, one KV head, 6 query rows, D = 128) `items` times to
// its running (m, l, O) state, from registers: no memory traffic, so the
// kernel's duration is the compute cost of a page.  MODE 0 is the decode
// kernel's own compute_page (QK and PV on v_mfma_f32_16x16x16f16); MODE 1 is
// a VALU formulation of the same page given every advantage: the query rows
// held in registers for the lane's channels, QK as v_dot2_f32_f16 over the
// lane's 32 channels of one token and a 4-lane sum, the softmax on 16-lane
// DPP rotations, PV with V in its natural channel-pair layout (lane l owns
// channels 2l, 2l + 1 of all 16 tokens) and the weights broadcast from
// registers.  Both write O = acc / l of each wave's 6 rows.
namespace {

constexpr int PROBE_ROWS = 6;
constexpr int PROBE_WAVES = 8;

// Synthetic page and query values, exact in fp16.
__device__ __forceinline__ half_t probe_k(int t, int ch) { return (half_t)(((t * 7 + ch * 3) % 17 - 8) * 0.0625f); }
__device__ __forceinline__ half_t probe_v(int t, int ch) { return (half_t)(((t * 5 + ch * 11) % 13 - 6) * 0.125f); }
__device__ __forceinline__ half_t probe_q(int r, int ch) { return (half_t)(((r * 13 + ch * 5) % 11 - 5) * 0.125f); }

__device__ __forceinline__ uint32_t pack_h2(half_t lo, half_t hi) {
    h2 t = {lo, hi};
    return __builtin_bit_cast(uint32_t, t);
}

// Opaque to the optimiser: the page is "new" every item (nothing hoisted).
template <typename T>
__device__ __forceinline__ void opaque(T& v) {
    asm volatile("" : "+v"(v));
}

__device__ __forceinline__ float row16_max(float v) {
    // rotations within each 16-lane row: every lane ends with the row's max
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false)));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
    return v;
}

template <int MODE>
__global__ __launch_bounds__(WAVE * PROBE_WAVES) void compute_probe_kernel(int items, float scale_log2, float* out) {
    const int lane = threadIdx.x % WAVE, c = lane & 15, g = lane >> 4;
    const int64_t w = (int64_t)blockIdx.x * PROBE_WAVES + threadIdx.x / WAVE;
    float* o = out + w * PROBE_ROWS * HEAD_DIM;
    if (MODE == 0) {
        PageBuf buf;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t d[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                d[e] = pack_h2(probe_k(c, 32 * j + 8 * g + 2 * e), probe_k(c, 32 * j + 8 * g + 2 * e + 1));
            buf.k[j] = (u4){d[0], d[1], d[2], d[3]};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t d[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                d[e] = pack_h2(probe_v(4 * g + i, 8 * c + 2 * e), probe_v(4 * g + i, 8 * c + 2 * e + 1));
            buf.v[i] = (u4){d[0], d[1], d[2], d[3]};
        }
        h4 qh[8];
        const int qr = c < PROBE_ROWS ? c : 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qh[2 * j][e] = probe_q(qr, 32 * j + 8 * g + e);
                qh[2 * j + 1][e] = probe_q(qr, 32 * j + 8 * g + 4 + e);
            }
        WaveState st;
#pragma unroll
        for (int t = 0; t < 8; ++t) st.acc[t] = (f4){0.f, 0.f, 0.f, 0.f};
        st.m = neg_inf();
        st.l = 0.f;
        st.z = 0.f;
        for (int it = 0; it < items; ++it) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                opaque(buf.k[j]);
                opaque(buf.v[j]);
            }
            compute_page<KV_FP16, false>(buf, st, qh, 0, PAGE, scale_log2, g, nullptr);
        }
        const float l = group4_sum(st.l);
        if (c < PROBE_ROWS)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[c * HEAD_DIM + 32 * g + 8 * i + jj] = st.acc[jj][i] / l;
    } else {
        // K: lane (token c, group g) holds channels 32j + 8g + [0, 8); the
        // query rows the same channels; V: lane holds channels 2 lane, 2 lane + 1
        uint32_t kk[16], qq[PROBE_ROWS][16], vv[PAGE];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int ch = 32 * j + 8 * g + 2 * e;
                kk[4 * j + e] = pack_h2(probe_k(c, ch), probe_k(c, ch + 1));
#pragma unroll
                for (int r = 0; r < PROBE_ROWS; ++r)
                    qq[r][4 * j + e] = pack_h2(probe_q(r, ch), probe_q(r, ch + 1));
            }
#pragma unroll
        for (int t = 0; t < PAGE; ++t) vv[t] = pack_h2(probe_v(t, 2 * lane), probe_v(t, 2 * lane + 1));
        float m[PROBE_ROWS], l[PROBE_ROWS], acc[PROBE_ROWS][2];
#pragma unroll
        for (int r = 0; r < PROBE_ROWS; ++r) {
            m[r] = neg_inf();
            l[r] = 0.f;
            acc[r][0] = acc[r][1] = 0.f;
        }
        for (int it = 0; it < items; ++it) {
#pragma unroll
            for (int j = 0; j < 16; ++j) opaque(kk[j]);
#pragma unroll
            for (int t = 0; t < PAGE; ++t) opaque(vv[t]);
#pragma unroll
            for (int r = 0; r < PROBE_ROWS; ++r) {
                // S[r][token c]: the lane's 32 channels, then the 4 lane groups
                float sr = 0.f;
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    sr = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, kk[j]),
                                                __builtin_bit_cast(h2, qq[r][j]), sr, false);
                sr += __shfl_xor(sr, 16);
                sr += __shfl_xor(sr, 32);
                const float x = sr * scale_log2;
                const float m_new = fmaxf(m[r], row16_max(x));
                const float alpha = fast_exp2(m[r] - m_new);
                const float p = fast_exp2(x - m_new);
                l[r] = l[r] * alpha + row16_sum(p);
                m[r] = m_new;
                acc[r][0] *= alpha;
                acc[r][1] *= alpha;
                // O[r][2 lane + e] += P[r][t] V[t][2 lane + e], P broadcast
#pragma unroll
                for (int t = 0; t < PAGE; ++t) {
                    const float pt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), t));
                    const h2 v2 = __builtin_bit_cast(h2, vv[t]);
                    acc[r][0] = fmaf(pt, (float)v2.x, acc[r][0]);
                    acc[r][1] = fmaf(pt, (float)v2.y, acc[r][1]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < PROBE_ROWS; ++r) {
            o[r * HEAD_DIM + 2 * lane] = acc[r][0] / l[r];
            o[r * HEAD_DIM + 2 * lane + 1] = acc[r][1] / l[r];
        }
    }
}

}  // namespace

hipError_t launch_compute_probe(int mode, int groups, int items, float scale, float* out,
                                hipStream_t stream) {
    const float scale_log2 = scale * LOG2E;
    if (mode == 0)
        hipLaunchKernelGGL(compute_probe_kernel<0>, dim3(groups), dim3(WAVE * PROBE_WAVES), 0, stream,
                           items, scale_log2, out);
    else
        hipLaunchKernelGGL(compute_probe_kernel<1>, dim3(groups), dim3(WAVE * PROBE_WAVES), 0, stream,
                           items, scale_log2, out);
    return hipGetLastError();
}

#endif  // LS_DIAGNOSTICS

}  // namespace ls

// ------------------------------------------------ no-allocation variant ----
//
// For callers that cannot allocate device memory (code under graph capture,
// tight serving loops): the fp16 decode with its split workspace and arrival
// counters in one fixed device array of this library instead of caller
// buffers.  Each GPU holds its own copy (until the process ends), found by
// its address on that device; every call on a GPU shares it, so calls that
// overlap on one GPU race.  The counters are cleared once per device at the
// first call and are left at zero by every call after (the last workgroup of
// each (sequence, head) resets its own).

static __device__ __align__(256) unsigned char scratch[ls::NOALLOC_WORK_BYTES +
                                                        ls::NOALLOC_COUNTERS * sizeof(int32_t)];

namespace ls {
namespace {

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

__global__ __launch_bounds__(256) void zero_i32_kernel(int32_t* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace

hipError_t noalloc_scratch(hipStream_t stream, float** work, int32_t** counters) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        // The array is zero when the code object is loaded (a static
        // __device__ array with no initializer), so the counters start at
        // zero; they are cleared once more here unless the first call is
        // being captured into a graph, where the clear would only be
        // recorded (and re-run by every replay), not run now.
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cap);
        if (e != hipSuccess) return e;
        if (cap == hipStreamCaptureStatusNone) {
            int32_t* cnt = reinterpret_cast<int32_t*>(static_cast<unsigned char*>(p) +
                                                      NOALLOC_WORK_BYTES);
            hipLaunchKernelGGL(zero_i32_kernel, dim3((NOALLOC_COUNTERS + 255) / 256), dim3(256), 0,
                               stream, cnt, NOALLOC_COUNTERS);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        g_scratch_ptr[dev] = p;
    }
    unsigned char* base = static_cast<unsigned char*>(g_scratch_ptr[dev]);
    *work = reinterpret_cast<float*>(base);
    *counters = reinterpret_cast<int32_t*>(base + NOALLOC_WORK_BYTES);
    return hipSuccess;
}

}  // namespace ls
