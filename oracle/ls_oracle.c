/*
 * CPU oracle for the paged GQA decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (latentserve_amd/) links,
 * loads or calls this file.  It is the checker that the HIP kernels are
 * compared against in tests/, in __graft_entry__.smoke(), and the CPU
 * baseline leg of bench.py.
 *
 * Each function restates, in plain fp32 C, one algorithm of the reference
 * (Jash-Vora/LatentServe).  Citations are file:line in that repository.
 *
 *   ls_ref_paged_decode    kernels/gqa/paged_decode.py:152-269 (per sequence,
 *                          per KV head, per split, per page online softmax;
 *                          split combine at :253-267), dequant at :122-148,
 *                          INT8 K residual read at :213-216.
 *   ls_ref_sparse_decode   kernels/cuda/paged_sparse_fp16.cu:205-329 (page
 *                          list, in-kernel budget at :242-247, skip of pages
 *                          past the end at :266); attention per page as above.
 *   ls_ref_combine         kernels/gqa/paged_decode.py:689-706.
 *   ls_ref_quantize_k      cache/int8_paged_cache.py:670-699 (_finalize_blocks).
 *   ls_ref_quantize_v      cache/int8_paged_cache.py:741-758 (write(), V part).
 *   ls_ref_page_scores     kernels/cuda/paged_sparse_fp16.cu:78-130 and
 *                          model/attention/sparse.py:57-74, 132-134.
 *   ls_ref_page_scores_mass kernels/cuda/paged_sparse.py:126-161 and
 *                          kernels/cuda/paged_sparse_fp16.cu:141-190.
 *   ls_ref_bounds_update   kernels/cuda/paged_sparse_fp16.cu:54-72 and
 *                          cache/paged_cache.py:452-465.
 *   ls_ref_gather          cache/paged_cache.py:486-506 and
 *                          cache/block_allocator.py:214-220 (slot rule).
 *
 * Arithmetic is fp32 with no contraction (build with -ffp-contract=off) so a
 * multiply followed by an add rounds twice, as the torch ops do.  Integer
 * codes use round-half-to-even (rintf, torch.round).  The quantizers take
 * `recip`: torch divides a tensor by a Python number as an IEEE division on
 * the CPU (recip = 0) and as a multiply by the fp32 reciprocal formed on the
 * host on a GPU (recip = 1, also what kernels/cuda/int8_write.cu:20-24, 62-73
 * computes); tensor-by-tensor divisions are IEEE divisions either way.
 *
 * fp16 values cross this boundary as raw uint16 bit patterns.  Strides are in
 * elements.  All (b, head) pairs are independent and are spread over OpenMP
 * threads; each writes only its own output rows.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 -- */

static float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                       /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; ++e; } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float ls_ref_h2f(uint16_t h) { return h2f(h); }

int ls_ref_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void ls_ref_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------- shared types --- */

/* Everything one attention call reads.  kv_kind: 0 = fp16 pools, 1 = int8. */
typedef struct {
    const uint16_t* q; int64_t sq_b, sq_h, sq_r;          /* [B, H, NR, D] fp16 */
    const void* k_pool; const void* v_pool;               /* [nb, PAGE, H, D]   */
    int64_t sk_b, sk_p, sk_h;                              /* shared by K and V  */
    int kv_kind;
    const float* k_scale; int64_t sks_b, sks_h;           /* [nb, H, D]         */
    const float* v_scale; int64_t svs_b, svs_p, svs_h;    /* [nb, PAGE, H]      */
    const float* k_zero; const float* v_zero;             /* same strides       */
    const uint16_t* k_res; int64_t sr_r, sr_p, sr_h;      /* [R, PAGE, H, D]    */
    const int32_t* res_rows;                              /* [B]                */
    const int32_t* block_tables; int64_t sbt_b;           /* [B, maxP]          */
    const int32_t* seq_lens;                              /* [B]                */
    int B, H, NR, D, PAGE;
    float scale;
} ls_ref_args;

/* Dequantised K row for (blk, token, head) into out[D] (fp32), following
 * _dequant_k: q.to(f32) * scale[ch] (+ zero[ch]).  For an fp16 pool it is the
 * exact widening. */
static void k_row(const ls_ref_args* a, int blk, int tok, int h, float* out) {
    const int64_t base = (int64_t)blk * a->sk_b + (int64_t)tok * a->sk_p + (int64_t)h * a->sk_h;
    if (a->kv_kind == 0) {
        const uint16_t* p = (const uint16_t*)a->k_pool + base;
        for (int d = 0; d < a->D; ++d) out[d] = h2f(p[d]);
        return;
    }
    const int8_t* p = (const int8_t*)a->k_pool + base;
    const float* s = a->k_scale ? a->k_scale + (int64_t)blk * a->sks_b + (int64_t)h * a->sks_h : NULL;
    const float* z = a->k_zero ? a->k_zero + (int64_t)blk * a->sks_b + (int64_t)h * a->sks_h : NULL;
    for (int d = 0; d < a->D; ++d) {
        float v = (float)p[d];
        if (s) {
            v = v * s[d];
            if (z) v = v + z[d];
        }
        out[d] = v;
    }
}

/* Dequantised V row: q.to(f32) * scale[tok] (+ zero[tok]) (_dequant_v). */
static void v_row(const ls_ref_args* a, int blk, int tok, int h, float* out) {
    const int64_t base = (int64_t)blk * a->sk_b + (int64_t)tok * a->sk_p + (int64_t)h * a->sk_h;
    if (a->kv_kind == 0) {
        const uint16_t* p = (const uint16_t*)a->v_pool + base;
        for (int d = 0; d < a->D; ++d) out[d] = h2f(p[d]);
        return;
    }
    const int8_t* p = (const int8_t*)a->v_pool + base;
    const int64_t si = (int64_t)blk * a->svs_b + (int64_t)tok * a->svs_p + (int64_t)h * a->svs_h;
    const float s = a->v_scale ? a->v_scale[si] : 1.0f;
    const float z = a->v_zero ? a->v_zero[si] : 0.0f;
    for (int d = 0; d < a->D; ++d) {
        float v = (float)p[d];
        if (a->v_scale) {
            v = v * s;
            if (a->v_zero) v = v + z;
        }
        out[d] = v;
    }
}

/* Online-softmax state of one split for one (b, head): m[NR], l[NR], acc[NR*D]. */
typedef struct { float* m; float* l; float* acc; } split_state;

/* Attend one logical page p of sequence b, head h into state st
 * (kernels/gqa/paged_decode.py:211-247). */
static void attend_page(const ls_ref_args* a, int b, int h, int p, int length, int num_pages,
                        const float* qi, split_state st, float* kbuf, float* vbuf, float* qk,
                        float* pw) {
    const int D = a->D, NR = a->NR, PAGE = a->PAGE;
    const int blk = a->block_tables[(int64_t)b * a->sbt_b + p];
    for (int t = 0; t < PAGE; ++t) {
        if (a->k_res && p == num_pages - 1) {
            /* The last page's K is exact fp16 in the residual (:213-216). */
            const uint16_t* r = a->k_res + (int64_t)a->res_rows[b] * a->sr_r + (int64_t)t * a->sr_p
                                + (int64_t)h * a->sr_h;
            for (int d = 0; d < D; ++d) kbuf[t * D + d] = h2f(r[d]);
        } else {
            k_row(a, blk, t, h, kbuf + t * D);
        }
        v_row(a, blk, t, h, vbuf + t * D);
    }
    for (int r = 0; r < NR; ++r) {
        float mx = -INFINITY;
        for (int t = 0; t < PAGE; ++t) {
            const int valid = p * PAGE + t < length;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += qi[r * D + d] * kbuf[t * D + d];
            qk[t] = valid ? dot * a->scale : -INFINITY;
            if (qk[t] > mx) mx = qk[t];
        }
        const float m_new = st.m[r] > mx ? st.m[r] : mx;
        /* A page entirely past the end leaves m_new at -inf: alpha is forced
         * to zero there rather than exp(-inf - -inf) = NaN (:236-242). */
        const float alpha = isinf(m_new) ? 0.0f : expf(st.m[r] - m_new);
        float sum = 0.0f;
        for (int t = 0; t < PAGE; ++t) {
            const int valid = p * PAGE + t < length;
            pw[t] = valid ? expf(qk[t] - m_new) : 0.0f;
            sum += pw[t];
        }
        st.l[r] = st.l[r] * alpha + sum;
        for (int d = 0; d < D; ++d) {
            float pv = 0.0f;
            for (int t = 0; t < PAGE; ++t) pv += pw[t] * vbuf[t * D + d];
            st.acc[r * D + d] = st.acc[r * D + d] * alpha + pv;
        }
        st.m[r] = m_new;
    }
}

/* Merge S split states into out (fp32 [NR, D] at out_row stride D), the
 * combine at kernels/gqa/paged_decode.py:258-267. */
static void merge_states(int S, int NR, int D, const float* m, const float* l, const float* acc,
                         float* out, int64_t so_r) {
    for (int r = 0; r < NR; ++r) {
        float mg = -INFINITY;
        for (int s = 0; s < S; ++s)
            if (m[s * NR + r] > mg) mg = m[s * NR + r];
        float lt = 0.0f;
        for (int s = 0; s < S; ++s) {
            const float w = isinf(mg) ? 0.0f : expf(m[s * NR + r] - mg);
            lt += l[s * NR + r] * w;
        }
        const float den = lt > 1e-20f ? lt : 1e-20f;
        for (int d = 0; d < D; ++d) {
            float at = 0.0f;
            for (int s = 0; s < S; ++s) {
                const float w = isinf(mg) ? 0.0f : expf(m[s * NR + r] - mg);
                at += acc[((int64_t)s * NR + r) * D + d] * w;
            }
            out[r * so_r + d] = at / den;
        }
    }
}

/* One (b, head) of either the dense or the page-list walk.  `pages` is NULL
 * for the dense walk (logical pages 0..num_pages-1), else a list of n logical
 * pages of which entries outside [0, num_pages) are skipped. */
static void run_pair(const ls_ref_args* a, int b, int h, int num_splits, const int32_t* pages,
                     int n_list, float* out, int64_t so_b, int64_t so_h, int64_t so_r) {
    const int D = a->D, NR = a->NR, PAGE = a->PAGE;
    const int length = a->seq_lens[b];
    const int num_pages = (length + PAGE - 1) / PAGE;
    const int n = pages ? n_list : num_pages;
    const int per = n > 0 ? ((n + num_splits - 1) / num_splits) : 1;
    const int pps = per < 1 ? 1 : per;

    float* qi = (float*)malloc(sizeof(float) * NR * D);
    float* kbuf = (float*)malloc(sizeof(float) * PAGE * D);
    float* vbuf = (float*)malloc(sizeof(float) * PAGE * D);
    float* qk = (float*)malloc(sizeof(float) * PAGE);
    float* pw = (float*)malloc(sizeof(float) * PAGE);
    float* m = (float*)malloc(sizeof(float) * num_splits * NR);
    float* l = (float*)malloc(sizeof(float) * num_splits * NR);
    float* acc = (float*)malloc(sizeof(float) * (size_t)num_splits * NR * D);

    for (int r = 0; r < NR; ++r)
        for (int d = 0; d < D; ++d)
            qi[r * D + d] = h2f(a->q[(int64_t)b * a->sq_b + (int64_t)h * a->sq_h + (int64_t)r * a->sq_r + d]);

    int used = 0;                      /* splits that had work (:253 `partial_acc`) */
    for (int s = 0; s < num_splits; ++s) {
        const int lo = s * pps;
        const int hi = lo + pps < n ? lo + pps : n;
        if (lo >= hi) continue;        /* empty split contributes nothing (:204) */
        split_state st = {m + used * NR, l + used * NR, acc + (size_t)used * NR * D};
        for (int r = 0; r < NR; ++r) {
            st.m[r] = -INFINITY;
            st.l[r] = 0.0f;
            for (int d = 0; d < D; ++d) st.acc[r * D + d] = 0.0f;
        }
        for (int i = lo; i < hi; ++i) {
            const int p = pages ? pages[i] : i;
            if (p < 0 || p >= num_pages) continue;
            attend_page(a, b, h, p, length, num_pages, qi, st, kbuf, vbuf, qk, pw);
        }
        ++used;
    }
    float* o = out + (int64_t)b * so_b + (int64_t)h * so_h;
    if (used == 0) {
        for (int r = 0; r < NR; ++r)
            for (int d = 0; d < D; ++d) o[r * so_r + d] = 0.0f;
    } else {
        merge_states(used, NR, D, m, l, acc, o, so_r);
    }
    free(qi); free(kbuf); free(vbuf); free(qk); free(pw); free(m); free(l); free(acc);
}

/* paged_decode_reference (kernels/gqa/paged_decode.py:152-269).
 * out: fp32 [B, H, NR, D] with the given strides. */
void ls_ref_paged_decode(const ls_ref_args* a, int num_splits, float* out, int64_t so_b,
                         int64_t so_h, int64_t so_r) {
    if (num_splits < 1) num_splits = 1;
    const int pairs = a->B * a->H;
#pragma omp parallel for schedule(dynamic, 1)
    for (int i = 0; i < pairs; ++i)
        run_pair(a, i / a->H, i % a->H, num_splits, NULL, 0, out, so_b, so_h, so_r);
}

/* In-kernel budget of paged_sparse_fp16.cu:242-247: with ratio > 0 each
 * sequence attends to the first max(recent+1, ceilf(ratio*pages)) entries of
 * its (score-sorted) list, capped at its pages and the list length. */
int ls_ref_sparse_count(int num_pages, int num_sel, float ratio, int recent) {
    int n = num_sel;
    if (ratio > 0.0f) {
        int want;
        if (ratio >= 1.0f) {
            want = num_pages;
        } else {
            const int c = (int)ceilf(ratio * (float)num_pages);
            want = c > recent + 1 ? c : recent + 1;
        }
        if (want > num_pages) want = num_pages;
        n = want < num_sel ? want : num_sel;
    }
    return n;
}

/* sparse_decode: attention over sel[b, h, 0:n] logical pages only. */
void ls_ref_sparse_decode(const ls_ref_args* a, const int32_t* sel, int64_t ssel_b, int64_t ssel_h,
                          int num_sel, float ratio, int recent, int num_splits, float* out,
                          int64_t so_b, int64_t so_h, int64_t so_r) {
    if (num_splits < 1) num_splits = 1;
    const int pairs = a->B * a->H;
#pragma omp parallel for schedule(dynamic, 1)
    for (int i = 0; i < pairs; ++i) {
        const int b = i / a->H, h = i % a->H;
        const int num_pages = (a->seq_lens[b] + a->PAGE - 1) / a->PAGE;
        const int n = ls_ref_sparse_count(num_pages, num_sel, ratio, recent);
        run_pair(a, b, h, num_splits, sel + (int64_t)b * ssel_b + (int64_t)h * ssel_h, n, out, so_b,
                 so_h, so_r);
    }
}

/* combine_splits (kernels/gqa/paged_decode.py:689-706).
 * acc fp32 [B, H, S, NR, D], m/l fp32 [B, H, S, NR] contiguous; out fp32 [B, H, NR, D]. */
void ls_ref_combine(int B, int H, int S, int NR, int D, const float* acc, const float* m,
                    const float* l, float* out) {
    for (int bh = 0; bh < B * H; ++bh)
        merge_states(S, NR, D, m + (int64_t)bh * S * NR, l + (int64_t)bh * S * NR,
                     acc + (int64_t)bh * S * NR * D, out + (int64_t)bh * NR * D, D);
}

/* ------------------------------------------------------------ INT8 ------ */

/* _finalize_blocks (cache/int8_paged_cache.py:670-699).
 * data fp16 [N, PAGE, H, D] contiguous -> codes int8 [N, PAGE, H, D],
 * step fp32 [N, H, D], zero fp32 [N, H, D] (asym only).
 * Symmetric: step = max(amax_tok |f|, eps) / qmax; q = clamp(rint(f/step), -qmax, qmax).
 * Asymmetric: step = max((hi - lo) / levels, eps); u = clamp(rint((f - lo)/step), 0, levels);
 * q = u - offset; zero = lo + offset * step. */
void ls_ref_quantize_k(const uint16_t* data, int N, int PAGE, int H, int D, int asym, float eps,
                       float qmax, float levels, float offset, int recip, int8_t* codes,
                       float* step, float* zero) {
    const float inv_qmax = 1.0f / qmax, inv_levels = 1.0f / levels;
#pragma omp parallel for schedule(static)
    for (int64_t nh = 0; nh < (int64_t)N * H; ++nh) {
        const int64_t n = nh / H;
        const int h = (int)(nh % H);
        for (int d = 0; d < D; ++d) {
            const int64_t sidx = (n * H + h) * D + d;
            float lo = INFINITY, hi = -INFINITY, amax = 0.0f;
            for (int t = 0; t < PAGE; ++t) {
                const float f = h2f(data[((n * PAGE + t) * H + h) * D + d]);
                const float af = fabsf(f);
                if (af > amax) amax = af;
                if (f < lo) lo = f;
                if (f > hi) hi = f;
            }
            float s;
            if (asym) {
                s = recip ? (hi - lo) * inv_levels : (hi - lo) / levels;
                if (s < eps) s = eps;
                zero[sidx] = lo + offset * s;
            } else {
                const float m = amax < eps ? eps : amax;
                s = recip ? m * inv_qmax : m / qmax;
            }
            step[sidx] = s;
            for (int t = 0; t < PAGE; ++t) {
                const int64_t ci = ((n * PAGE + t) * H + h) * D + d;
                const float f = h2f(data[ci]);
                float q;
                if (asym) {
                    q = rintf((f - lo) / s);
                    q = q < 0.0f ? 0.0f : (q > levels ? levels : q);
                    q = q - offset;
                } else {
                    q = rintf(f / s);
                    q = q < -qmax ? -qmax : (q > qmax ? qmax : q);
                }
                codes[ci] = (int8_t)(int)q;
            }
        }
    }
}

/* V's per-token quantizer (cache/int8_paged_cache.py:741-758).
 * v fp16 [T, H, D] contiguous -> codes int8 [T, H, D], step/zero fp32 [T, H]. */
void ls_ref_quantize_v(const uint16_t* v, int T, int H, int D, int asym, float eps, float qmax,
                       float levels, float offset, int recip, int8_t* codes, float* step,
                       float* zero) {
    const float inv_qmax = 1.0f / qmax, inv_levels = 1.0f / levels;
#pragma omp parallel for schedule(static)
    for (int64_t th = 0; th < (int64_t)T * H; ++th) {
        const uint16_t* row = v + th * D;
        float lo = INFINITY, hi = -INFINITY, amax = 0.0f;
        for (int d = 0; d < D; ++d) {
            const float f = h2f(row[d]);
            const float af = fabsf(f);
            if (af > amax) amax = af;
            if (f < lo) lo = f;
            if (f > hi) hi = f;
        }
        float s;
        if (asym) {
            s = recip ? (hi - lo) * inv_levels : (hi - lo) / levels;
            if (s < eps) s = eps;
            zero[th] = lo + offset * s;
        } else {
            const float m = amax < eps ? eps : amax;
            s = recip ? m * inv_qmax : m / qmax;
        }
        step[th] = s;
        for (int d = 0; d < D; ++d) {
            const float f = h2f(row[d]);
            float q;
            if (asym) {
                q = rintf((f - lo) / s);
                q = q < 0.0f ? 0.0f : (q > levels ? levels : q);
                q = q - offset;
            } else {
                q = rintf(f / s);
                q = q < -qmax ? -qmax : (q > qmax ? qmax : q);
            }
            codes[th * D + d] = (int8_t)(int)q;
        }
    }
}

/* ---------------------------------------------------------- selector ---- */

/* page_index (paged_sparse_fp16.cu:78-130): per (b, h, page) the Quest bound
 * max_r sum_d max(q_rd * kmin_d, q_rd * kmax_d); +inf for page 0 and the last
 * `recent` pages, -inf past the end.  kmin/kmax fp16 [nb, H, D] strides
 * (sb_b, sb_h); scores fp32 [B, H, maxP] contiguous. */
void ls_ref_page_scores(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_r,
                        const uint16_t* kmin, const uint16_t* kmax, int64_t sb_b, int64_t sb_h,
                        const int32_t* block_tables, int64_t sbt_b, const int32_t* seq_lens,
                        int B, int H, int NR, int D, int PAGE, int max_pages, int recent,
                        float* scores) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const int np = (seq_lens[b] + PAGE - 1) / PAGE;
        for (int p = 0; p < max_pages; ++p) {
            float out;
            if (p >= np) {
                out = -INFINITY;
            } else if (p == 0 || p >= np - recent) {
                out = INFINITY;
            } else {
                const int blk = block_tables[(int64_t)b * sbt_b + p];
                const uint16_t* mn = kmin + (int64_t)blk * sb_b + (int64_t)h * sb_h;
                const uint16_t* mx = kmax + (int64_t)blk * sb_b + (int64_t)h * sb_h;
                out = -INFINITY;
                for (int r = 0; r < NR; ++r) {
                    const uint16_t* qr = q + (int64_t)b * sq_b + (int64_t)h * sq_h + (int64_t)r * sq_r;
                    float s = 0.0f;
                    for (int d = 0; d < D; ++d) {
                        const float qd = h2f(qr[d]);
                        const float x = qd * h2f(mn[d]), y = qd * h2f(mx[d]);
                        s += x > y ? x : y;
                    }
                    if (s > out) out = s;
                }
            }
            scores[(int64_t)bh * max_pages + p] = out;
        }
    }
}

/* Summed-mass page scores (kernels/cuda/paged_sparse.py:126-161, per-head
 * bounds of paged_sparse_fp16.cu:141-190): for each query head r the bound
 * b_r(p) = sum_d max(q_d lo_d, q_d hi_d), logits b_r(p) * scale + log(count
 * of tokens in page p) (count 0, so -inf, past the end), a softmax over the
 * row's max_pages pages (max subtracted, expf, fp32 sum in page order), the
 * softmaxes summed over r; page 0 and the last `recent` pages +inf, pages
 * past the end -inf.  scores fp32 [B, H, max_pages]. */
void ls_ref_page_scores_mass(const uint16_t* q, int64_t sq_b, int64_t sq_h, int64_t sq_r,
                             const uint16_t* kmin, const uint16_t* kmax, int64_t sb_b,
                             int64_t sb_h, const int32_t* block_tables, int64_t sbt_b,
                             const int32_t* seq_lens, int B, int H, int NR, int D, int PAGE,
                             int max_pages, int recent, float scale, float* scores) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const int L = seq_lens[b];
        const int np = (L + PAGE - 1) / PAGE;
        float* out = scores + (int64_t)bh * max_pages;
        float* logit = (float*)malloc(sizeof(float) * (size_t)max_pages);
        for (int p = 0; p < max_pages; ++p) out[p] = 0.0f;
        for (int r = 0; r < NR; ++r) {
            const uint16_t* qr = q + (int64_t)b * sq_b + (int64_t)h * sq_h + (int64_t)r * sq_r;
            float mx = -INFINITY;
            for (int p = 0; p < max_pages; ++p) {
                int cnt = L - p * PAGE;
                cnt = cnt < 0 ? 0 : (cnt > PAGE ? PAGE : cnt);
                if (cnt == 0) {
                    logit[p] = -INFINITY;
                    continue;
                }
                const int blk = block_tables[(int64_t)b * sbt_b + p];
                const uint16_t* mn = kmin + (int64_t)blk * sb_b + (int64_t)h * sb_h;
                const uint16_t* mxp = kmax + (int64_t)blk * sb_b + (int64_t)h * sb_h;
                float s = 0.0f;
                for (int d = 0; d < D; ++d) {
                    const float qd = h2f(qr[d]);
                    const float x = qd * h2f(mn[d]), y = qd * h2f(mxp[d]);
                    s += x > y ? x : y;
                }
                const float bs = s * scale;
                logit[p] = bs + logf((float)cnt);
                if (logit[p] > mx) mx = logit[p];
            }
            if (mx == -INFINITY) continue;
            float sum = 0.0f;
            for (int p = 0; p < max_pages; ++p) sum += expf(logit[p] - mx);
            for (int p = 0; p < max_pages; ++p) out[p] += expf(logit[p] - mx) / sum;
        }
        for (int p = 0; p < max_pages; ++p) {
            if (p >= np) out[p] = -INFINITY;
            else if (p == 0 || p >= np - recent) out[p] = INFINITY;
        }
        free(logit);
    }
}

/* Running per-page bounds on write (paged_sparse_fp16.cu:54-72): the first
 * token of a page resets, later tokens widen.  k_new fp16 [B, H, D]
 * contiguous; slots int64 [B]; kmin/kmax fp16 [nb, H, D] contiguous. */
void ls_ref_bounds_update(const uint16_t* k_new, const int64_t* slots, int B, int H, int D,
                          int PAGE, uint16_t* kmin, uint16_t* kmax) {
    for (int b = 0; b < B; ++b) {
        const int64_t blk = slots[b] / PAGE;
        const int off = (int)(slots[b] % PAGE);
        for (int h = 0; h < H; ++h)
            for (int d = 0; d < D; ++d) {
                const uint16_t v = k_new[((int64_t)b * H + h) * D + d];
                const int64_t i = (blk * H + h) * D + d;
                if (off == 0) {
                    kmin[i] = v;
                    kmax[i] = v;
                } else {
                    if (h2f(v) < h2f(kmin[i])) kmin[i] = v;
                    if (h2f(v) > h2f(kmax[i])) kmax[i] = v;
                }
            }
    }
}

/* ------------------------------------------------------------ gather ---- */

/* The gather read path (cache/paged_cache.py:486-506 with _build_read_slots,
 * :305-323): token p < L of sequence b lives at flat slot
 * blocks[p / PAGE] * PAGE + p % PAGE; positions past a sequence's length
 * read flat slot 0 (the reference pads its slot table with 0 and leaves the
 * masking to the caller).  pool [nb, PAGE, H, D] of `elem`-byte elements,
 * contiguous; out [B, H, Lmax, D] contiguous. */
void ls_ref_gather(const void* pool, int elem, const int32_t* block_tables, int64_t sbt_b,
                   const int32_t* seq_lens, int B, int H, int D, int PAGE, int Lmax, void* out) {
    const char* src = (const char*)pool;
    char* dst = (char*)out;
    for (int b = 0; b < B; ++b) {
        const int L = seq_lens[b];
        for (int p = 0; p < Lmax; ++p) {
            const int64_t slot =
                p < L ? (int64_t)block_tables[(int64_t)b * sbt_b + p / PAGE] * PAGE + p % PAGE : 0;
            for (int h = 0; h < H; ++h)
                memcpy(dst + ((((int64_t)b * H + h) * Lmax + p) * D) * elem,
                       src + ((slot * H + h) * D) * elem, (size_t)D * elem);
        }
    }
}
