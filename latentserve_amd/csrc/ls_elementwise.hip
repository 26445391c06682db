// Fused elementwise kernels of the decode step on gfx950: RMSNorm with the
// residual add folded in, SiLU-and-multiply, RoPE, and the decode-token
// RoPE + KV-store + query fold.
//
// Reference: kernels/fused_elementwise.py (rms_norm_ref :75-80,
// fused_add_rms_norm_ref :83-85, silu_and_mul_ref :88-90, rope_qk_ref
// :98-110; their launchers :194-252), which reproduce Hugging Face's Qwen2
// computation in fp16: every product, sum and cast below rounds to fp16
// where that computation does, in its order.  The decode-token kernel
// replaces three separate steps of the reference's decode layer:
// rope_qk (model/attention/gqa.py:251-253), the paged-cache store of the new
// K/V rows (cache/paged_cache.py write) and the query fold to
// [B, H_kv, n_rep, D] (model/attention/gqa.py:290-341).
//
// Each launch moves a few hundred kilobytes at decode batch sizes: the
// kernels are latency-bound, so the design goal is one launch per fused op
// with one memory round trip, not bandwidth.
#include "ls_common.h"
#include "ls_elementwise.h"

#pragma clang fp contract(off)

namespace ls {

namespace {

__device__ __forceinline__ float f(half_t h) { return (float)h; }
__device__ __forceinline__ half_t hf(float v) { return (half_t)v; }


__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Sum over a 256-thread block, returned to every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    if (threadIdx.x % WAVE == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ void unpack8(u4 v, half_t* h) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 t = __builtin_bit_cast(h2, w[i]);
        h[2 * i] = t.x;
        h[2 * i + 1] = t.y;
    }
}
__device__ __forceinline__ u4 pack8(const half_t* h) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2 t;
        t.x = h[2 * i];
        t.y = h[2 * i + 1];
        w[i] = __builtin_bit_cast(uint32_t, t);
    }
    u4 r;
    r.x = w[0];
    r.y = w[1];
    r.z = w[2];
    r.w = w[3];
    return r;
}

constexpr int NORM_THREADS = 256;
constexpr int NORM_MAXV = 4;          // 16-byte vectors a thread keeps: n <= 8192

// One row per block; the row's (summed) values stay in registers between
// the variance and the scaling.
// x row of output row `row`: itself, or the table row its id names.
__device__ __forceinline__ int64_t x_row(const NormParams& a, int64_t row) {
    if (!a.ids) return row;
    const int64_t id = a.ids[row];
    return id < 0 ? 0 : id >= a.id_rows ? a.id_rows - 1 : id;
}

template <bool RES>
__global__ __launch_bounds__(NORM_THREADS) void rms_norm_vec_kernel(NormParams a) {
    __shared__ float red[NORM_THREADS / WAVE];
    const int64_t row = blockIdx.x;
    const half_t* x = (const half_t*)a.x + x_row(a, row) * a.sx;
    const half_t* r = (const half_t*)a.res + row * a.sr;
    half_t* ro = (half_t*)a.res_out + row * a.sro;
    half_t* y = (half_t*)a.y + row * a.sy;
    const half_t* w = (const half_t*)a.w;
    half_t s[NORM_MAXV][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NORM_MAXV; ++k) {
        const int i = (threadIdx.x + k * NORM_THREADS) * 8;
        if (i < a.n) {
            unpack8(*(const u4*)(x + i), s[k]);
            if (RES) {
                half_t rv[8];
                unpack8(*(const u4*)(r + i), rv);
#pragma unroll
                for (int e = 0; e < 8; ++e) s[k][e] = hf(f(rv[e]) + f(s[k][e]));
                *(u4*)(ro + i) = pack8(s[k]);
            } else if (a.res_out) {
                *(u4*)(ro + i) = pack8(s[k]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += f(s[k][e]) * f(s[k][e]);
        }
    }
    const float var = block_sum(ss, red) / (float)a.n;
    const float inv = 1.f / sqrtf(var + a.eps);
#pragma unroll
    for (int k = 0; k < NORM_MAXV; ++k) {
        const int i = (threadIdx.x + k * NORM_THREADS) * 8;
        if (i < a.n) {
            half_t wv[8], o[8];
            unpack8(*(const u4*)(w + i), wv);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = hf(f(wv[e]) * f(hf(f(s[k][e]) * inv)));
            *(u4*)(y + i) = pack8(o);
        }
    }
}

// Any width and alignment: element loop, the summed row re-read from
// res_out (or x) for the scaling pass.
template <bool RES>
__global__ __launch_bounds__(NORM_THREADS) void rms_norm_any_kernel(NormParams a) {
    __shared__ float red[NORM_THREADS / WAVE];
    const int64_t row = blockIdx.x;
    const half_t* x = (const half_t*)a.x + x_row(a, row) * a.sx;
    const half_t* r = (const half_t*)a.res + row * a.sr;
    half_t* ro = (half_t*)a.res_out + row * a.sro;
    half_t* y = (half_t*)a.y + row * a.sy;
    const half_t* w = (const half_t*)a.w;
    float ss = 0.f;
    for (int i = threadIdx.x; i < a.n; i += NORM_THREADS) {
        half_t v = x[i];
        if (RES) {
            v = hf(f(r[i]) + f(v));
            ro[i] = v;
        } else if (a.res_out) {
            ro[i] = v;
        }
        ss += f(v) * f(v);
    }
    const float var = block_sum(ss, red) / (float)a.n;
    const float inv = 1.f / sqrtf(var + a.eps);
    for (int i = threadIdx.x; i < a.n; i += NORM_THREADS) {
        // each thread re-reads the elements it summed (its own writes)
        const half_t v = RES ? ro[i] : x[i];
        y[i] = hf(f(w[i]) * f(hf(f(v) * inv)));
    }
}

__global__ __launch_bounds__(256) void silu_mul_vec_kernel(SiluParams a) {
    const int64_t row = blockIdx.y;
    const int i = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (i >= a.inter) return;
    const half_t* gu = (const half_t*)a.gu + row * a.sgu;
    half_t g[8], u[8], o[8];
    unpack8(*(const u4*)(gu + i), g);
    unpack8(*(const u4*)(gu + a.inter + i), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = silu_mul_h(g[e], u[e]);
    *(u4*)((half_t*)a.out + row * a.so + i) = pack8(o);
}

__global__ __launch_bounds__(256) void silu_mul_any_kernel(SiluParams a) {
    const int64_t row = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.inter) return;
    const half_t* gu = (const half_t*)a.gu + row * a.sgu;
    ((half_t*)a.out)[row * a.so + i] = silu_mul_h(gu[i], gu[a.inter + i]);
}

// grid (rows, hq + hk), d / 2 threads: thread i rotates the pair (i, i + d/2).
__global__ __launch_bounds__(512) void rope_qk_kernel(RopeParams a) {
    const int64_t r = blockIdx.x;
    const int j = blockIdx.y, i = threadIdx.x, hd = a.d / 2;
    const bool isq = j < a.hq;
    const int h = isq ? j : j - a.hq;
    const half_t* src = (isq ? (const half_t*)a.q + r * a.sq : (const half_t*)a.k + r * a.sk) +
                        (int64_t)h * a.d;
    half_t* dst = (isq ? (half_t*)a.qo + r * a.sqo : (half_t*)a.ko + r * a.sko) + (int64_t)h * a.d;
    const half_t* c = (const half_t*)a.cos + r * a.sc;
    const half_t* s = (const half_t*)a.sin + r * a.ss;
    const half_t x0 = src[i], x1 = src[i + hd];
    dst[i] = rope_h(x0, c[i], -x1, s[i]);
    dst[i + hd] = rope_h(x1, c[i + hd], x0, s[i + hd]);
}

// grid (hq + 2 hk, B), d / 2 threads.  Heads [0, hq) are queries, then hk
// keys, then hk values.
__global__ __launch_bounds__(512) void rope_write_decode_kernel(RopeWriteParams a) {
    const int64_t b = blockIdx.y;
    const int j = blockIdx.x, i = threadIdx.x, hd = a.d / 2;
    const half_t* row = (const half_t*)a.qkv + b * a.sqkv + (int64_t)j * a.d;
    int64_t p = a.pos[b];
    p = p < 0 ? 0 : (p >= a.tab_rows ? a.tab_rows - 1 : p);
    const half_t* c = (const half_t*)a.cos + p * a.st;
    const half_t* s = (const half_t*)a.sin + p * a.st;
    const half_t x0 = row[i], x1 = row[i + hd];
    if (j < a.hq) {
        const int n_rep = a.hq / a.hk;
        half_t* dst = (half_t*)a.q_out + b * a.sq_b + (int64_t)(j / n_rep) * a.sq_h +
                      (int64_t)(j % n_rep) * a.sq_r;
        dst[i] = rope_h(x0, c[i], -x1, s[i]);
        dst[i + hd] = rope_h(x1, c[i + hd], x0, s[i + hd]);
        return;
    }
    const int64_t slot = a.slots[b];
    if (slot < 0) return;
    const int64_t blk = slot / a.page, off = slot % a.page;
    if (blk >= a.num_blocks) return;
    const bool isk = j < a.hq + a.hk;
    const int h = isk ? j - a.hq : j - a.hq - a.hk;
    half_t* dst = (half_t*)(isk ? a.k_pool : a.v_pool) + blk * a.sp_b + off * a.sp_t +
                  (int64_t)h * a.sp_h;
    if (isk) {
        const half_t k0 = rope_h(x0, c[i], -x1, s[i]);
        const half_t k1 = rope_h(x1, c[i + hd], x0, s[i + hd]);
        dst[i] = k0;
        dst[i + hd] = k1;
        if (a.kmin) {
            // the page's K bounds: its first token resets them (fp16 min /
            // max are exact)
            half_t* mn = (half_t*)a.kmin + blk * a.sb_b + (int64_t)h * a.sb_h;
            half_t* mx = (half_t*)a.kmax + blk * a.sb_b + (int64_t)h * a.sb_h;
            if (off == 0) {
                mn[i] = k0;
                mn[i + hd] = k1;
                mx[i] = k0;
                mx[i + hd] = k1;
            } else {
                mn[i] = hf(fminf(f(mn[i]), f(k0)));
                mn[i + hd] = hf(fminf(f(mn[i + hd]), f(k1)));
                mx[i] = hf(fmaxf(f(mx[i]), f(k0)));
                mx[i + hd] = hf(fmaxf(f(mx[i + hd]), f(k1)));
            }
        }
    } else {
        dst[i] = x0;
        dst[i + hd] = x1;
    }
}

constexpr int ARGMAX_THREADS = 1024;
constexpr int ARGMAX_BATCH = 8;           // 16-byte loads a thread keeps in flight

// (v, i) replaces the best (bv, bi): larger value, NaN above any number,
// the smaller index among equals (torch.argmax's first occurrence).
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
    const bool vn = v != v, bn = bv != bv;
    if (vn || bn) return vn && (!bn || i < bi);
    return v > bv || (v == bv && i < bi);
}

// Write-through store (the row's last workgroup may run on another XCD).
__device__ __forceinline__ void store_through(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_through(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide best of (bv, bi), returned to thread 0.
__device__ __forceinline__ void argmax_block(float& bv, int& bi, float* sv, int* si) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (argmax_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (threadIdx.x % WAVE == 0) {
        sv[threadIdx.x / WAVE] = bv;
        si[threadIdx.x / WAVE] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < (int)blockDim.x / WAVE; ++w)
            if (argmax_better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
}

// grid (rows, parts): workgroup p scans chunks [p * cpp, (p + 1) * cpp) of
// its row, each thread its 16-byte chunks in increasing order (batches of
// loads issued together).  With parts > 1 the part bests go through the
// workspace and the row's last workgroup to arrive takes the best of them
// (ties to the smaller index, so arrival order does not matter).
__global__ __launch_bounds__(ARGMAX_THREADS) void argmax_rows_kernel(ArgmaxParams a) {
    __shared__ float sv[ARGMAX_THREADS / WAVE];
    __shared__ int si[ARGMAX_THREADS / WAVE];
    __shared__ bool last;
    const int row = blockIdx.x, part = blockIdx.y;
    const half_t* x = (const half_t*)a.x + (int64_t)row * a.sx;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    if (a.vec) {
        const int chunks = a.n / 8, cpp = (chunks + a.parts - 1) / a.parts;
        const int c_begin = part * cpp, c_end = c_begin + cpp < chunks ? c_begin + cpp : chunks;
        for (int c0 = c_begin; c0 < c_end; c0 += ARGMAX_THREADS * ARGMAX_BATCH) {
            u4 v[ARGMAX_BATCH];
#pragma unroll
            for (int k = 0; k < ARGMAX_BATCH; ++k) {
                const int c = c0 + k * ARGMAX_THREADS + threadIdx.x;
                v[k] = *(const u4*)(x + 8 * (c < c_end ? c : c_begin));
            }
#pragma unroll
            for (int k = 0; k < ARGMAX_BATCH; ++k) {
                const int c = c0 + k * ARGMAX_THREADS + threadIdx.x;
                if (c >= c_end) continue;
                half_t h[8];
                unpack8(v[k], h);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (argmax_better(f(h[e]), 8 * c + e, bv, bi)) {
                        bv = f(h[e]);
                        bi = 8 * c + e;
                    }
            }
        }
    } else {
        const int epp = (a.n + a.parts - 1) / a.parts;
        const int e_begin = part * epp, e_end = e_begin + epp < a.n ? e_begin + epp : a.n;
        for (int i = e_begin + threadIdx.x; i < e_end; i += ARGMAX_THREADS)
            if (argmax_better(f(x[i]), i, bv, bi)) {
                bv = f(x[i]);
                bi = i;
            }
    }
    argmax_block(bv, bi, sv, si);
    if (a.parts == 1) {
        if (threadIdx.x == 0) a.out[row] = bi;
        return;
    }
    if (threadIdx.x == 0) {
        store_through(a.part_v + (int64_t)row * a.parts + part, bv);
        store_through(a.part_i + (int64_t)row * a.parts + part, bi);
        handoff_release();
        last = __hip_atomic_fetch_add(a.counters + row, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (unsigned)a.parts - 1;
    }
    __syncthreads();
    if (!last || threadIdx.x != 0) return;
    for (int p = 0; p < a.parts; ++p) {                // device-coherent loads
        const float v = load_coherent(a.part_v + (int64_t)row * a.parts + p);
        const int i = load_coherent(a.part_i + (int64_t)row * a.parts + p);
        if (p == 0 || argmax_better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    a.out[row] = bi;
    __hip_atomic_store(a.counters + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// A part scans at least 16K values: a row of the 151936-word vocabulary
// takes 10 workgroups (11.7 us for 16 rows; 38 parts of 4K took 22 us).
constexpr int ARGMAX_PART_VALUES = 16384;
constexpr int ARGMAX_MAX_PARTS = 64;

int argmax_parts(int n) {
    const int p = (n + ARGMAX_PART_VALUES - 1) / ARGMAX_PART_VALUES;
    return p < 1 ? 1 : p > ARGMAX_MAX_PARTS ? ARGMAX_MAX_PARTS : p;
}

size_t argmax_workspace_bytes(int rows, int n) {
    const int p = argmax_parts(n);
    if (p == 1) return 0;
    return (size_t)rows * (sizeof(unsigned) + (size_t)p * (sizeof(float) + sizeof(int)));
}

hipError_t launch_argmax_rows(const ArgmaxParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(p.rows, p.parts), dim3(ARGMAX_THREADS), 0, stream,
                       p);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const NormParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    const bool res = p.res != nullptr;
    const bool vec = p.vec && p.n <= NORM_THREADS * 8 * NORM_MAXV;
    if (vec && res)
        hipLaunchKernelGGL(rms_norm_vec_kernel<true>, dim3(p.rows), dim3(NORM_THREADS), 0, stream, p);
    else if (vec)
        hipLaunchKernelGGL(rms_norm_vec_kernel<false>, dim3(p.rows), dim3(NORM_THREADS), 0, stream, p);
    else if (res)
        hipLaunchKernelGGL(rms_norm_any_kernel<true>, dim3(p.rows), dim3(NORM_THREADS), 0, stream, p);
    else
        hipLaunchKernelGGL(rms_norm_any_kernel<false>, dim3(p.rows), dim3(NORM_THREADS), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_silu_and_mul(const SiluParams& p, hipStream_t stream) {
    if (p.rows == 0 || p.inter == 0) return hipSuccess;
    if (p.vec) {
        const int per = 256 * 8;
        hipLaunchKernelGGL(silu_mul_vec_kernel, dim3((p.inter + per - 1) / per, p.rows), dim3(256),
                           0, stream, p);
    } else {
        hipLaunchKernelGGL(silu_mul_any_kernel, dim3((p.inter + 255) / 256, p.rows), dim3(256), 0,
                           stream, p);
    }
    return hipGetLastError();
}

hipError_t launch_rope_qk(const RopeParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_qk_kernel, dim3(p.rows, p.hq + p.hk), dim3(p.d / 2), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_rope_write_decode(const RopeWriteParams& p, hipStream_t stream) {
    if (p.B == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_write_decode_kernel, dim3(p.hq + 2 * p.hk, p.B), dim3(p.d / 2), 0,
                       stream, p);
    return hipGetLastError();
}

}  // namespace ls
