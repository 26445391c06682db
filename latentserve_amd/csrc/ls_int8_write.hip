// INT8 KV cache write side on gfx950: the decode-step write (V quantized per
// token into the pool, K copied into the fp16 last-page residual) and the
// per-block K quantizer that runs when a page completes.
//
// Reference: kernels/cuda/int8_write.cu:46-80 (int8_decode_write, launched by
// kernels/cuda/int8_write.py:61-82) and cache/int8_paged_cache.py:670-699
// (_finalize_blocks), :741-758 (write(), V part).
//
// Codes are bit-exact with the reference's torch ops: fp32 throughout, every
// multiply / add / divide rounded on its own (no contraction), rintf for
// torch.round (half to even), the same epsilon floor.  One choice is left to
// the caller: torch divides a tensor by a Python number on the GPU as a
// multiply by the fp32 reciprocal formed on the host, and on the CPU as a
// true division (they differ in the last bit of a few percent of scales).
// `recip` = 1 reproduces the GPU form (what the reference stores when it runs
// on a GPU, and what its int8_write.cu computes); 0 the CPU form.
//
// Layout: one wave per (row, head) of 128 channels, two channels a lane; the
// row's max / min is a wave reduction (no LDS).  HBM-bound byte work.
#include "ls_common.h"
#include "ls_int8_write.h"

#pragma clang fp contract(off)

namespace ls {

namespace {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, shfl_xor(v, o));
    return v;
}

struct QuantStep {
    float step, zero, lo;
};

// Scale (and zero point) of one row from its max |x| (sym) or min / max (asym).
__device__ __forceinline__ QuantStep fit(float amax, float lo, float hi, const QuantArgs& q) {
    QuantStep s;
    s.lo = lo;
    s.zero = 0.f;
    if (!q.asym) {
        const float m = fmaxf(amax, q.eps);                       // clamp_min(eps)
        s.step = q.recip ? m * q.inv_qmax : m / q.qmax;           // / qmax
    } else {
        const float r = hi - lo;
        const float t = q.recip ? r * q.inv_levels : r / q.levels;  // / levels
        s.step = fmaxf(t, q.eps);                                  // clamp_min(eps)
        s.zero = lo + q.offset * s.step;
    }
    return s;
}

__device__ __forceinline__ int8_t code(float x, const QuantStep& s, const QuantArgs& q) {
    if (!q.asym) {
        const float r = rintf(x / s.step);
        return (int8_t)(int)fminf(fmaxf(r, -q.qmax), q.qmax);
    }
    const float u = fminf(fmaxf(rintf((x - s.lo) / s.step), 0.f), q.levels);
    return (int8_t)(int)(u - q.offset);
}

// One wave per (b, h): grid (ceil(B * H / 4)), 256 threads.
__global__ __launch_bounds__(256) void decode_write_kernel(DecodeWriteParams a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (int64_t)a.B * a.H) return;
    const int b = (int)(row / a.H), h = (int)(row % a.H);
    const int d = 2 * lane;
    const h2 vv = *(const h2*)((const half_t*)a.v + (int64_t)b * a.sv_b + (int64_t)h * a.sv_h + d);
    const float x0 = (float)vv.x, x1 = (float)vv.y;
    const int64_t slot = a.slots[b];
    if (slot >= 0 && slot < a.num_slots) {
        float amax = 0.f, lo = 0.f, hi = 0.f;
        if (!a.q.asym) {
            amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
        } else {
            hi = wave_max(fmaxf(x0, x1));
            lo = wave_min(fminf(x0, x1));
        }
        const QuantStep s = fit(amax, lo, hi, a.q);
        const int64_t r = slot * a.H + h;            // flat [slots, H] row
        char2 c;
        c.x = code(x0, s, a.q);
        c.y = code(x1, s, a.q);
        *(char2*)((int8_t*)a.flat_v + r * HEAD_DIM + d) = c;
        if (lane == 0) {
            a.flat_v_scale[r] = s.step;
            if (a.q.asym) a.flat_v_zero[r] = s.zero;
        }
    }
    // K into the fp16 residual: its page is quantized when it completes.
    const int64_t ri = a.res_idx[b];
    if (ri >= 0 && ri < a.num_res)
        *(h2*)((half_t*)a.k_res + (ri * a.H + h) * HEAD_DIM + d) =
            *(const h2*)((const half_t*)a.k + (int64_t)b * a.sk_b + (int64_t)h * a.sk_h + d);
}

// One wave per (block n, head h): the 16 token rows, two channels a lane;
// step per (block, head, channel) over the 16 tokens.
__global__ __launch_bounds__(256) void finalize_k_kernel(FinalizeParams a) {
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= (int64_t)a.N * a.H) return;
    const int64_t n = item / a.H;
    const int h = (int)(item % a.H);
    const int64_t blk = a.ids[n];
    if (blk < 0 || blk >= a.num_blocks) return;
    const int d = 2 * lane;
    const half_t* src = (const half_t*)a.data + n * a.sd_n + (int64_t)h * a.sd_h + d;
    float x[PAGE][2];
#pragma unroll
    for (int t = 0; t < PAGE; ++t) {
        const h2 v = *(const h2*)(src + (int64_t)t * a.sd_t);
        x[t][0] = (float)v.x;
        x[t][1] = (float)v.y;
    }
    int8_t* dst = (int8_t*)a.k_pool + blk * a.sp_b + (int64_t)h * a.sp_h + d;
    const int64_t si = blk * a.ss_b + (int64_t)h * a.ss_h + d;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        float amax = 0.f, lo = x[0][e], hi = x[0][e];
#pragma unroll
        for (int t = 0; t < PAGE; ++t) {
            amax = fmaxf(amax, fabsf(x[t][e]));
            lo = fminf(lo, x[t][e]);
            hi = fmaxf(hi, x[t][e]);
        }
        const QuantStep s = fit(amax, lo, hi, a.q);
        a.k_scale[si + e] = s.step;
        if (a.q.asym) a.k_zero[si + e] = s.zero;
#pragma unroll
        for (int t = 0; t < PAGE; ++t) x[t][e] = (float)code(x[t][e], s, a.q);
    }
#pragma unroll
    for (int t = 0; t < PAGE; ++t) {
        char2 c;
        c.x = (int8_t)(int)x[t][0];
        c.y = (int8_t)(int)x[t][1];
        *(char2*)(dst + (int64_t)t * a.sp_t) = c;
    }
}

}  // namespace

hipError_t launch_decode_write(const DecodeWriteParams& p, hipStream_t stream) {
    const int64_t rows = (int64_t)p.B * p.H;
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(decode_write_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream,
                       p);
    return hipGetLastError();
}

hipError_t launch_finalize_k(const FinalizeParams& p, hipStream_t stream) {
    const int64_t items = (int64_t)p.N * p.H;
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(finalize_k_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream,
                       p);
    return hipGetLastError();
}

hipError_t int8_write_resources(int what, KernelResources* r) {
    if (what == 0) return func_resources(decode_write_kernel, 256, r);
    if (what == 1) return func_resources(finalize_k_kernel, 256, r);
    return hipErrorInvalidValue;
}

}  // namespace ls
