// The Quest page bound, shared by the page index kernel and the selecting
// decode's own scoring, so both produce the same bits: for a query row q and
// a page's per-channel K bounds [lo, hi], sum_d max(q_d lo_d, q_d hi_d)
// (kernels/cuda/paged_sparse_fp16.cu:78-130), formed by 16 lanes of 8
// channels each (quest_part) and four DPP adds over the 16 lanes.
#pragma once

#include "ls_common.h"

namespace ls {

typedef short short2_t __attribute__((ext_vector_type(2)));

template <int CTRL>
__device__ __forceinline__ float quest_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                         0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each row of 16 lanes, result in every lane of the row: quad
// swaps (xor 1, xor 2), then half-row and row mirrors.
__device__ __forceinline__ float quest_row16_sum(float v) {
    v += quest_dpp<0xB1>(v);
    v += quest_dpp<0x4E>(v);
    v += quest_dpp<0x141>(v);
    v += quest_dpp<0x140>(v);
    return v;
}

// (Components are named, not indexed: subscripting a vector-typed reference
// inside an unrolled loop lost all but the first component in this build.)
__device__ __forceinline__ void quest_h8_to_f8(u4 x, float* f) {
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 t = __builtin_bit_cast(h2, w[i]);
        f[2 * i] = (float)t.x;
        f[2 * i + 1] = (float)t.y;
    }
}

// The sign masks of a query part's eight fp16 channels: 0xFFFF in each half
// whose q is negative (a packed arithmetic shift).  Computed once a query
// row and passed to quest_part opaque, so the select there stays one
// bitfield insert a channel pair (seen through, the compiler rebuilt it as
// compares and selects, three instructions a pair).
__device__ __forceinline__ u4 quest_masks(u4 q) {
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    uint32_t m[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2_t, qw[i]) >> (short)15);
        asm volatile("" : "+v"(m[i]));
    }
    return u4{m[0], m[1], m[2], m[3]};
}

// The lane's 8-channel part of one query row's bound, from the raw fp16
// words of the query, its sign masks and the page's bounds: max(q lo, q hi)
// = q * (q < 0 ? lo : hi), so each channel pair is one bitfield insert (v_bfi_b32) and
// one v_dot2_f32_f16 (fp16 products are exact in fp32) accumulated in fp32
// in channel-pair order.
__device__ __forceinline__ float quest_part(u4 q, u4 m, u4 lo, u4 hi) {
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    const uint32_t mw[4] = {m.x, m.y, m.z, m.w};
    const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w};
    const uint32_t hw[4] = {hi.x, hi.y, hi.z, hi.w};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t sel;   // lw where the mask is set, else hw
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(sel) : "v"(mw[i]), "v"(lw[i]), "v"(hw[i]));
        s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qw[i]), __builtin_bit_cast(h2, sel),
                                   s, false);
    }
    return s;
}
// (the same, the masks formed on the spot: for one-off scores)
__device__ __forceinline__ float quest_part(u4 q, u4 lo, u4 hi) {
    return quest_part(q, quest_masks(q), lo, hi);
}

}  // namespace ls
