// Fused elementwise kernels of the decode step (the work around attention).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

// y = w * fp16(s * rsqrt(mean(s^2) + eps)), s = x (+ res, rounded to fp16 and
// stored to res_out).  Strides are row strides in elements; rows are unit
// stride.
struct NormParams {
    const void* x;
    int64_t sx;
    const void* res;          // NULL: plain norm
    int64_t sr;
    const void* w;
    void* y;
    int64_t sy;
    void* res_out;            // written when res is given; without res, a copy of x
    int64_t sro;
    const int64_t* ids;       // non-NULL: row r of x is x row ids[r] (a table lookup)
    int64_t id_rows;          // rows of that table (ids clamped into it)
    int rows;
    int n;
    float eps;
    bool vec;                 // every row 16-byte aligned and n a multiple of 8
};

// out[r] = the first index of the largest value of x row r (NaN counts as
// largest), as int64.
struct ArgmaxParams {
    const void* x;
    int64_t sx;
    int64_t* out;
    float* part_v;            // [rows][parts] a part's best value and index
    int* part_i;
    unsigned* counters;       // [rows] arrivals, zero on entry and on exit
    int parts;                // workgroups a row is split over (1: no workspace)
    int rows;
    int n;
    bool vec;                 // rows 16-byte aligned and n a multiple of 8
};

// Workgroups a row of n values is split over, and the workspace that needs.
int argmax_parts(int n);
size_t argmax_workspace_bytes(int rows, int n);

// out = fp16(fp16(silu(g)) * u), g = gu[:, :inter], u = gu[:, inter:].
struct SiluParams {
    const void* gu;
    int64_t sgu;
    void* out;
    int64_t so;
    int rows;
    int inter;
    bool vec;
};

// RoPE on [rows, H * D] q and k (rotate-half pairing), fp16 tables.
struct RopeParams {
    const void* q;
    int64_t sq;
    const void* k;
    int64_t sk;
    const void* cos;
    int64_t sc;               // table row stride (0: one row for all)
    const void* sin;
    int64_t ss;
    void* qo;
    int64_t sqo;
    void* ko;
    int64_t sko;
    int rows;
    int hq;
    int hk;
    int d;
};

// One decode token per sequence: q/k/v rows of the fused projection output,
// RoPE at each sequence's position, q folded to [B, H_kv, n_rep, D], k and v
// stored into the paged pools at each sequence's flat slot.
struct RopeWriteParams {
    const void* qkv;
    int64_t sqkv;             // row stride of qkv [B, (hq + 2 hk) * d]
    const int64_t* pos;       // [B]
    const void* cos;          // [tab_rows, d] fp16, row stride st
    const void* sin;
    int64_t st;
    int tab_rows;
    const int64_t* slots;     // [B] flat slot (block * page + offset); < 0: not written
    void* k_pool;             // [num_blocks, page, hk, d]
    void* v_pool;
    int64_t sp_b, sp_t, sp_h; // pool strides (elements), shared by K and V
    int num_blocks;
    int page;
    void* q_out;              // [B, hk, n_rep, d]
    int64_t sq_b, sq_h, sq_r;
    void* kmin;               // [num_blocks, hk, d] page bounds of K, or NULL
    void* kmax;
    int64_t sb_b, sb_h;
    int B;
    int hq;
    int hk;
    int d;
};

hipError_t launch_rms_norm(const NormParams& p, hipStream_t stream);
hipError_t launch_silu_and_mul(const SiluParams& p, hipStream_t stream);
hipError_t launch_rope_qk(const RopeParams& p, hipStream_t stream);
hipError_t launch_rope_write_decode(const RopeWriteParams& p, hipStream_t stream);
hipError_t launch_argmax_rows(const ArgmaxParams& p, hipStream_t stream);

}  // namespace ls
