// INT8 KV cache write side: decode-step write and per-block K quantizer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

struct KernelResources;   // ls_common.h

struct QuantArgs {
    int asym;          // 0: symmetric absmax, 1: asymmetric min/max
    int recip;         // 1: x / qmax as x * fp32(1 / qmax) (torch on a GPU); 0: true division
    float eps, qmax, inv_qmax, levels, inv_levels, offset;
};

struct DecodeWriteParams {
    const void* k;                 // fp16 [B, H, 128]
    int64_t sk_b, sk_h;
    const void* v;                 // fp16 [B, H, 128]
    int64_t sv_b, sv_h;
    const int64_t* slots;          // [B] flat token slot of the written token
    const int64_t* res_idx;        // [B] flat row of the fp16 residual
    void* flat_v;                  // int8 [num_slots, H, 128] contiguous
    float* flat_v_scale;           // [num_slots, H]
    float* flat_v_zero;            // [num_slots, H] (asym)
    void* k_res;                   // fp16 [num_res, H, 128] contiguous
    int64_t num_slots, num_res;
    int B, H;
    QuantArgs q;
};

struct FinalizeParams {
    const void* data;              // fp16 [N, 16, H, 128]
    int64_t sd_n, sd_t, sd_h;
    const int64_t* ids;            // [N] destination block of each
    void* k_pool;                  // int8 [num_blocks, 16, H, 128]
    int64_t sp_b, sp_t, sp_h;
    float* k_scale;                // [num_blocks, H, 128]
    float* k_zero;                 // same (asym)
    int64_t ss_b, ss_h;
    int64_t num_blocks;
    int N, H;
    QuantArgs q;
};

hipError_t launch_decode_write(const DecodeWriteParams& p, hipStream_t stream);
hipError_t launch_finalize_k(const FinalizeParams& p, hipStream_t stream);
// what: 0 decode_write, 1 finalize_k
hipError_t int8_write_resources(int what, KernelResources* r);

}  // namespace ls
