// Block-table gather of a paged K or V pool into [B, L, H, D].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

struct GatherParams {
    const void* pool;              // [num_blocks, 16, H, D], `elem`-byte elements
    int64_t sp_b, sp_t, sp_h;      // element strides
    int num_blocks;
    const int32_t* block_tables;
    int64_t sbt_b;
    int max_pages;
    const int32_t* seq_lens;
    void* out;                     // [B, L, H, D]
    int64_t so_b, so_t, so_h;      // element strides
    int elem, row_bytes;           // bytes per element, per (token, head) row (multiple of 16)
    int B, L, H;
};

hipError_t launch_gather(const GatherParams& p, hipStream_t stream);

}  // namespace ls
