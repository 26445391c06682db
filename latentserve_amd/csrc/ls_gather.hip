// Block-table gather on gfx950: the paged cache's read path, copying every
// live token's K (or V) rows out of the pool into [B, L, H, D].
//
// Reference: cache/paged_cache.py:486-506 (read(): flat pool indexed by the
// padded slot table of :305-323) and cache/block_allocator.py:214-220 (the
// slot rule).  Token p < L of sequence b is flat slot
// table[b][p / 16] * 16 + p % 16; positions past a sequence's length read
// flat slot 0, as the reference's zero-padded slot table does (block ids
// outside the pool read slot 0 too, where the reference would fault).
//
// Pure byte movement, HBM-bound: one thread moves 16 bytes, a (token, head)
// row of 128 channels is 16 (fp16) or 8 (int8) adjacent threads, and the
// rows of a token's heads are adjacent, so both sides stream whole lines.
#include "ls_common.h"
#include "ls_gather.h"

namespace ls {

namespace {

// grid (ceil(L * H * pieces / 256), B): 32-bit indexing within a sequence.
__global__ __launch_bounds__(256) void gather_kernel(GatherParams a) {
    const int vpr = a.row_bytes / 16;                        // 16-byte pieces per head row
    const int per_tok = a.H * vpr;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.L * per_tok) return;
    const int b = blockIdx.y;
    const int p = i / per_tok;
    const int r = i - p * per_tok;
    const int h = r / vpr, piece = r - h * vpr;
    int64_t blk = 0;
    int row = 0;
    if (p < a.seq_lens[b] && p / PAGE < a.max_pages) {
        const int id = a.block_tables[(int64_t)b * a.sbt_b + p / PAGE];
        if (id >= 0 && id < a.num_blocks) {
            blk = id;
            row = p % PAGE;
        }
    }
    const char* src = (const char*)a.pool +
                      (blk * a.sp_b + (int64_t)row * a.sp_t + (int64_t)h * a.sp_h) * a.elem +
                      16 * piece;
    char* dst = (char*)a.out +
                ((int64_t)b * a.so_b + (int64_t)p * a.so_t + (int64_t)h * a.so_h) * a.elem +
                16 * piece;
    __builtin_nontemporal_store(stream_load((const u4*)src), (u4*)dst);
}

}  // namespace

hipError_t launch_gather(const GatherParams& p, hipStream_t stream) {
    const int64_t per_seq = (int64_t)p.L * p.H * (p.row_bytes / 16);
    if (per_seq == 0 || p.B == 0) return hipSuccess;
    hipLaunchKernelGGL(gather_kernel, dim3((unsigned)((per_seq + 255) / 256), p.B), dim3(256), 0,
                       stream, p);
    return hipGetLastError();
}

}  // namespace ls
