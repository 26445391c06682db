// Page selection for sparse (page-subset) decode: Quest-style page scores,
// top-k selection and the per-page K bounds they read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

struct KernelResources;   // ls_common.h

// Largest page count the selection keeps in registers (32 keys per thread of
// a 256-thread group).
constexpr int SELECT_MAX_PAGES = 8192;
// How long a selecting decode that scores its own pages waits for the other
// workgroups' scores before scoring the missing ones itself, by default
// (100 MHz ticks: 50 us).
constexpr uint64_t COOP_WAIT_TICKS = 5000;
// Pages scored per index workgroup (4 waves x 2 rounds x 4 pages).
constexpr int INDEX_PAGES_PER_GROUP = 32;

struct IndexParams {
    const void* q;          // fp16 [B, H, n_rep, 128]
    int64_t sq_b, sq_h, sq_r;
    const void* kmin;       // fp16 [num_blocks, H, 128]
    const void* kmax;
    int64_t sb_b, sb_h;
    int num_blocks;
    const int32_t* block_tables;
    int64_t sbt_b;
    int max_pages;
    const int32_t* seq_lens;
    float* scores;          // fp32 [B, H, >= max_pages]
    int64_t ss_b, ss_h;
    int B, H, NR, recent;
    // summed-mass scoring only: per-head logits fp32 [B, H, NR, >= max_pages]
    float* heads;
    int64_t sh_b, sh_h, sh_r;
    float scale_log2;       // softmax scale * log2(e)
};

struct SelectParams {
    const float* scores;
    int64_t ss_b, ss_h;
    const int32_t* seq_lens;
    int B, H, P, k, recent, sorted;
    float ratio;
    int32_t* sel;
    int64_t sl_b, sl_h;
};

struct BoundsParams {
    const void* src;        // update: k_new fp16 [B, H, 128]; rebuild: pool [nb, 16, H, 128]
    int64_t s0, s1, s2;     // update: (b, h, -); rebuild: (block, token, head)
    const int64_t* slots;   // update only: flat slot per sequence
    void* kmin;
    void* kmax;
    int64_t sb_b, sb_h;
    int num_blocks, B, H;
};

hipError_t launch_page_index(const IndexParams& p, hipStream_t stream);
hipError_t launch_page_select(const SelectParams& p, hipStream_t stream);
// Summed-mass scores: the per-head index launch, then the row softmaxes.
hipError_t launch_page_mass(const IndexParams& p, hipStream_t stream);
hipError_t launch_bounds_update(const BoundsParams& p, hipStream_t stream);
hipError_t launch_bounds_rebuild(const BoundsParams& p, hipStream_t stream);
// what: 0 page_index, 1 page_index_heads (mass), 2 page_mass, 3 page_select,
// 4 bounds_update, 5 bounds_rebuild; index kernels at n_rep rows.
hipError_t sparse_index_resources(int what, int n_rep, KernelResources* r);

}  // namespace ls
