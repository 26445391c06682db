// Internal launch descriptors shared by the kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

struct KernelResources;   // ls_common.h

enum KvKind { KV_FP16 = 0, KV_INT8 = 1 };

// List entries one group of a selecting page-subset walk keeps in its item
// table (a split's share of the list must fit).
constexpr int SELECT_SPLIT_ENTRIES = 1024;
// The one-launch bounds path (each group scores a share of its sequence's
// pages, then selects from the whole rows): rows of at most COOP_MAX_PAGES
// pages (eight keys a thread) and at most COOP_MAX_NREP query rows a KV head
// (their parts and sign masks stay in registers); larger shapes take the
// index kernel and the two-launch path.
constexpr int COOP_MAX_PAGES = 2048;
constexpr int COOP_MAX_NREP = 8;

// Arrival counters are COUNTER_STRIDE int32 apart (one 128-byte line each):
// the split groups of different (sequence, head) pairs bump them from all
// XCDs at once, and counters sharing a line serialise those atomics (c5
// 51.0 -> 50.0 us, c3 52.7 -> 52.1 us when they were given a line each).
constexpr int COUNTER_STRIDE = 32;

// Everything one decode launch reads.  Strides are in elements.
struct DecodeParams {
    const _Float16* q;
    int64_t sq_b, sq_h, sq_r;
    const void* k_pool;
    const void* v_pool;
    int64_t sk_b, sk_p, sk_h;          // shared by K and V
    int kind;
    const float* k_scale;
    int64_t sks_b, sks_h;
    const float* v_scale;
    int64_t svs_b, svs_p, svs_h;
    const float* k_zero;               // same strides as k_scale
    const float* v_zero;               // same strides as v_scale
    const _Float16* k_res;
    int64_t sr_r, sr_p, sr_h;
    const int32_t* res_rows;
    const int32_t* block_tables;
    int64_t sbt_b;
    int max_pages;                     // block-table width: pages past it are not read
    int num_blocks;                    // pool size: out-of-range block ids are not read
    int res_cap;                       // residual rows: out-of-range res_rows are not read
    const int32_t* seq_lens;
    const int32_t* sel;                // page-subset walk when non-null
    int64_t ssel_b, ssel_h;
    int num_sel;
    float ratio;
    int recent;
    float* scores;                     // non-null: page-subset walk whose list the kernel
    int64_t ssc_b, ssc_h;              // selects itself from page scores [B, H, score_pages]
    int score_pages;                   // (num_sel = the list width k)
    // non-null with scores: the kernel computes the scores itself from the
    // page K bounds fp16 [num_blocks, H, 128] (scores then starts all ones
    // and is left so)
    const void* kmin;
    const void* kmax;
    int64_t sb_b, sb_h;
    uint64_t coop_wait_ticks;          // how long (100 MHz ticks) a reader waits for the
                                       // other groups' scores before scoring them itself
    float* work;                       // [B * S, H] records of NR*128 + 32 floats:
                                       // acc[NR][128], m[16] (natural log), l[16]
    int pages_per_split;               // > 0: dense walk partition given by the host
    int32_t* counters;                 // [B * H * COUNTER_STRIDE], zero at rest, reset by
                                       // the kernel
    _Float16* out;
    int64_t so_b, so_h, so_r;
    int B, H, NR, num_splits;
    float scale;
};

struct CombineParams {
    const float* acc;
    int64_t sa_b, sa_h, sa_s, sa_r;
    const float* m;
    const float* l;
    int64_t sm_b, sm_h, sm_s;          // shared by m and l, unit stride over rows
    void* out;
    int out_f32;
    int64_t so_b, so_h, so_r;
    int B, H, S, NR;
};

hipError_t launch_decode(const DecodeParams& a, hipStream_t stream);

// The no-allocation decode's fixed device scratch: split records
// (NOALLOC_WORK_BYTES) then arrival counters (NOALLOC_COUNTERS int32, so
// batch * kv_heads <= NOALLOC_COUNTERS / COUNTER_STRIDE).
constexpr size_t NOALLOC_WORK_BYTES = size_t(16) << 20;
constexpr int NOALLOC_COUNTERS = 1 << 16;
// This device's scratch (looked up, and its counters cleared on `stream`,
// at the first call on the device).
hipError_t noalloc_scratch(hipStream_t stream, float** work, int32_t** counters);
hipError_t launch_combine(const CombineParams& p, hipStream_t stream);
// The kernel a decode launch runs: walk 0 dense, 1 a given list, 2 selecting
// from given scores, 3 scoring and selecting itself; `pair_heads` an even
// head count; INT8 with `asym` / `has_res`.  combine: ls_combine_splits's.
hipError_t decode_resources(int kind, int walk, bool asym, bool has_res, bool pair_heads,
                            KernelResources* r);
hipError_t combine_resources(KernelResources* r);
#ifdef LS_DIAGNOSTICS
// Page-compute probe (measurement only): groups x 8 waves, each applying one
// register-resident page `items` times; mode 0 MFMA (compute_page), 1 VALU.
// out: [groups * 8][6][128] fp32, O of each wave.
hipError_t launch_compute_probe(int mode, int groups, int items, float scale, float* out,
                                hipStream_t stream);
#endif

}  // namespace ls
