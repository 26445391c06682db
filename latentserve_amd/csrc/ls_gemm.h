// Weight-streaming GEMM of the decode step: Y[M, N] = X[M, K] . W[N, K]^T
// (+ bias[N]) for the small M of decode batches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

struct GemmParams {
    const void* x;       // fp16 [M, K], row stride ldx
    int64_t ldx;
    const void* w;       // fp16 [N, K], row stride ldw (a torch Linear weight)
    int64_t ldw;
    const void* bias;    // fp16 [N] or NULL
    void* y;             // fp16 [M, N], row stride ldy
    int64_t ldy;
    int M, N, K;
    int vec_y;           // y 8-byte aligned and ldy % 4 == 0: 8-byte stores
    float* part;         // fp32 partial sums [splits][M][ldp] when splits > 1
    unsigned* counters;  // arrivals a tile group, zero on entry and on exit
    int splits;          // workgroups a 16-row tile's K is split over
    int glu;             // 1: y[M, N/2] = silu(gate) * up of w = [gate; up]
};

// Largest M one launch takes (four 16-row column blocks of the MFMA tile).
constexpr int GEMM_MAX_M = 64;

// Splits of K over workgroups for an [M, N, K] product (1: no workspace).
int decode_gemm_splits(int M, int N, int K);
// Workspace of a split product: GEMM_COUNTERS arrival counters (one a
// tile group; the same bytes for every shape, so counters that one call
// leaves at zero are never another call's partial sums), then the fp32
// partials.
constexpr int GEMM_COUNTERS = 16384;
constexpr size_t GEMM_PART_OFFSET = GEMM_COUNTERS * sizeof(unsigned);
// Bytes of workspace the product needs (0 when it is not split).
size_t decode_gemm_workspace_bytes(int M, int N, int K);
// Tile groups (arrival counters) of the product.
int decode_gemm_units(int M, int N, int K);

// p.splits and p.part are set by the caller from the two functions above.
hipError_t launch_decode_gemm(const GemmParams& p, hipStream_t stream);

}  // namespace ls
