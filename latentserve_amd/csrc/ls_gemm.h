// Weight-streaming GEMM of the decode step: Y[M, N] = X[M, K] . W[N, K]^T
// (+ bias[N]) for the small M of decode batches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ls_elementwise.h"

namespace ls {

struct GemmParams {
    const void* x;       // fp16 [M, K], row stride ldx
    int64_t ldx;
    const void* w;       // fp16 [N, K], row stride ldw (a torch Linear weight), or
    int64_t ldw;         // packed (w_packed): see gemm_packed_bytes
    int w_packed;
    const void* bias;    // fp16 [N] or NULL
    void* y;             // fp16 [M, N], row stride ldy
    int64_t ldy;
    int M, N, K;
    int vec_y;           // y 8-byte aligned and ldy % 4 == 0: 8-byte stores
    float* part;         // fp32 partial sums [splits][M][ldp] when splits > 1
    unsigned* counters;  // arrivals a tile group, zero on entry and on exit
    int splits;          // workgroups a 16-row tile's K is split over
    int epi;             // GEMM_PLAIN, GEMM_GLU: y[M, N/2] = silu(gate) * up of w =
                         // [gate; up], GEMM_ROPE: the fused q/k/v projection's outputs
                         // rotated and stored as `rope` describes (y unused)
    RopeWriteParams rope;
    // norm != 0: the X operand is rms_norm(x + nres) (the decode layer's
    // residual add and RMSNorm, weight nw, eps), computed in the prologue;
    // workgroup 0 stores x + nres to nres_out.  One column block, K not
    // split over workgroups.
    int norm = 0;
    const void* nres = nullptr;
    int64_t ldr = 0;
    const void* nw = nullptr;
    void* nres_out = nullptr;
    int64_t ldro = 0;
    float eps = 0.f;
};

enum GemmEpilogue { GEMM_PLAIN = 0, GEMM_GLU = 1, GEMM_ROPE = 2 };

// Largest M one launch takes (four 16-row column blocks of the MFMA tile).
constexpr int GEMM_MAX_M = 64;

// Packed weights: the 16-row tiles of an epilogue's row mapping, each
// 32-channel step of a tile 1 KiB in the order the lanes load it (lane
// (r, g) holds row r's channels 8g .. 8g + 7 of the step), tiles padded to a
// multiple of 4 with zero rows.  Every weight load of a packed launch reads
// 1 KiB contiguous.  Bytes of the packed form of an [N, K] weight:
size_t gemm_packed_bytes(int N, int K, int epi, int head_dim);
hipError_t launch_pack_gemm_weight(const void* w, int64_t ldw, int N, int K, int epi, int head_dim,
                                   void* packed, hipStream_t stream);

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
