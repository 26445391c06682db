// Weight-streaming GEMM of the decode step on gfx950:
//   Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]),  fp16 in and out, fp32 sums,
// and its gate/up form Y[M, I] = silu(X . Wg^T) * (X . Wu^T) for a weight
// [Wg; Wu] of 2I rows, the MLP activation applied in the epilogue.
//
// At decode batch sizes (M <= 64) every projection of a layer is a pass over
// its weight matrix: HBM-bound on W (M * K activations stay in L2).  The
// library GEMMs pick 16 x 16 output tiles with no split of K for these
// shapes, which leaves the small-N projections (N = 1536 or 2048 on a
// 256-CU chip) to 96-128 workgroups.  Here the work unit is a 16-row tile of
// W (16 output features) and K is split over the waves of a workgroup (the
// partial tiles summed through LDS) and, where the tiles are too few to fill
// the chip, over workgroups too: those write fp32 partial sums to the
// workspace and the last workgroup of a tile to finish adds them, in split
// order, so the result does not depend on which one that is.
//
// Each wave takes a K chunk of at most SPW steps of 32 channels as
// straight-line code: its loads are all issued before the first is used, so
// the whole chunk is in flight and the compiler's load counting needs no
// joins (loads under a branch, or issued in a loop after the sums that
// precede them, made it wait for every load in flight at each step).
// Chunks shorter than SPW repeat their last step, whose lines are cached,
// and add zeros for it.  Plain loads: the non-temporal hint measured slower
// here (4.9 against 5.9 TB/s on the vocabulary projection).
//
// MFMA v_mfma_f32_16x16x16f16 with A = 16 rows of W and B = X^T: a lane
// loads 16 bytes of its W row and 16 bytes of its X row per step (64
// contiguous bytes of each of 16 rows per load instruction), and the two
// MFMAs of the step take elements 0-3 and 4-7 of those loads, the channel
// order of both operands being the same.  Output lane (r, g) holds
// Y[r][n0 + 4g .. 4g + 3]: one 8-byte store where y's alignment allows.
//
// The gate/up form gives a tile 8 gate rows (lanes g = 0, 1 of the output)
// and the 8 matching up rows (g = 2, 3); the up values cross to the gate
// lanes with one swizzle, and each output is rounded exactly as the two
// launches it replaces round it (fp16 gate and up, then the fp16 SiLU
// product), so the fused and separate paths are bit-equal.
//
// The reference runs these projections as torch (cuBLAS) GEMMs inside its
// model layers (model/fused.py, model/latentserve_qwen.py) and the
// activation as silu_and_mul (kernels/fused_elementwise.py:222-233).
#include "ls_common.h"
#include "ls_gemm.h"

#pragma clang fp contract(off)

namespace ls {

namespace {

// Device-coherent (write-through, sc1) 16-byte store: the workgroup that
// sums a tile's partials may run on another XCD, whose L2 does not see this
// one's.
__device__ __forceinline__ void store_through4(float* p, f4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// Stores one lane's four outputs y[m][nc .. nc + 3] (fewer at the right
// edge of a width-n output).
__device__ __forceinline__ void store_out(const GemmParams& a, int m, int nc, int n,
                                          const half_t* v) {
    half_t* yp = (half_t*)a.y + (int64_t)m * a.ldy + nc;
    if (a.vec_y && nc + 3 < n) {
        h4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = v[e];
        *(h4*)yp = o;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (nc + e < n) yp[e] = v[e];
    }
}

// W row of output-tile row r: plain tiles hold 16 consecutive rows; gate/up
// tiles hold gate rows 8T .. 8T + 7 and the up rows I + 8T .. (rows past the
// edge clamped to a valid one: their outputs are not stored).
template <bool GLU>
__device__ __forceinline__ int w_row(const GemmParams& a, int tile, int r) {
    if (GLU) {
        const int half_n = a.N / 2, j0 = 8 * tile + (r & 7), j = j0 < half_n ? j0 : half_n - 1;
        return r < 8 ? j : half_n + j;
    }
    const int n = 16 * tile + r;
    return n < a.N ? n : a.N - 1;
}

// One workgroup a (TPW tiles, split); its blockDim.x / 64 waves take
// consecutive K chunks of the split's range.  MB column blocks of 16 rows
// of X.  The waves' tiles are summed through LDS (blockDim.x / 64 * TPW *
// MB KiB of dynamic shared memory).
template <int SPW, int TPW, int MB, bool GLU>
__global__ __launch_bounds__(256) void decode_gemm_kernel(GemmParams a) {
    extern __shared__ f4 red[];                       // [waves][TPW][MB][WAVE]
    const int nw = blockDim.x / WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int r = lane & 15, g = lane >> 4;
    const int tile0 = TPW * blockIdx.x;
    const int steps = a.K >> 5;
    const int c = blockIdx.y * nw + wv, nc_ = a.splits * nw;   // chunk c of nc_
    const int s0 = (int)((int64_t)steps * c / nc_);
    const int ns = (int)((int64_t)steps * (c + 1) / nc_) - s0;  // 1..SPW (host)
    const int last = ns - 1;
    const half_t* xp[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = 16 * mb + r < a.M ? 16 * mb + r : a.M - 1;
        xp[mb] = (const half_t*)a.x + (int64_t)m * a.ldx + 32 * s0 + 8 * g;
    }
    // The wave's X chunk is loaded once and serves its TPW weight tiles,
    // which stream through two register sets: tile t + 2 is issued once
    // tile t is consumed, so one tile is always in flight behind the one
    // being summed.
    u4 xb[SPW][MB];
    u4 wb[2][SPW];
    auto load_w = [&](int b, int t) {
        const half_t* wp = (const half_t*)a.w + (int64_t)w_row<GLU>(a, tile0 + t, r) * a.ldw +
                           32 * s0 + 8 * g;
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int st = i < last ? i : last;
            wb[b][i] = *(const u4*)(wp + 32 * st);
        }
    };
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
        const int st = i < last ? i : last;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) xb[i][mb] = *(const u4*)(xp[mb] + 32 * st);
    }
    load_w(0, 0);
    if (TPW > 1) load_w(1, 1);
    f4 acc[TPW][MB];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        // (scheduling barriers keep the loads ahead of the sums that need
        // them, where the instruction scheduler would sink them)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[t][mb] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const bool live = i == 0 || i < ns;       // a chunk has a step at least
            const u4 z = {0u, 0u, 0u, 0u};
            const u4 w = wb[t & 1][i];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const u4 xv = live ? xb[i][mb] : z;
                acc[t][mb] = mfma16(as_h4(w.x, w.y), as_h4(xv.x, xv.y), acc[t][mb]);
                acc[t][mb] = mfma16(as_h4(w.z, w.w), as_h4(xv.z, xv.w), acc[t][mb]);
            }
        }
        if (t + 2 < TPW) {
            __builtin_amdgcn_sched_barrier(0);
            load_w(t & 1, t + 2);
        }
    }

    if (nw > 1) {
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                red[((wv * TPW + t) * MB + mb) * WAVE + lane] = acc[t][mb];
        __syncthreads();
        if (wv != 0) return;
        for (int p = 1; p < nw; ++p)
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[t][mb] += red[((p * TPW + t) * MB + mb) * WAVE + lane];
    }
    // wave 0 alone from here

    if (GLU) {
        // splits == 1 (host): lanes g = 0, 1 hold gate columns 8T + 4g + e,
        // lanes g + 2 the matching up columns
        const int half_n = a.N / 2;
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                f4 up;
#pragma unroll
                for (int e = 0; e < 4; ++e) up[e] = __shfl_xor(acc[t][mb][e], 32);
                const int m = 16 * mb + r, j = 8 * (tile0 + t) + 4 * g;
                if (g >= 2 || m >= a.M || j >= half_n) continue;
                half_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float gv = acc[t][mb][e], uv = up[e];
                    if (a.bias && j + e < half_n) {
                        gv += (float)((const half_t*)a.bias)[j + e];
                        uv += (float)((const half_t*)a.bias)[half_n + j + e];
                    }
                    o[e] = silu_mul_h((half_t)gv, (half_t)uv);
                }
                store_out(a, m, j, half_n, o);
            }
        return;
    }

    if (a.splits == 1) {
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const int nc = 16 * (tile0 + t) + 4 * g;   // this lane's 4 output columns
            if (nc >= a.N) continue;
            f4 bv = {0.f, 0.f, 0.f, 0.f};
            if (a.bias) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    bv[e] = nc + e < a.N ? (float)((const half_t*)a.bias)[nc + e] : 0.f;
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = 16 * mb + r;
                if (m >= a.M) continue;
                half_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = (half_t)(acc[t][mb][e] + bv[e]);
                store_out(a, m, nc, a.N, o);
            }
        }
        return;
    }

    // ---- split K: partials through the workspace, the last group sums ----
    const int ldp = (a.N + 3) & ~3;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int nc = 16 * (tile0 + t) + 4 * g;
        if (nc >= a.N) continue;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int m = 16 * mb + r;
            if (m < a.M)
                store_through4(a.part + ((int64_t)blockIdx.y * a.M + m) * ldp + nc, acc[t][mb]);
        }
    }
    // The partials bypass the non-coherent L2 path, so ordering needs only
    // their completion before the arrival count (no whole-L2 writeback or
    // invalidate, which a device-scope fence would issue).
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    int prev = 0;
    if (lane == 0)
        prev = __hip_atomic_fetch_add(a.counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0);
    if (prev != a.splits - 1) return;
    // Every split of these tiles has arrived.  Their partials were written
    // through to memory and no group has read those lines in this launch,
    // so plain loads see them.  Unit u = (t, m, q): four columns.
    const int64_t split_stride = (int64_t)a.M * ldp;
    for (int u = lane; u < TPW * a.M * 4; u += WAVE) {
        const int t = u / (a.M * 4), m = (u / 4) % a.M, q = u % 4;
        const int nc = 16 * (tile0 + t) + 4 * q;
        if (nc >= a.N) continue;
        const float* pp = a.part + (int64_t)m * ldp + nc;
        f4 s = *(const f4*)pp;
        for (int sp = 1; sp < a.splits; ++sp) s += *(const f4*)(pp + sp * split_stride);
        half_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (a.bias && nc + e < a.N) s[e] += (float)((const half_t*)a.bias)[nc + e];
            o[e] = (half_t)s[e];
        }
        store_out(a, m, nc, a.N, o);
    }
    // back to zero for the next launch
    if (lane == 0)
        __hip_atomic_store(a.counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Steps of 32 channels a wave takes at most, per column-block count of X
// (the chunk's loads live in registers: 4 VGPRs a step and block of X, 8 a
// step of W).
constexpr int spw_for(int mb) { return mb == 1 ? 16 : mb == 2 ? 8 : 4; }
// Waves a launch aims for (8 a CU), and the most waves a workgroup.
constexpr int TARGET_WAVES = 2048;
constexpr int MAX_GROUP_WAVES = 4;
// With one block of X, a wave takes 2 or 4 weight tiles when the launch
// keeps at least this many waves (fewer X loads a weight byte).
constexpr int TPW_MIN_WAVES = 2048;

struct GemmShape {
    int mb, tpw, splits, group_waves, units;
};

// The launch shape of an [M, N, K] product (N: weight rows, 2I for the
// gate/up form, whose tiles cover as many rows).
GemmShape gemm_shape(int M, int N, int K) {
    GemmShape s;
    s.mb = (M + 15) / 16 <= 1 ? 1 : (M + 15) / 16 <= 2 ? 2 : 4;
    const int tiles = (N + 15) / 16, steps = K / 32, spw = spw_for(s.mb);
    const int chunks = (steps + spw - 1) / spw;              // chunks of <= SPW steps
    s.tpw = 1;
    if (s.mb == 1) {
        if ((int64_t)(tiles + 3) / 4 * chunks >= TPW_MIN_WAVES)
            s.tpw = 4;
        else if ((int64_t)(tiles + 1) / 2 * chunks >= TPW_MIN_WAVES)
            s.tpw = 2;
    }
    s.units = (tiles + s.tpw - 1) / s.tpw;                   // groups of TPW tiles
    int w = chunks;
    // enough waves on the chip, without splitting K over workgroups for it
    int spread = (TARGET_WAVES + s.units - 1) / s.units;
    if (spread > MAX_GROUP_WAVES) spread = MAX_GROUP_WAVES;
    if (spread > steps) spread = steps;
    if (w < spread) w = spread;
    s.splits = (w + MAX_GROUP_WAVES - 1) / MAX_GROUP_WAVES;
    s.group_waves = (w + s.splits - 1) / s.splits;
    // every chunk of steps / (splits * group_waves) must fit SPW
    while ((steps + s.splits * s.group_waves - 1) / (s.splits * s.group_waves) > spw)
        ++s.group_waves;
    return s;
}

template <int TPW, int MB, bool GLU>
void launch_kernel(const GemmParams& p, const GemmShape& sh, hipStream_t stream) {
    const dim3 grid(sh.units, p.splits), block(WAVE * sh.group_waves);
    const size_t lds =
        sh.group_waves > 1 ? (size_t)sh.group_waves * TPW * MB * WAVE * sizeof(f4) : 0;
    hipLaunchKernelGGL((decode_gemm_kernel<spw_for(MB), TPW, MB, GLU>), grid, block, lds, stream,
                       p);
}

template <bool GLU>
void launch_any(const GemmParams& p, const GemmShape& sh, hipStream_t stream) {
    if (sh.mb == 1 && sh.tpw == 4)
        launch_kernel<4, 1, GLU>(p, sh, stream);
    else if (sh.mb == 1 && sh.tpw == 2)
        launch_kernel<2, 1, GLU>(p, sh, stream);
    else if (sh.mb == 1)
        launch_kernel<1, 1, GLU>(p, sh, stream);
    else if (sh.mb == 2)
        launch_kernel<1, 2, GLU>(p, sh, stream);
    else
        launch_kernel<1, 4, GLU>(p, sh, stream);
}

}  // namespace

int decode_gemm_splits(int M, int N, int K) { return gemm_shape(M, N, K).splits; }

int decode_gemm_units(int M, int N, int K) { return gemm_shape(M, N, K).units; }

size_t decode_gemm_workspace_bytes(int M, int N, int K) {
    const GemmShape sh = gemm_shape(M, N, K);
    if (sh.splits == 1) return 0;
    return GEMM_PART_OFFSET + (size_t)sh.splits * M * ((N + 3) & ~3) * sizeof(float);
}

hipError_t launch_decode_gemm(const GemmParams& p, hipStream_t stream) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    const GemmShape sh = gemm_shape(p.M, p.N, p.K);
    if (sh.splits != p.splits || sh.group_waves > MAX_GROUP_WAVES) return hipErrorInvalidValue;
    if (p.glu) {
        if (p.splits != 1 || p.N % 2 != 0) return hipErrorInvalidValue;
        launch_any<true>(p, sh, stream);
    } else {
        launch_any<false>(p, sh, stream);
    }
    return hipGetLastError();
}

}  // namespace ls
