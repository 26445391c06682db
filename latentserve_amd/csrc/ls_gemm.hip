// Weight-streaming GEMM of the decode step on gfx950:
//   Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]),  fp16 in and out, fp32 sums.
//
// At decode batch sizes (M <= 64) every projection of a layer is a pass over
// its weight matrix: HBM-bound on W (M * K activations stay in L2).  The
// library GEMMs pick 16 x 16 output tiles with no split of K for these
// shapes, which leaves the small-N projections (N = 1536 or 2048 on a
// 256-CU chip) to 96-128 workgroups.  Here the work unit is a 16-row tile of
// W (16 output features) and K is split over the waves of a workgroup (the
// partial tiles summed through LDS) and, where the tiles are too few to fill
// the chip, over workgroups too: those write fp32 partial sums and a second
// launch adds them (no atomics: device-scope atomics return slowly while the
// chip streams).
//
// MFMA v_mfma_f32_16x16x16f16 with A = 16 rows of W and B = X^T: a lane
// loads 16 bytes of its W row and 16 bytes of its X row per 32-channel step
// (64 contiguous bytes of each of 16 rows per load instruction), and the two
// MFMAs of the step take elements 0-3 and 4-7 of those loads, the channel
// order of both operands being the same.  Output lane (r, g) holds
// Y[r][n0 + 4g .. 4g + 3]: one 8-byte store where y's alignment allows.
//
// The reference runs these projections as torch (cuBLAS) GEMMs inside its
// model layers (model/fused.py, model/latentserve_qwen.py).
#include "ls_common.h"
#include "ls_gemm.h"

#pragma clang fp contract(off)

namespace ls {

namespace {

// One workgroup a (16-row tile, split); its blockDim.x / 64 waves take
// consecutive K chunks of at most SPW steps of 32 channels.  A wave's chunk
// is straight-line code (plain loads: the non-temporal hint measured slower
// here, 4.9 against 5.9 TB/s on the vocabulary projection): all its loads
// issued at once (repeats of the last
// step where the chunk is shorter than SPW, which re-read cached lines and
// add zeros), then consumed in order, so the compiler's load counting needs
// no joins and the whole chunk is in flight.  MB column blocks of 16 rows
// of X.  The waves' tiles are summed through LDS (blockDim.x / 64 * MB * 1
// KiB of dynamic shared memory).
template <int SPW, int TPW, int MB>
__global__ __launch_bounds__(256) void decode_gemm_kernel(GemmParams a) {
    extern __shared__ f4 red[];                       // [waves][TPW][MB][WAVE]
    const int nw = blockDim.x / WAVE;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = 16 * TPW * blockIdx.x;
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
        // rows past N read a valid row (clamped); their outputs are not stored
        const int n = n0 + 16 * t + r, nr = n < a.N ? n : a.N - 1;
        const half_t* wp = (const half_t*)a.w + (int64_t)nr * a.ldw + 32 * s0 + 8 * g;
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
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int nc = n0 + 16 * t + 4 * g;   // this lane's 4 output columns
        if (nc >= a.N) continue;
        if (a.splits > 1) {
            const int ldp = (a.N + 3) & ~3;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = 16 * mb + r;
                if (m < a.M)
                    *(f4*)(a.part + ((int64_t)blockIdx.y * a.M + m) * ldp + nc) = acc[t][mb];
            }
            continue;
        }
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
            half_t* yp = (half_t*)a.y + (int64_t)m * a.ldy + nc;
            if (a.vec_y && nc + 3 < a.N) {
                h4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = (half_t)(acc[t][mb][e] + bv[e]);
                *(h4*)yp = o;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (nc + e < a.N) yp[e] = (half_t)(acc[t][mb][e] + bv[e]);
            }
        }
    }
}

// y[m][n] = fp16(sum over splits of part[s][m][n] + bias[n]), four columns
// a thread.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams a) {
    const int ldp = (a.N + 3) & ~3, q = ldp / 4;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.M * q) return;
    const int m = i / q, nc = 4 * (i % q);
    const int64_t split_stride = (int64_t)a.M * ldp;
    const float* pp = a.part + (int64_t)m * ldp + nc;
    f4 t = *(const f4*)pp;
    for (int s = 1; s < a.splits; ++s) t += *(const f4*)(pp + s * split_stride);
    half_t* yp = (half_t*)a.y + (int64_t)m * a.ldy + nc;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (a.bias && nc + e < a.N) t[e] += (float)((const half_t*)a.bias)[nc + e];
    if (a.vec_y && nc + 3 < a.N) {
        h4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (half_t)t[e];
        *(h4*)yp = o;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (nc + e < a.N) yp[e] = (half_t)t[e];
    }
}

}  // namespace

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
    int mb, tpw, splits, group_waves;
};

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
    const int units = (tiles + s.tpw - 1) / s.tpw;           // groups of TPW tiles
    int w = chunks;
    // enough waves on the chip, without splitting K over workgroups for it
    int spread = (TARGET_WAVES + units - 1) / units;
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

int decode_gemm_splits(int M, int N, int K) { return gemm_shape(M, N, K).splits; }

size_t decode_gemm_workspace_bytes(int M, int N, int K) {
    const int s = decode_gemm_splits(M, N, K);
    return s > 1 ? (size_t)s * M * ((N + 3) & ~3) * sizeof(float) : 0;
}

template <int TPW, int MB>
void launch_kernel(const GemmParams& p, const GemmShape& sh, hipStream_t stream) {
    const dim3 grid((p.N + 16 * TPW - 1) / (16 * TPW), p.splits), block(WAVE * sh.group_waves);
    const size_t lds = sh.group_waves > 1 ? (size_t)sh.group_waves * TPW * MB * WAVE * sizeof(f4) : 0;
    hipLaunchKernelGGL((decode_gemm_kernel<spw_for(MB), TPW, MB>), grid, block, lds, stream, p);
}

hipError_t launch_decode_gemm(const GemmParams& p, hipStream_t stream) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    const GemmShape sh = gemm_shape(p.M, p.N, p.K);
    if (sh.splits != p.splits || sh.group_waves > MAX_GROUP_WAVES) return hipErrorInvalidValue;
    if (sh.mb == 1 && sh.tpw == 4)
        launch_kernel<4, 1>(p, sh, stream);
    else if (sh.mb == 1 && sh.tpw == 2)
        launch_kernel<2, 1>(p, sh, stream);
    else if (sh.mb == 1)
        launch_kernel<1, 1>(p, sh, stream);
    else if (sh.mb == 2)
        launch_kernel<1, 2>(p, sh, stream);
    else
        launch_kernel<1, 4>(p, sh, stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.splits == 1) return e;
    const int q = p.M * (((p.N + 3) & ~3) / 4);
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3((q + 255) / 256), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace ls
