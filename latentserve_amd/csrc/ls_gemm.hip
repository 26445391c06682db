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
// The fused q/k/v form pairs each head's channel with its rotate-half
// partner the same way and finishes as ls_rope_write_decode: RoPE, the
// query folded to [B, H_kv, n_rep, D], the key and value stored at the
// sequence's slot (with the page K bounds), bit-equal to the two launches.
//
// The reference runs these projections as torch (cuBLAS) GEMMs inside its
// model layers (model/fused.py, model/latentserve_qwen.py), the activation
// as silu_and_mul (kernels/fused_elementwise.py:222-233) and the decode
// token's rope_qk and cache write in its attention layer
// (model/attention/gqa.py:251-253, cache/paged_cache.py write).
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
// edge clamped to a valid one: their outputs are not stored); RoPE tiles
// hold 8 channels of a head's first half and their rotate-half partners,
// head T / (d / 16), channels 8 (T % (d / 16)) + [0, 8) and + d / 2.
template <int EPI>
__device__ __forceinline__ int w_row_of(int N, int d, int tile, int r, bool& real) {
    if (EPI == GEMM_GLU) {
        const int half_n = N / 2, j0 = 8 * tile + (r & 7), j = j0 < half_n ? j0 : half_n - 1;
        real = j0 < half_n;
        return r < 8 ? j : half_n + j;
    }
    int n;
    if (EPI == GEMM_ROPE) {
        const int tph = d / 16, head = tile / tph, i = 8 * (tile % tph) + (r & 7);
        n = head * d + i + (r < 8 ? 0 : d / 2);
    } else {
        n = 16 * tile + r;
    }
    real = n < N;
    return n < N ? n : N - 1;
}
template <int EPI>
__device__ __forceinline__ int w_row(const GemmParams& a, int tile, int r) {
    bool real;
    return w_row_of<EPI>(a.N, a.rope.d, tile, r, real);
}

// Packed weights (gemm_packed_bytes): tile T's step s is 64 lanes x 16 B at
// ((T * steps + s) * 64 + lane) * 8 halves.
constexpr int GEMM_PACK_TILES = 4;    // tiles padded to a multiple of the largest TPW


// LDS rows of a wave's X chunk (one column block, 16 steps): 16 rows of 512
// channels, padded by 16 bytes so the rows of a 16-lane read fall in
// different banks.
constexpr int XROW_BYTES = 16 * 64 + 16;
constexpr int XREG_BYTES = 16 * XROW_BYTES;

// The fused q/k/v projection's epilogue for one lane: channels i .. i + 3
// of head `head` (i < d / 2) and their partners i + d / 2 .. for sequence
// m, as x0 / x1 (fp16, bias added); rotated and stored as
// rope_write_decode_kernel stores them (the same rounding, bit-equal).
__device__ __forceinline__ void rope_store(const RopeWriteParams& a, int m, int head, int i,
                                           const half_t* x0, const half_t* x1) {
    const int hd = a.d / 2;
    int64_t p = a.pos[m];
    p = p < 0 ? 0 : (p >= a.tab_rows ? a.tab_rows - 1 : p);
    const half_t* c = (const half_t*)a.cos + p * a.st;
    const half_t* s = (const half_t*)a.sin + p * a.st;
    half_t o0[4], o1[4];
    if (head < a.hq + a.hk) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o0[e] = rope_h(x0[e], c[i + e], -x1[e], s[i + e]);
            o1[e] = rope_h(x1[e], c[i + hd + e], x0[e], s[i + hd + e]);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o0[e] = x0[e];
            o1[e] = x1[e];
        }
    }
    half_t* dst;
    if (head < a.hq) {
        const int n_rep = a.hq / a.hk;
        dst = (half_t*)a.q_out + (int64_t)m * a.sq_b + (int64_t)(head / n_rep) * a.sq_h +
              (int64_t)(head % n_rep) * a.sq_r;
    } else {
        const int64_t slot = a.slots[m];
        if (slot < 0) return;
        const int64_t blk = slot / a.page, off = slot % a.page;
        if (blk >= a.num_blocks) return;
        const bool isk = head < a.hq + a.hk;
        const int h = isk ? head - a.hq : head - a.hq - a.hk;
        dst = (half_t*)(isk ? a.k_pool : a.v_pool) + blk * a.sp_b + off * a.sp_t +
              (int64_t)h * a.sp_h;
        if (isk && a.kmin) {
            // the page's K bounds: its first token resets them (fp16 min /
            // max are exact)
            half_t* mn = (half_t*)a.kmin + blk * a.sb_b + (int64_t)h * a.sb_h;
            half_t* mx = (half_t*)a.kmax + blk * a.sb_b + (int64_t)h * a.sb_h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (off == 0) {
                    mn[i + e] = o0[e];
                    mx[i + e] = o0[e];
                    mn[i + hd + e] = o1[e];
                    mx[i + hd + e] = o1[e];
                } else {
                    mn[i + e] = (half_t)fminf((float)mn[i + e], (float)o0[e]);
                    mx[i + e] = (half_t)fmaxf((float)mx[i + e], (float)o0[e]);
                    mn[i + hd + e] = (half_t)fminf((float)mn[i + hd + e], (float)o1[e]);
                    mx[i + hd + e] = (half_t)fmaxf((float)mx[i + hd + e], (float)o1[e]);
                }
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        dst[i + e] = o0[e];
        dst[i + hd + e] = o1[e];
    }
}

// One workgroup a (TPW tiles, split); its blockDim.x / 64 waves take
// consecutive K chunks of the split's range.  MB column blocks of 16 rows
// of X.  The waves' tiles are summed through LDS (blockDim.x / 64 * TPW *
// MB KiB of dynamic shared memory).
// PW: the weight is packed.  LX (one column block of 16-step chunks): the
// wave's X chunk is brought to its own LDS rows by direct loads (1 KiB of
// one row each) and read from there in MFMA order; the same LDS then holds
// the wave's partial tiles for the group's sum.  (X loaded straight to
// registers reads 64 bytes of each of 16 rows per instruction.)
// One step of a reduce-scatter over the lanes: lanes with `BIT` clear keep
// values 0 .. HALF - 1 and send the upper HALF, lanes with it set the
// reverse; each kept value adds the partner's.  (Selecting by value keeps
// the array in registers; selecting an index would turn into a search.)
// h = fp16(w * fp16(s * inv)) on 8 channels: the fp32 scale rounded to
// fp16, then the weight product in packed fp16 (exact product, one rounding)
__device__ __forceinline__ u4 norm_row(u4 sv, u4 wv, float inv) {
    // (bit casts take named scalars: this compiler casts an element of a
    // vector lvalue from the vector's first element)
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t hw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const h2 s2 = __builtin_bit_cast(h2, sw[e]);
        const h2 n2 = {(half_t)((float)s2.x * inv), (half_t)((float)s2.y * inv)};
        hw[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, ww[e]) * n2);
    }
    return (u4){hw[0], hw[1], hw[2], hw[3]};
}

template <int HALF, int BIT>
__device__ __forceinline__ void reduce_step(float* v, int lane) {
    const uint32_t hi = (lane & BIT) ? ~0u : 0u;
#pragma unroll
    for (int j = 0; j < HALF; ++j) {
        const uint32_t a = __builtin_bit_cast(uint32_t, v[j]);
        const uint32_t b = __builtin_bit_cast(uint32_t, v[j + HALF]);
        const float send = __builtin_bit_cast(float, (a & hi) | (b & ~hi));
        const float keep = __builtin_bit_cast(float, (b & hi) | (a & ~hi));
        v[j] = keep + __shfl_xor(send, BIT);
    }
}

template <int SPW, int TPW, int MB, int EPI, bool PW, bool LX, bool NRM = false>
__global__ __launch_bounds__(256) void decode_gemm_kernel(GemmParams a) {
    static_assert(!LX || (MB == 1 && SPW == 16), "LDS X: one column block, 16-step chunks");
    static_assert(!NRM || LX, "the norm prologue works on the LDS rows");
    __shared__ float nrm_part[NRM ? 4 : 1][16];       // [wave][row] sums of squares
    extern __shared__ f4 red[];                       // [waves][TPW][MB][WAVE] (LX: per wave)
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
    u4 xb[LX ? 1 : SPW][MB];
    u4 wb[2][SPW];
    char* const xl = (char*)red + wv * XREG_BYTES;    // LX: this wave's X rows
    auto load_w = [&](int b, int t) {
        const half_t* wp;
        int step_halves;
        if (PW) {
            wp = (const half_t*)a.w + (((int64_t)(tile0 + t) * steps + s0) * WAVE + lane) * 8;
            step_halves = WAVE * 8;
        } else {
            wp = (const half_t*)a.w + (int64_t)w_row<EPI>(a, tile0 + t, r) * a.ldw + 32 * s0 +
                 8 * g;
            step_halves = 32;
        }
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int st = i < last ? i : last;
            wb[b][i] = *(const u4*)(wp + step_halves * st);
        }
    };
    if constexpr (LX) {
        // row q's 512 channels of the chunk: lane l brings channels 8l ..
        // 8l + 7 (a chunk shorter than 16 steps reads clamped channels whose
        // steps are masked)
        const int col = 32 * s0 + 8 * lane < a.K - 8 ? 32 * s0 + 8 * lane : a.K - 8;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int m = q < a.M ? q : a.M - 1;
            __builtin_amdgcn_global_load_lds(
                (const void*)((const half_t*)a.x + (int64_t)m * a.ldx + col),
                (__attribute__((address_space(3))) void*)(xl + q * XROW_BYTES), 16, 0, 0);
        }
    } else {
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int st = i < last ? i : last;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) xb[i][mb] = *(const u4*)(xp[mb] + 32 * st);
        }
    }
    // norm prologue: this lane's residual channels of every row, and the
    // norm weight of its channels (requested before the weight loads)
    u4 rv[NRM ? 16 : 1];
    u4 nwv = {0u, 0u, 0u, 0u};
    const int ncol = 32 * s0 + 8 * lane < a.K - 8 ? 32 * s0 + 8 * lane : a.K - 8;
    if constexpr (NRM) {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int m = q < a.M ? q : a.M - 1;
            rv[q] = *(const u4*)((const half_t*)a.nres + (int64_t)m * a.ldr + ncol);
        }
        nwv = *(const u4*)((const half_t*)a.nw + ncol);
    }
    load_w(0, 0);
    // with the norm prologue the second tile's weights are requested after
    // it, so the residual rows and those weights are not in registers at once
    if (TPW > 1 && !NRM) load_w(1, 1);
    if constexpr (LX) {
        // the X rows were requested before every weight load: once no more
        // than the weight loads are outstanding, they are in LDS
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(SPW * (TPW > 1 && !NRM ? 2 : 1)));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NRM) {
        // Every workgroup normalises the rows itself (they are 16 x K), so
        // this is written for few instructions: packed fp16 adds and
        // multiplies, which round as the fp32 operation rounded to fp16 does
        // (the fp32 sum or product of two fp16 values is exact, or rounds
        // innocuously), and one butterfly reduce-scatter for the 16 rows'
        // sums of squares.
        //
        // s = res + x (fp16) on the lane's 8 channels of each row, written
        // over x in LDS; channels past the wave's chunk belong to the next
        // wave and are not counted.
        const bool mine = 8 * lane < 32 * ns;
        float ss[16];
        u4 sv[16];
        // all 16 reads first, then the sums, then the writes: one LDS round
        // trip for the rows rather than one a row
#pragma unroll
        for (int q = 0; q < 16; ++q) sv[q] = *(const u4*)(xl + q * XROW_BYTES + lane * 16);
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const uint32_t xw[4] = {sv[q].x, sv[q].y, sv[q].z, sv[q].w};
            const uint32_t rw[4] = {rv[q].x, rv[q].y, rv[q].z, rv[q].w};
            uint32_t sw[4];
            float acc = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const h2 t = __builtin_bit_cast(h2, rw[e]) + __builtin_bit_cast(h2, xw[e]);
                acc = __builtin_amdgcn_fdot2(t, t, acc, false);
                sw[e] = __builtin_bit_cast(uint32_t, t);
            }
            sv[q] = (u4){sw[0], sw[1], sw[2], sw[3]};
            ss[q] = mine ? acc : 0.f;
        }
#pragma unroll
        for (int q = 0; q < 16; ++q) *(u4*)(xl + q * XROW_BYTES + lane * 16) = sv[q];
        // workgroup 0 stores the new residual (its waves cover the row)
        if (blockIdx.x == 0 && mine) {
#pragma unroll
            for (int q = 0; q < 16; ++q)
                if (q < a.M) *(u4*)((half_t*)a.nres_out + (int64_t)q * a.ldro + ncol) = sv[q];
        }
        // reduce-scatter over the lanes: after the xor-32/16/8/4 steps lane l
        // holds row (l >> 2) summed over the 16 lanes sharing its low 2 bits
        reduce_step<8, 32>(ss, lane);
        reduce_step<4, 16>(ss, lane);
        reduce_step<2, 8>(ss, lane);
        reduce_step<1, 4>(ss, lane);
        float tot = ss[0];
        tot += __shfl_xor(tot, 2);
        tot += __shfl_xor(tot, 1);
        if ((lane & 3) == 0) nrm_part[wv][lane >> 2] = tot;
        __syncthreads();
        if (TPW > 1) load_w(1, 1);
        // lane q < 16: 1 / rms of row q over the group's waves (in wave order)
        float inv;
        {
            const int q = lane & 15;
            float t = 0.f;
            for (int p = 0; p < nw; ++p) t += nrm_part[p][q];
            inv = 1.f / sqrtf(t / (float)a.K + a.eps);
        }
        // h = fp16(w * fp16(s * inv)) in place, the rounding of Qwen2RMSNorm
        // in fp16 (applied here once rather than per weight tile as the
        // product reads the rows: that costs more where tiles are many)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            char* row = xl + q * XROW_BYTES + lane * 16;
            const float iq = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv), q));
            *(u4*)row = norm_row(*(const u4*)row, nwv, iq);
        }
        asm volatile("" ::: "memory");
    }
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
                u4 xv;
                if constexpr (LX)
                    xv = live ? *(const u4*)(xl + r * XROW_BYTES + (32 * i + 8 * g) * 2) : z;
                else
                    xv = live ? xb[i][mb] : z;
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
        // wave p's partials: its own X rows when LX (another wave may still
        // be reading its own), else slot p
        auto slot = [&](int p) {
            return LX ? (f4*)((char*)red + p * XREG_BYTES) : red + p * TPW * MB * WAVE;
        };
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) slot(wv)[(t * MB + mb) * WAVE + lane] = acc[t][mb];
        __syncthreads();
        if (wv != 0) return;
        for (int p = 1; p < nw; ++p)
#pragma unroll
            for (int t = 0; t < TPW; ++t)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[t][mb] += slot(p)[(t * MB + mb) * WAVE + lane];
    }
    // wave 0 alone from here

    if (EPI == GEMM_ROPE) {
        // splits == 1 (host): lanes g = 0, 1 hold channels 8t + 4g + e of the
        // tile's head, lanes g + 2 their rotate-half partners
        const int tph = a.rope.d / 16;
#pragma unroll
        for (int t = 0; t < TPW; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                f4 up;
#pragma unroll
                for (int e = 0; e < 4; ++e) up[e] = __shfl_xor(acc[t][mb][e], 32);
                const int tile = tile0 + t, head = tile / tph, i = 8 * (tile % tph) + 4 * g;
                const int m = 16 * mb + r;
                if (g >= 2 || m >= a.M || head >= a.rope.hq + 2 * a.rope.hk) continue;
                const int n0 = head * a.rope.d + i, n1 = n0 + a.rope.d / 2;
                half_t x0[4], x1[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v0 = acc[t][mb][e], v1 = up[e];
                    if (a.bias) {
                        v0 += (float)((const half_t*)a.bias)[n0 + e];
                        v1 += (float)((const half_t*)a.bias)[n1 + e];
                    }
                    x0[e] = (half_t)v0;
                    x1[e] = (half_t)v1;
                }
                rope_store(a.rope, m, head, i, x0, x1);
            }
        return;
    }
    if (EPI == GEMM_GLU) {
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
    // the write-through partials complete before the arrival count
    handoff_release();
    int prev = 0;
    if (lane == 0)
        prev = __hip_atomic_fetch_add(a.counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0);
    if (prev != a.splits - 1) return;
    // Every split of these tiles has arrived; their partials are read with
    // device-coherent loads.  Unit u = (t, m, q): four columns.
    const int64_t split_stride = (int64_t)a.M * ldp;
    for (int u = lane; u < TPW * a.M * 4; u += WAVE) {
        const int t = u / (a.M * 4), m = (u / 4) % a.M, q = u % 4;
        const int nc = 16 * (tile0 + t) + 4 * q;
        if (nc >= a.N) continue;
        const float* pp = a.part + (int64_t)m * ldp + nc;
        f4 s = {0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < a.splits; ++sp)
#pragma unroll
            for (int e = 0; e < 4; ++e) s[e] += load_coherent(pp + sp * split_stride + e);
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

template <int TPW, int MB, int EPI>
void launch_kernel(const GemmParams& p, const GemmShape& sh, hipStream_t stream) {
    const dim3 grid(sh.units, p.splits), block(WAVE * sh.group_waves);
    if (p.w_packed && MB == 1) {
        const size_t lds = (size_t)sh.group_waves * XREG_BYTES;
        if (p.norm)
            hipLaunchKernelGGL((decode_gemm_kernel<spw_for(MB), TPW, MB, EPI, true, MB == 1, MB == 1>),
                               grid, block, lds, stream, p);
        else
            hipLaunchKernelGGL((decode_gemm_kernel<spw_for(MB), TPW, MB, EPI, true, MB == 1>),
                               grid, block, lds, stream, p);
        return;
    }
    const size_t lds =
        sh.group_waves > 1 ? (size_t)sh.group_waves * TPW * MB * WAVE * sizeof(f4) : 0;
    if (p.w_packed)
        hipLaunchKernelGGL((decode_gemm_kernel<spw_for(MB), TPW, MB, EPI, true, false>), grid,
                           block, lds, stream, p);
    else
        hipLaunchKernelGGL((decode_gemm_kernel<spw_for(MB), TPW, MB, EPI, false, false>), grid,
                           block, lds, stream, p);
}

template <int EPI>
void launch_any(const GemmParams& p, const GemmShape& sh, hipStream_t stream) {
    if (sh.mb == 1 && sh.tpw == 4)
        launch_kernel<4, 1, EPI>(p, sh, stream);
    else if (sh.mb == 1 && sh.tpw == 2)
        launch_kernel<2, 1, EPI>(p, sh, stream);
    else if (sh.mb == 1)
        launch_kernel<1, 1, EPI>(p, sh, stream);
    else if (sh.mb == 2)
        launch_kernel<1, 2, EPI>(p, sh, stream);
    else
        launch_kernel<1, 4, EPI>(p, sh, stream);
}

}  // namespace

int decode_gemm_splits(int M, int N, int K) { return gemm_shape(M, N, K).splits; }

int decode_gemm_units(int M, int N, int K) { return gemm_shape(M, N, K).units; }

namespace {

// grid (padded tiles, steps), 64 threads: lane (r, g) copies row r's
// channels 8g .. 8g + 7 of the step (zeros for rows past the weight).
template <int EPI>
__global__ __launch_bounds__(64) void pack_gemm_kernel(const half_t* w, int64_t ldw, int N, int K,
                                                       int d, half_t* out) {
    const int T = blockIdx.x, s = blockIdx.y, lane = threadIdx.x, r = lane & 15, g = lane >> 4;
    const int steps = K / 32;
    bool real;
    const int row = w_row_of<EPI>(N, d, T, r, real);
    u4 v = {0u, 0u, 0u, 0u};
    if (real) v = *(const u4*)(w + (int64_t)row * ldw + 32 * s + 8 * g);
    *(u4*)(out + (((int64_t)T * steps + s) * WAVE + lane) * 8) = v;
}

}  // namespace

size_t gemm_packed_bytes(int N, int K, int epi, int head_dim) {
    (void)epi;
    (void)head_dim;
    const int tiles = (N + 15) / 16;
    const int padded = (tiles + GEMM_PACK_TILES - 1) / GEMM_PACK_TILES * GEMM_PACK_TILES;
    return (size_t)padded * (K / 32) * WAVE * 16;
}

hipError_t launch_pack_gemm_weight(const void* w, int64_t ldw, int N, int K, int epi, int head_dim,
                                   void* packed, hipStream_t stream) {
    const int tiles = (N + 15) / 16;
    const int padded = (tiles + GEMM_PACK_TILES - 1) / GEMM_PACK_TILES * GEMM_PACK_TILES;
    const dim3 grid(padded, K / 32);
    if (epi == GEMM_GLU)
        hipLaunchKernelGGL(pack_gemm_kernel<GEMM_GLU>, grid, dim3(WAVE), 0, stream,
                           (const half_t*)w, ldw, N, K, head_dim, (half_t*)packed);
    else if (epi == GEMM_ROPE)
        hipLaunchKernelGGL(pack_gemm_kernel<GEMM_ROPE>, grid, dim3(WAVE), 0, stream,
                           (const half_t*)w, ldw, N, K, head_dim, (half_t*)packed);
    else
        hipLaunchKernelGGL(pack_gemm_kernel<GEMM_PLAIN>, grid, dim3(WAVE), 0, stream,
                           (const half_t*)w, ldw, N, K, head_dim, (half_t*)packed);
    return hipGetLastError();
}

size_t decode_gemm_workspace_bytes(int M, int N, int K) {
    const GemmShape sh = gemm_shape(M, N, K);
    if (sh.splits == 1) return 0;
    return GEMM_PART_OFFSET + (size_t)sh.splits * M * ((N + 3) & ~3) * sizeof(float);
}

hipError_t launch_decode_gemm(const GemmParams& p, hipStream_t stream) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    const GemmShape sh = gemm_shape(p.M, p.N, p.K);
    if (sh.splits != p.splits || sh.group_waves > MAX_GROUP_WAVES) return hipErrorInvalidValue;
    // the norm prologue: the LDS X path (packed weight, one column block),
    // a group covering the whole row
    if (p.norm && (!p.w_packed || sh.mb != 1 || p.splits != 1)) return hipErrorInvalidValue;
    if (p.epi == GEMM_GLU) {
        if (p.splits != 1 || p.N % 2 != 0) return hipErrorInvalidValue;
        launch_any<GEMM_GLU>(p, sh, stream);
    } else if (p.epi == GEMM_ROPE) {
        if (p.splits != 1 || p.N % 16 != 0 || p.rope.d % 16 != 0) return hipErrorInvalidValue;
        launch_any<GEMM_ROPE>(p, sh, stream);
    } else {
        launch_any<GEMM_PLAIN>(p, sh, stream);
    }
    return hipGetLastError();
}

}  // namespace ls
