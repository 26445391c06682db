// Shared device helpers for the gfx950 paged-decode kernels.
//
// Wave64 throughout.  Every kernel here is written for CDNA4 directly: 64-lane
// wavefronts, 16x16x16 f16 MFMA tiles, cross-lane traffic by ds_bpermute /
// readlane, no warp-32 assumptions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ls {

typedef _Float16 half_t;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// Measurement builds only (-DLS_STAMPS, never the shipped library): thread 0
// of each workgroup records the 100 MHz clock at numbered points of the
// decode (ls_diag_read_stamps copies the last launch's to the host).
#ifdef LS_STAMPS
constexpr int LS_NSTAMP = 32;   // 0-15: the group's points; 16-31: per wave (dense walks)
static __device__ uint64_t g_ls_stamps[8192 * LS_NSTAMP];
#define LS_STAMP(i)                                                                              \
    do {                                                                                         \
        if (threadIdx.x == 0)                                                                    \
            ::ls::g_ls_stamps[(blockIdx.x + gridDim.x * blockIdx.y) * ::ls::LS_NSTAMP + (i)] =   \
                __builtin_amdgcn_s_memrealtime();                                                \
    } while (0)
#else
#define LS_STAMP(i) do {} while (0)
#endif
constexpr int HEAD_DIM = 128;   // the lane mapping below covers exactly 128 channels
constexpr int PAGE = 16;        // one page = the M=16 side of a 16x16 MFMA tile
constexpr int MAX_NREP = 16;    // query rows per KV head = the N=16 side of the tile

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// A word of a buffer that other workgroups of the same launch fill: all ones
// (a NaN payload no arithmetic here produces) until its value is stored.
constexpr uint32_t EMPTY_WORD = 0xFFFFFFFFu;

// 2^x on the transcendental unit (v_exp_f32): exact 0 for -inf.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float shfl_xor(float v, int mask) {
    const int lane = __lane_id();
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2,
                                                                   __builtin_bit_cast(int, v)));
}

// Max / sum over the four 16-lane groups that share a lane's `lane & 15`.
__device__ __forceinline__ float group4_max(float v) {
    v = fmaxf(v, shfl_xor(v, 16));
    return fmaxf(v, shfl_xor(v, 32));
}
__device__ __forceinline__ float group4_sum(float v) {
    v += shfl_xor(v, 16);
    return v + shfl_xor(v, 32);
}

// Four signed int8 (one dword) -> four fp16, exactly: each byte, offset by
// 128, is spliced under the exponent of 1024.0h (0x64xx = 1024 + xx) and the
// 1152 bias is removed with one packed fp16 subtract per pair.
__device__ __forceinline__ u2 i8x4_to_h4(uint32_t x) {
    const uint32_t u = x ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2 bias = {(half_t)1152.0f, (half_t)1152.0f};
    const h2 a = __builtin_bit_cast(h2, lo) - bias;
    const h2 b = __builtin_bit_cast(h2, hi) - bias;
    u2 r;
    r.x = __builtin_bit_cast(uint32_t, a);
    r.y = __builtin_bit_cast(uint32_t, b);
    return r;
}

__device__ __forceinline__ h4 as_h4(uint32_t lo, uint32_t hi) {
    u2 t;
    t.x = lo;
    t.y = hi;
    return __builtin_bit_cast(h4, t);
}

// KV pages are read exactly once per call: non-temporal loads keep them from
// displacing the block tables, queries and partials in the caches.
template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
    return __builtin_nontemporal_load(p);
}

// A page's K or V of one KV head, as the decode walk reads it: one wave
// reads one (page, head) item, so the item's base address is the same in
// every lane and becomes a buffer resource in scalar registers; each lane
// adds its byte offset (below 2^31).  The loads carry the nontemporal and
// sc0 cache policy.  Against global nontemporal loads of the same bytes
// (B16 x 16K, one box, alternating): 48.87 -> 48.56 us (buffer loads with
// the nontemporal policy alone 48.65; sc1 with it 48.57; sc1 alone 54.2;
// plain loads 52.7).
// `fetch` false (the same in every lane): a resource of no bytes, whose
// loads return zeros without a memory request (the walk's requests for
// items past its end, which the compute masks).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const void* wave_uniform_base,
                                                            bool fetch = true) {
    const uint64_t x = (uint64_t)wave_uniform_base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    const int n = __builtin_amdgcn_readfirstlane(fetch ? 0x7fffffff : 0);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), 0, n, 0x00020000);
}
constexpr int PAGE_POLICY = 1 /* sc0 */ | 2 /* nt */;
__device__ __forceinline__ u4 page_load16(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, PAGE_POLICY));
}
// A scheduling barrier after each of an fp16 page's loads: the loads go out
// where the walk issues them, in order.  Left to the scheduler, they were
// moved among the compute of the page before (B16 x 16K: 48.46 -> 47.15 us
// with the barriers; an s_nop after each load, which also pins them,
// 47.51).  The INT8 walk is faster without them (B16 x 16K: 33.37 against
// 34.13 us).
__device__ __forceinline__ void issue_here() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ float page_load4(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, PAGE_POLICY));
}
__device__ __forceinline__ u2 page_load8(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, PAGE_POLICY));
}

// fp16(fp16(silu(g)) * u): the MLP activation as Hugging Face's fp16
// computation rounds it (silu in fp32 on the fp16 gate, rounded, then the
// fp16 product).  One definition serves every kernel that applies it, so
// their results are bit-equal.
__device__ __forceinline__ _Float16 silu_mul_h(_Float16 g, _Float16 u) {
#pragma clang fp contract(off)
    const float gf = (float)g;
    const _Float16 sg = (_Float16)(gf / (1.f + expf(-gf)));
    return (_Float16)((float)sg * (float)u);
}

// One RoPE output as Hugging Face's fp16 apply_rotary_pos_emb rounds it:
// fp16(fp16(x * c) + fp16(y * s)), y the rotate-half partner (negated for
// the first half).  Shared, so every kernel that rotates is bit-equal.
__device__ __forceinline__ _Float16 rope_h(_Float16 x, _Float16 c, _Float16 y, _Float16 s) {
#pragma clang fp contract(off)
    const _Float16 xc = (_Float16)((float)x * (float)c);
    const _Float16 ys = (_Float16)((float)y * (float)s);
    return (_Float16)((float)xc + (float)ys);
}

// Hand-off of partial results between the workgroups of one launch: many
// groups write their partials, then bump an arrival counter (a relaxed
// agent-scope RMW); the group that brings the count to its target reads
// them all.
//
// Release side: the partials are stored write-through at device coherence
// (sc1: the line is written to memory, not held dirty in this XCD's L2) and
// handoff_release() waits for those stores to complete before the RMW is
// issued.  This is the release the partials need, stated at the ISA level:
// the HIP model's agent-scope release fence would add a write-back of the
// whole L2 (buffer_wbl2) in every wave, measured at +16 us a launch on the
// B16 x 16K decode (49.6 -> 65.5 us).  Only stores made write-through may
// be handed off this way.
// Acquire side: the last arriver reads the partials with device-coherent
// loads (sc1: relaxed agent-scope atomic loads of up to 8 bytes, 16-byte
// buffer loads with the sc1 policy), issued after its RMW has
// returned the final count (the branch on it orders them), so no line can
// come from a stale copy in its XCD's L2.  The model's agent-scope acquire
// fence (an invalidate of the reader's whole L2) measured +2.1 us a launch
// on the same decode; these loads +0.65 us (49.5 -> 50.2 us), over the
// plain loads an earlier form used, which were right only while the
// reader's L2 held no copy of the partials' lines.
// Device-coherent loads (sc1: served from memory or a coherent copy, never
// from a stale line in this XCD's L2), as relaxed agent-scope atomic loads.
template <class T>
__device__ __forceinline__ T load_coherent(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sixteen bytes the same way: a raw buffer load with the sc1 cache policy
// (buffer_load_dwordx4 ... sc1 nt), from a resource over `base` (offsets in
// bytes, below 2^31).  A builtin, so the compiler inserts the wait before
// any use of the value, as for the atomic loads above.  (An inline-asm load
// is not tracked: with an explicit wait after it the compiler still took
// the asm's outputs as ready at once, and reading m and l of the records
// that way gave wrong results.)
// A pointer that is the same in every lane of the wave, declared so: the
// compiler otherwise keeps a value derived from threadIdx (a head of the
// group, say) in vector registers, and a buffer resource built from it
// becomes a loop of one-lane-group loads, each waiting for the one before.
template <class T>
__device__ __forceinline__ T* wave_uniform(T* p) {
    const uint64_t x = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return (T*)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const float* base) {
    // (dword 3: the raw-buffer format bits CDNA's buffer instructions expect)
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ f4 load_coherent4(__amdgpu_buffer_rsrc_t rs, int byte_off) {
    // the cache-policy operand: sc1 (device coherent) | nt (each record is
    // read once: 0.05 us faster at B16 x 16K than sc1 alone)
    constexpr int POLICY = 16 | 2;
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, POLICY));
}

// (soff: a wave-uniform byte offset, in a scalar register)
__device__ __forceinline__ f4 load_coherent4(__amdgpu_buffer_rsrc_t rs, int byte_off, int soff) {
    constexpr int POLICY = 16 | 2;
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, soff, POLICY));
}
__device__ __forceinline__ uint64_t load_coherent8(__amdgpu_buffer_rsrc_t rs, int byte_off, int soff) {
    constexpr int POLICY = 16 | 2;
    return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(rs, byte_off, soff, POLICY));
}

// Workgroup ids renumbered XCD-major.  The dispatcher deals a launch's
// workgroups to the 8 XCDs in turn (linear id L goes to XCD L % 8, the
// XCD's (L / 8)-th), so numbering the XCD's groups contiguously,
//   u = (groups on XCDs before L % 8) + L / 8,
// gives the groups of one sequence (adjacent u) one XCD and its L2: the
// sequence's block table, query and split records stay in one cache.  A
// bijection of [0, N) for any N; correctness never depends on where a
// group actually runs, only the speed does.
__device__ __forceinline__ int xcd_major(int L, int N) {
    constexpr int XCDS = 8;
    const int q = N / XCDS, rem = N % XCDS, x = L % XCDS;
    return x * q + (x < rem ? x : rem) + L / XCDS;
}

// s_waitcnt with vmcnt = n and the other counters left alone (gfx9 encoding).
constexpr int vmcnt_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Wait until at most n vector memory instructions of this wave are
// outstanding, as a compiler barrier for memory: the compiler does not track
// the LDS writes of direct-to-LDS loads, so LDS reads of their data follow
// such a wait (n counted from the instructions issued after those loads).
template <int N_AFTER>
__device__ __forceinline__ void wait_vm_lds() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_wait(N_AFTER));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// What the runtime reports of a loaded kernel (ls_kernel_resources).
struct KernelResources {
    int regs, local_bytes, shared_bytes, threads, groups_per_cu;
};
template <class F>
inline hipError_t func_resources(F* fn, int threads, KernelResources* r) {
    hipFuncAttributes at;
    hipError_t e = hipFuncGetAttributes(&at, reinterpret_cast<const void*>(fn));
    if (e != hipSuccess) return e;
    r->regs = at.numRegs;
    r->local_bytes = (int)at.localSizeBytes;
    r->shared_bytes = (int)at.sharedSizeBytes;
    r->threads = threads;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&r->groups_per_cu,
                                                        reinterpret_cast<const void*>(fn), threads, 0);
}

__device__ __forceinline__ void handoff_release() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace ls
