// dev_common.h — device helpers shared by the gfx950 kernels (decode,
// routing, batched): operand types and conversions, buffer loads, LDS
// barriers, work-group reductions, the top-k, and the routing arithmetic that
// the decode and routing kernels must share bit for bit. Included by the
// kernel translation units only.
#pragma once
#include <hip/hip_runtime.h>

#include "internal.h"

namespace wl {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

#define WL_DEV static __device__ __forceinline__

WL_DEV float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
WL_DEV uint32_t f2bf(float f) {  // round to nearest even
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}
// E8M0 byte -> 2^(b-127); 0xFF is NaN (reference e8m0_to_f32, src/glm_kernels.cuh:53-61).
WL_DEV float e8m0f(uint32_t b) {
    float v = __uint_as_float(b << 23);
    v = (b == 0u) ? __uint_as_float(0x00400000u) : v;
    v = (b == 0xFFu) ? __uint_as_float(0x7FC00000u) : v;
    return v;
}
// e8m0f(b) if on, else +0, for a wave-uniform on: the decoded bits ANDed
// with an all-ones or all-zero scalar mask. (A select on a uniform condition
// compiles to a branch around the decode, several per step; the mask is kept
// opaque so it is not folded back into that select.)
WL_DEV float e8m0f_if(uint32_t b, bool on) {
    uint32_t m = __builtin_amdgcn_readfirstlane(on ? ~0u : 0u);
    asm("" : "+s"(m));
    return __uint_as_float(__float_as_uint(e8m0f(b)) & m);
}
// 8 FP4 values (one dword, low nibble first) -> 8 scaled bf16 values.
WL_DEV bf16x8 fp4x8_bf16(uint32_t w, float sc) {
    bf16x2 c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
    bf16x2 c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
    bf16x2 c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
    bf16x2 c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
    u32x4 u = {__builtin_bit_cast(uint32_t, c0), __builtin_bit_cast(uint32_t, c1),
               __builtin_bit_cast(uint32_t, c2), __builtin_bit_cast(uint32_t, c3)};
    return __builtin_bit_cast(bf16x8, u);
}
WL_DEV f32x4 mma(bf16x8 a, bf16x8 b, f32x4 d) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, d, 0, 0, 0);
}
WL_DEV bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
typedef __attribute__((address_space(1))) const uint8_t g_u8;
// 16-byte and 1-byte loads from global memory (never through the flat path:
// a flat access also counts against the LDS wait counter, so every LDS wait
// would wait for it too).
WL_DEV u32x4 gld16(const void* p) { return *(g_u32x4*)p; }
WL_DEV uint32_t gld1(const uint8_t* p) { return *(g_u8*)p; }
template <class T>
WL_DEV T gld(const T* p) { return *(const __attribute__((address_space(1))) T*)p; }
template <class T>
WL_DEV void gst(T* p, T v) { *(__attribute__((address_space(1))) T*)p = v; }
// Raw buffer loads: a uniform 128-bit resource (base, size) in SGPRs, a
// per-lane byte offset in a VGPR and a uniform per-instruction offset in an
// SGPR, so a batch of loads costs no address registers per load. Offsets past
// `bytes` read as zero instead of faulting.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
WL_DEV rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}
WL_DEV u32x4 bld16(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}
// Weight streams (read once per call): the non-temporal hint (aux bit 1).
// Measured on MI355X: a 240 MB one-launch stream takes 38.6 us with it and
// 43.3 us without.
constexpr int kNT = 2;
WL_DEV u32x4 bld16_nt(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kNT);
}
// A lane offset past every resource: the load returns zeros without a
// memory access. (The range check sees the lane offset; an out-of-range
// value must be put there, not in the uniform offset.)
constexpr uint32_t kOOB = 0x80000000u;
WL_DEV uint32_t bld1(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, (int)voff, (int)soff, 0);
}
// Agent-scope (sc1) accesses for data one work-group writes and others read:
// the store writes through the writer's L2, the load bypasses the reader's L1
// and L2 (aux bit 4 of the buffer instructions is sc1).
constexpr int kSC1 = 16;
WL_DEV void st_ag(float* p, float v) {
    __hip_atomic_store((__attribute__((address_space(1))) uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
WL_DEV uint32_t bld4_ag(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, kSC1);
}
WL_DEV u32x4 bld16_ag(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kSC1);
}
// A value the compiler must treat as uniform across the wave (it is).
WL_DEV uint32_t uni(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }
WL_DEV const uint8_t* uni_ptr(const uint8_t* p) {
    const uint64_t u = (uint64_t)p;
    return (const uint8_t*)(((uint64_t)uni((uint32_t)(u >> 32)) << 32) | uni((uint32_t)u));
}

// A operand: piece row r (< 3) of a [3][stride] bf16 array, 8 values at col;
// zero for the other rows and for masked k tiles (valid == false).
WL_DEV bf16x8 a_lds(const uint16_t* base, uint32_t stride, uint32_t r, uint32_t col, bool valid) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < 3u && valid) v = *(const u32x4*)(base + r * stride + col);
    return as_bf16x8(v);
}
// The A operand of an MFMA whose callers read output rows 0-2 only (the
// three pieces of one vector): lanes of rows 3-15 read row 2 again, so the
// read needs no per-lane condition (their output rows are never read). A
// masked item (valid false, wave-uniform) reads column 0 instead; its B
// operand is exactly zero, so the finite values read there add nothing.
WL_DEV bf16x8 a_rows3(const uint16_t* base, uint32_t stride, uint32_t r, uint32_t col, bool valid) {
    return as_bf16x8(*(const u32x4*)(base + min(r, 2u) * stride + (valid ? col : 0u)));
}
WL_DEV bf16x8 a_any(const uint16_t* base, uint32_t stride, uint32_t r, uint32_t col, bool valid) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < 3u && valid) v = *(const u32x4*)(base + r * stride + col);
    return as_bf16x8(v);
}
WL_DEV float sum3(f32x4 d) { return d[0] + d[1] + d[2]; }

WL_DEV void split3(float x, uint32_t& h, uint32_t& m, uint32_t& l) {
    h = f2bf(x);
    const float r1 = x - bf2f(h);
    m = f2bf(r1);
    const float r2 = r1 - bf2f(m);
    l = f2bf(r2);
}

WL_DEV float silu_mul(float g, float u) {
    // x / (1 + exp(-x)) * u, as tools/ref_glm_chain.py:123-124 and
    // src/glm_layer_runner.cuh:338-341 (with an accurate exp).
    return (g / (1.0f + expf(-g))) * u;
}

// v_permlane32_swap: lo = [x lanes 0-31, y lanes 0-31], hi = [x lanes 32-63, y lanes 32-63].
WL_DEV void swap32(uint32_t x, uint32_t y, uint32_t& lo, uint32_t& hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
    lo = r[0];
    hi = r[1];
}

// ---- barriers ------------------------------------------------------------
// A work-group barrier that orders LDS only. __syncthreads() also waits for
// every outstanding global load of the wave, which would drain the weights a
// wave has in flight for its next batch.
WL_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Wait until this wave's global stores (and, the counter being in order, its
// earlier loads) have completed.
WL_DEV void vm_drain() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0), expcnt/lgkmcnt untouched

typedef __attribute__((address_space(1))) uint32_t g_u32;
WL_DEV uint32_t ld_sync(uint32_t* p) {
    return __hip_atomic_load((g_u32*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
WL_DEV void st_sync(uint32_t* p, uint32_t v) {
    __hip_atomic_store((g_u32*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
WL_DEV uint32_t rmw_inc(uint32_t* p) {
    return __hip_atomic_fetch_add((g_u32*)p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Records error bits (sticky) and marks call `epoch` as aborted, so the other
// work-groups of this call stop waiting for data that will not come.
WL_DEV void raise_error(uint32_t* sync, const SyncMap& m, uint32_t bits, uint32_t epoch) {
    __hip_atomic_fetch_or((g_u32*)(sync + m.error), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    st_sync(sync + m.abort, epoch);
}
// Whether call `epoch` was aborted by one of its work-groups.
WL_DEV bool aborted(uint32_t* sync, const SyncMap& m, uint32_t epoch) { return ld_sync(sync + m.abort) == epoch; }


// Sum over the 512 threads of the work-group (result in every thread).
WL_DEV float block_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; i++) s += red[i];
    lds_barrier();
    return s;
}

// ---- batches ------------------------------------------------------------
constexpr int kNB = 8;
static_assert(16 % kNB == 0, "a batch's scales must lie in one 16-byte chunk");
struct Batch {
    u32x4 w[kNB];
    u32x4 sv;  // the 16-byte scale chunk holding this batch's scales (MXFP4 streams)
};
// Scale chunks hold 16 consecutive items, and a batch's first item is a
// multiple of kNB = 8, so its scales are one half of the chunk: the half is
// chosen once per batch (lo, hi = its two dwords), and item i's byte sits at
// a compile-time position.
static_assert(kNB == 8, "a batch's scales are half of a 16-byte chunk");
struct BatchScales {
    uint32_t lo, hi;
};
WL_DEV BatchScales batch_scales(const Batch& B, uint32_t item0) {
    const bool upper = (item0 & 8u) != 0u;
    return BatchScales{upper ? B.sv.z : B.sv.x, upper ? B.sv.w : B.sv.y};
}
WL_DEV uint32_t batch_scale8(const BatchScales& s, int i) { return ((i < 4 ? s.lo : s.hi) >> (8 * (i % 4))) & 0xFFu; }

// A batch of the bf16 shared expert's gate/up stream: kSNB k tiles per wave,
// plus one 8-byte read of a logit slot, so the logits are collected while the
// weights stream. (Measured on MI355X: 4-tile batches shorten the norm's wait
// but starve the stream, 8 is faster overall.)
constexpr int kSNB = 8;
struct SBatch {
    u32x4 w[kSNB];
    uint64_t pl;
};

// A batch of an MXFP4 shared expert's gate/up stream (decode kernel): kSNB4
// k tiles of this wave's share of the work-group's tile, their scale dwords,
// and a logit slot read.
constexpr int kSNB4 = 4;
struct SBatch4 {
    u32x4 w[kSNB4];
    uint32_t s[kSNB4];
    uint64_t pl;
};

// Two-deep software pipeline over nb >= 2 batches: A holds batch 0 and B
// batch 1 on entry, both already issued. Batch b+2 is issued right after
// batch b is consumed; no batch is issued that is not consumed.
template <class BT, class IssueF, class ConsumeF>
WL_DEV void pingpong(uint32_t nb, BT& A, BT& B, IssueF issue, ConsumeF consume) {
    uint32_t b = 0;
#pragma unroll 1
    for (; b + 3 < nb; b += 2) {
        consume(b, A);
        issue(b + 2, A);
        consume(b + 1, B);
        issue(b + 3, B);
    }
    if (nb - b == 3u) {
        consume(b, A);
        issue(b + 2, A);
        consume(b + 1, B);
        consume(b + 2, A);
    } else {
        consume(b, A);
        consume(b + 1, B);
    }
}

WL_DEV uint32_t cdiv(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }
WL_DEV uint32_t at_least2(uint32_t a) { return a < 2u ? 2u : a; }

// ---- top-k -------------------------------------------------------------------
// Scores, biased choices (a NaN choice never wins), ranks with ties to the
// lowest index, then the K selected ids and unbiased scores in descending
// biased order (reference router_sigmoid_topk, src/glm_layer_runner.cuh:
// 304-336; tools/ref_glm_chain.py:127-149): sidx[0..K) and sw[0..K) in LDS.
WL_DEV void topk_score(float logit, float bias, uint32_t e, float* sc, float* ch) {
    const float s = 1.0f / (1.0f + expf(-logit));
    float c = s + bias;
    if (c != c) c = -INFINITY;
    sc[e] = s;
    ch[e] = c;
}
// Rank of every expert among the E choices (one thread per expert, the
// choices read as broadcast 16-byte LDS loads, 16 in flight at a time).
WL_DEV void topk_rank(uint32_t E, uint32_t K, const float* sc, const float* ch, uint32_t* sidx, float* sw) {
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        const float c = ch[e];
        uint32_t rank = 0;
#pragma unroll 16
        for (uint32_t j = 0; j < E; j += 4) {
            const float4 q = *(const float4*)(ch + j);
            rank += (q.x > c || (q.x == c && j + 0 < e)) ? 1u : 0u;
            rank += (q.y > c || (q.y == c && j + 1 < e)) ? 1u : 0u;
            rank += (q.z > c || (q.z == c && j + 2 < e)) ? 1u : 0u;
            rank += (q.w > c || (q.w == c && j + 3 < e)) ? 1u : 0u;
        }
        if (rank < K) {
            sidx[rank] = e;
            sw[rank] = sc[e];
        }
    }
    lds_barrier();
}
// Largest value over the 64 lanes, returned uniform. DPP quad permutes, row
// shifts and row broadcasts (VALU only) leave the maximum in lane 63.
template <int CTRL, int ROWS>
WL_DEV uint32_t max_step(uint32_t x) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, ROWS, 0xF, false);
    return o > x ? o : x;
}
WL_DEV uint32_t wave_max_u32(uint32_t x) {
    x = max_step<0xB1, 0xF>(x);   // quad_perm [1,0,3,2]
    x = max_step<0x4E, 0xF>(x);   // quad_perm [2,3,0,1]
    x = max_step<0x114, 0xF>(x);  // row_shr:4
    x = max_step<0x118, 0xF>(x);  // row_shr:8
    x = max_step<0x142, 0xA>(x);  // row_bcast:15
    x = max_step<0x143, 0xC>(x);  // row_bcast:31
    return __builtin_amdgcn_readlane(x, 63);
}
// Order-preserving map of a float to uint32 (NaN never reaches it).
WL_DEV uint32_t fkey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// E <= 256: K rounds of a wave-wide argmax (one whole wave, expert lane +
// 64m in slot m of each lane) over fkey(choice): the largest choice, ties to
// the lowest index (the first set bit of the first slot that holds the
// maximum), i.e. the reference's K serial argmax passes
// (src/glm_layer_runner.cuh:318-330). Keys of real experts are > 0
// (fkey(-inf) > 0); 0 marks an empty slot or a taken expert. No barrier: the
// caller orders sidx/sw for the other waves.
WL_DEV void topk_argmax_wave(uint32_t E, uint32_t K, const float* sc, const float* ch, uint32_t* sidx, float* sw) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t key[4];
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const uint32_t e = lane + 64u * m;
        key[m] = e < E ? fkey(ch[e]) : 0u;
    }
    for (uint32_t k = 0; k < K; k++) {
        const uint32_t a01 = key[0] > key[1] ? key[0] : key[1];
        const uint32_t a23 = key[2] > key[3] ? key[2] : key[3];
        const uint32_t mx = wave_max_u32(a01 > a23 ? a01 : a23);
        const uint64_t b0 = __builtin_amdgcn_ballot_w64(key[0] == mx);
        const uint64_t b1 = __builtin_amdgcn_ballot_w64(key[1] == mx);
        const uint64_t b2 = __builtin_amdgcn_ballot_w64(key[2] == mx);
        const uint64_t b3 = __builtin_amdgcn_ballot_w64(key[3] == mx);
        const uint32_t e = b0 ? (uint32_t)__builtin_ctzll(b0)
                         : b1 ? 64u + (uint32_t)__builtin_ctzll(b1)
                         : b2 ? 128u + (uint32_t)__builtin_ctzll(b2)
                              : 192u + (uint32_t)__builtin_ctzll(b3);
#pragma unroll
        for (int m = 0; m < 4; m++)
            if (lane + 64u * m == e) key[m] = 0u;
        if (lane == 0) sidx[k] = e;
    }
    // one wave: its LDS accesses complete in program order
    if (lane < K) sw[lane] = sc[sidx[lane]];
}
// The same by wave 0 of the work-group, then a barrier.
WL_DEV void topk_argmax(uint32_t E, uint32_t K, const float* sc, const float* ch, uint32_t* sidx, float* sw) {
    if (threadIdx.x < 64) topk_argmax_wave(E, K, sc, ch, sidx, sw);
    lds_barrier();
}

// Routing weight of slot k: score / (sum of the K scores + 1e-20) x scaling.
WL_DEV float topk_weight(const DecodeArgs& a, uint32_t K, const float* sw, uint32_t k) {
    float sum = 0.f;
    for (uint32_t i = 0; i < K; i++) sum += sw[i];
    float w = sw[k];
    if (a.norm_topk) w = w / (sum + 1e-20f);
    return w * a.scaling;
}

// AND of a per-thread predicate over the work-group (LDS only).
WL_DEV bool block_all(bool p, uint32_t* flags) {
    const bool wv = __all(p);
    if ((threadIdx.x & 63) == 0) flags[threadIdx.x >> 6] = wv ? 1u : 0u;
    lds_barrier();
    const uint4 f0 = *(const uint4*)flags, f1 = *(const uint4*)(flags + 4);
    const bool r = (f0.x & f0.y & f0.z & f0.w & f1.x & f1.y & f1.z & f1.w) != 0u;
    lds_barrier();
    return r;
}

// ---- routing prologue pieces shared by the decode and route kernels ---------
// Both kernels must produce bit-identical logits (a cache-backed layer is
// routed by route_kernel, its experts resolved by the host, and then run by
// the decode kernel, which routes again and must select the same ids), so the
// arithmetic lives here once.
constexpr int kHV = 4;   // float4 of the hidden state per thread: H <= 8192
constexpr int kRCH = 2;  // 16-byte router chunks per thread: H <= 8192
// 1 / sqrt(mean(x^2) + eps) over the work-group's hidden-state registers.
WL_DEV float norm_rinv(const float4 (&hv)[kHV], float* red, uint32_t H, float eps) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kHV; i++) {
        ss = __fadd_rn(ss, __fmul_rn(hv[i].x, hv[i].x));
        ss = __fadd_rn(ss, __fmul_rn(hv[i].y, hv[i].y));
        ss = __fadd_rn(ss, __fmul_rn(hv[i].z, hv[i].z));
        ss = __fadd_rn(ss, __fmul_rn(hv[i].w, hv[i].w));
    }
    const float tot = block_sum(ss, red);
    return 1.0f / sqrtf(tot / (float)H + eps);
}
// w * (x * rinv) (tools/ref_glm_chain.py:63-80; src/glm_primitives.cuh:35-62)
WL_DEV float norm_value(float x, float rinv, bool has_ln, uint32_t ln_bits) {
    float y = __fmul_rn(x, rinv);
    if (has_ln) y = __fmul_rn(y, bf2f(ln_bits));
    return y;
}
// This thread's share of one router row (bf16 x f32, fp32 accumulate),
// reduced over the wave. x(m, h) returns xn[8c + 4h .. 8c + 4h + 4) for the
// thread's chunk c = threadIdx.x + kThreads * m (from LDS or registers: the
// arithmetic is the same either way).
template <class XF>
WL_DEV float router_chain_x(const u32x4 (&rw)[kRCH], XF x, uint32_t nch) {
    float pd = 0.f;
#pragma unroll
    for (int m = 0; m < kRCH; m++) {
        const uint32_t c = threadIdx.x + kThreads * m;
        if (c < nch) {
            const float4 x0 = x(m, 0), x1 = x(m, 1);
            pd = fmaf(bf2f(rw[m].x & 0xFFFFu), x0.x, pd);
            pd = fmaf(bf2f(rw[m].x >> 16), x0.y, pd);
            pd = fmaf(bf2f(rw[m].y & 0xFFFFu), x0.z, pd);
            pd = fmaf(bf2f(rw[m].y >> 16), x0.w, pd);
            pd = fmaf(bf2f(rw[m].z & 0xFFFFu), x1.x, pd);
            pd = fmaf(bf2f(rw[m].z >> 16), x1.y, pd);
            pd = fmaf(bf2f(rw[m].w & 0xFFFFu), x1.z, pd);
            pd = fmaf(bf2f(rw[m].w >> 16), x1.w, pd);
        }
    }
    return pd;
}
// The wave sum of router_chain_x: the butterfly x += shfl_xor(x, o), o = 32,
// 16, ..., 1 (every lane ends with the same bits: fp32 addition commutes).
template <class XF>
WL_DEV float router_partial_x(const u32x4 (&rw)[kRCH], XF x, uint32_t nch) {
    float pd = router_chain_x(rw, x, nch);
    for (int o = 32; o > 0; o >>= 1) pd += __shfl_xor(pd, o, 64);
    return pd;
}
WL_DEV float router_partial(const u32x4 (&rw)[kRCH], const float* xn, uint32_t nch) {
    return router_partial_x(
        rw, [&](int m, int h) { return *(const float4*)(xn + 8u * (threadIdx.x + kThreads * m) + 4u * h); }, nch);
}
// Sum of the 8 wave partials of router row r (slot 48 of each wave's red
// line), published as one 64-bit word (epoch << 32 | bits) with an
// agent-scope store: a reader that sees this call's epoch has the value.
WL_DEV void router_publish(float pd, float* red, uint64_t* lslot, uint32_t r, uint32_t epoch) {
    if ((threadIdx.x & 63) == 0) red[(threadIdx.x >> 6) * 64 + 48] = pd;
    lds_barrier();
    if (threadIdx.x == 0) {
        float sum = 0.f;
#pragma unroll
        for (int wv = 0; wv < kWaves; wv++) sum += red[wv * 64 + 48];
        __hip_atomic_store((__attribute__((address_space(1))) uint64_t*)(lslot + r),
                           ((uint64_t)epoch << 32) | __float_as_uint(sum), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    lds_barrier();
}

}  // namespace wl
