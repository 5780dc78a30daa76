// moe_decode.hip — gfx950 kernels of the bs=1 MoE decode layer.
//
// One persistent launch of G work-groups (one per CU, 8 wave64s each) runs a
// layer in three segments separated by grid barriers:
//
//   0  every work-group normalises the hidden state (RMSNorm, redundantly),
//      computes one router row (logit) and one 8-gate + 8-up tile of the bf16
//      shared expert, and publishes the logit and the 8 SwiGLU values.
//      reference: rms_norm_bf16, matvec_bf16 (router), shared expert gate/up,
//      src/glm_primitives.cuh:35-62,87-116, src/glm_layer_runner.cuh:370,387,431
//   1  every work-group recomputes the top-k from the published logits
//      (sigmoid, +e_score_correction_bias, top-K with ties to the lowest index,
//      renormalise, x routed_scaling; src/glm_layer_runner.cuh:304-336), then
//      (a) applies 3 (16-row tile, k-half) units of the shared down projection,
//          whose weights it loaded before the barrier, and
//      (b) runs one routed unit (expert slot k, slice j): the 64 SwiGLU rows
//          [64j, 64j+64) of expert k — MXFP4 gate/up, kept in LDS — times
//          the 64 matching columns of its MXFP4 down projection, i.e. a
//          split-K partial of expert k's output over all H rows.
//      reference: dequant_matvec_mxfp4 x3 + silu_mul, src/glm_kernels.cuh:63-110,
//      src/glm_layer_runner.cuh:338-341,424-427
//   2  every work-group combines RB output rows: e_k = sum_j partial(k, j),
//      out = sum_k w_k e_k (slot order) + shared (src/glm_layer_runner.cuh:
//      403,428,436).
//
// Splitting the down projection by the SwiGLU slice a work-group computed
// means no work-group waits for another one's SwiGLU output: the only
// cross-work-group dependencies are the two grid barriers. Work-group w runs
// routed unit u = w, i.e. expert slot w mod 8 at K = 8; work-groups are
// dispatched round-robin over the 8 XCDs, so all 32 slices of one expert run
// on one XCD and the down-projection rows they share (32 bytes each per
// slice, 128-byte lines) are fetched into that XCD's L2 once.
//
// Dot products run on the matrix cores. A 16-row weight tile is the B operand
// of v_mfma_f32_16x16x32_bf16 (lane n%16 holds row n, lane/16 selects 8
// consecutive k values); the A operand carries the activation split into three
// bf16 pieces x = hi + mid + lo (exact for fp32 x), one piece per A row, so
// D[0..2][n] summed is the full-precision dot product of row n. MXFP4 weights
// are widened to bf16 with v_cvt_scalef32_pk_bf16_fp4, which applies the E8M0
// block scale exactly (e2m1 x 2^(s-127) is representable in bf16), low nibble =
// even column as in the reference (src/glm_kernels.cuh:4-33).
//
// Weight loads are 16 bytes per lane (one 1 KB request per wave instruction)
// and are issued in batches of kNB, two batches in flight per wave: a wave
// issues batch b+2 right after it has consumed batch b. Every batch is issued
// unconditionally (indices past the end are clamped to a valid address and
// their contribution masked), so the compiler's wait counts stay exact.
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
WL_DEV uint32_t bld1(rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, (int)voff, (int)soff, 0);
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
WL_DEV void raise_error(uint32_t* sync, const SyncMap& m, uint32_t bits) {
    __hip_atomic_fetch_or((g_u32*)(sync + m.error), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Grid barrier `seq` (a value no earlier barrier of the context used). All
// cross-work-group data is in uncached memory, so completing a work-group's
// stores before its arrival is the whole release, and nothing is needed to
// acquire. Arrival: one counter per group of work-groups (w mod 8, i.e. one
// per XCD) and one counter of complete groups; the work-group that completes
// the last group zeroes the counters and then writes `seq` to every
// work-group's release word, which each work-group polls. Bounded: returns
// false, with E_SPIN raised, if the release does not come, and false if
// another work-group raised an error meanwhile.
WL_DEV bool grid_barrier(uint32_t* sync, const SyncMap& m, uint32_t seq, uint32_t w, uint32_t G,
                         uint32_t* s_flag, bool all_waves_stored) {
    // Only wave 0 wrote cross-work-group data unless all_waves_stored; the
    // other waves then keep whatever loads they have in flight.
    if (all_waves_stored || threadIdx.x < 64) vm_drain();
    lds_barrier();
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x;
        const uint32_t grp = w & 7u;
        const uint32_t members = (G - grp + 7u) / 8u;
        const uint32_t groups = G < 8u ? G : 8u;
        uint32_t old = 0;
        if (lane == 0) old = rmw_inc(sync + m.bar_grp + grp * kLineWords);
        old = __shfl(old, 0, 64);
        if (old == members - 1u) {
            uint32_t old2 = 0;
            if (lane == 0) old2 = rmw_inc(sync + m.bar_all);
            old2 = __shfl(old2, 0, 64);
            if (old2 == groups - 1u) {
                if (lane < 8) st_sync(sync + m.bar_grp + lane * kLineWords, 0u);
                if (lane == 0) st_sync(sync + m.bar_all, 0u);
                vm_drain();
                for (uint32_t f = lane; f < G; f += 64) st_sync(sync + m.bar_rel + f * kLineWords, seq);
            }
        }
        uint32_t ok = 1u;
        for (uint32_t spins = 0;; spins++) {
            uint32_t r = 0, e = 0;
            if (lane == 0) {
                r = ld_sync(sync + m.bar_rel + w * kLineWords);
                if ((spins & 255u) == 255u) e = ld_sync(sync + m.error);
            }
            r = __shfl(r, 0, 64);
            e = __shfl(e, 0, 64);
            if (r == seq) break;
            if (e != 0u) { ok = 0u; break; }
            if (spins > (1u << 22)) {
                if (lane == 0) raise_error(sync, m, E_SPIN);
                ok = 0u;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0) *s_flag = ok;
    }
    lds_barrier();
    const bool ok = *s_flag != 0u;
    lds_barrier();
    return ok;
}

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
struct Batch {
    u32x4 w[kNB];
    uint32_t s[kNB];
};
// Shared-down batch: kSPU k tiles of each of 3 units.
constexpr uint32_t kSPU = 4;
struct SdBatch {
    u32x4 w[3 * kSPU];
};

// Two-deep software pipeline over nb >= 2 batches: A holds batch 0 and B
// batch 1 on entry, both already issued. Batch b+2 is issued right after
// batch b is consumed; no batch is issued that is not consumed.
template <class IssueF, class ConsumeF>
WL_DEV void pingpong(uint32_t nb, Batch& A, Batch& B, IssueF issue, ConsumeF consume) {
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
WL_DEV void topk_rank(uint32_t E, uint32_t K, const float* sc, const float* ch, uint32_t* sidx, float* sw) {
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        const float c = ch[e];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < E; j += 4) {
            const float4 v = *(const float4*)(ch + j);
            rank += (v.x > c || (v.x == c && j + 0 < e)) ? 1u : 0u;
            rank += (v.y > c || (v.y == c && j + 1 < e)) ? 1u : 0u;
            rank += (v.z > c || (v.z == c && j + 2 < e)) ? 1u : 0u;
            rank += (v.w > c || (v.w == c && j + 3 < e)) ? 1u : 0u;
        }
        if (rank < K) {
            sidx[rank] = e;
            sw[rank] = sc[e];
        }
    }
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

// Shared down projection, any shape: units vu = w + G*i, one at a time, k
// tiles spread over the waves, then a cross-wave sum (fixed order) per row.
// Not on the GLM path (kept out of line so it does not add to the decode
// kernel's register pressure).
__device__ __noinline__ void sd_general(const DecodeArgs& a, const Plan& P, const uint16_t* smp, uint32_t sps,
                                        float* red, uint32_t H, uint32_t SI, uint32_t w, uint32_t G) {
    const uint32_t lane = threadIdx.x & 63, v = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
    const uint32_t SIh = SI / P.KS, nkts = SIh / 32;
    for (uint32_t vu = w; vu < P.NSD; vu += G) {
        const uint32_t tr = vu / P.KS, h = vu % P.KS;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t kt = v; kt < nkts; kt += kWaves) {
            const u32x4 b = gld16(a.sh_down + (size_t)(16u * tr + n) * SI + h * SIh + kt * 32u + 8u * g);
            acc = mma(a_lds(smp, sps, n, h * SIh + kt * 32u + 8u * g, true), as_bf16x8(b), acc);
        }
        if (lane < 16) red[v * 64 + n] = sum3(acc);
        lds_barrier();
        if (threadIdx.x < 16) {
            float s = 0.f;
            for (int wv = 0; wv < kWaves; wv++) s += red[wv * 64 + threadIdx.x];
            gst(a.sdpart + (size_t)h * H + 16u * tr + threadIdx.x, s);
        }
        lds_barrier();
    }
}

// ---- the decode kernel -------------------------------------------------------
// GLM = true compiles the GLM shape (H 6144, I 2048, SI 2048, E 256, K 8) with
// every shape constant known; GLM = false reads the shapes from the record.
template <bool GLM>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
moe_decode_kernel(const DecodeArgs* __restrict__ pa, const DecodeDyn d) {
    const DecodeArgs& a = *pa;
    const uint32_t H = GLM ? 6144u : a.H, I = GLM ? 2048u : a.I, SI = GLM ? 2048u : a.SI,
                   E = GLM ? 256u : a.E, K = GLM ? 8u : a.K;
    const uint32_t G = gridDim.x, w = blockIdx.x, tid = threadIdx.x;
    __builtin_assume(tid < (uint32_t)kThreads);
    const uint32_t v = uni(tid >> 6) & 7u, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const Plan P = Plan::make(H, I, SI, K, G);
    const LdsMap L = LdsMap::make(H, SI, E, K, P);
    const SyncMap SM = SyncMap::make();
    extern __shared__ __align__(16) uint8_t lds[];
    uint16_t* xp = (uint16_t*)(lds + L.xp);
    const uint32_t xps = H + 8;
    float* xn = (float*)(lds + L.xn);
    float* fin = xn;
    uint16_t* smp = (uint16_t*)(lds + L.smp);
    const uint32_t sps = SI + 8;
    uint16_t* rmp = (uint16_t*)(lds + L.rmp);
    constexpr uint32_t rps = kSlice + 8;
    float* red = (float*)(lds + L.red);
    float* tk_sc = (float*)(lds + L.topk);
    float* tk_ch = tk_sc + E;
    uint32_t* tk_idx = (uint32_t*)(tk_ch + E);
    float* tk_w = (float*)(tk_idx + 32);
    const uint8_t** tk_blk = (const uint8_t**)(lds + L.slots);
    uint32_t* misc = (uint32_t*)(lds + L.misc);

    Batch bA, bB;
    SdBatch bP;

    // ---- shared down: units vu = w + G*i ((16-row tile, k half) pairs).
    // Fast path (at most 3 units per work-group and SI/KS <= 8*kSPU*32): one
    // batch holds kSPU 32-wide k tiles of each unit for every wave (slot
    // lu*kSPU + i: unit lu, k tile kSPU*v + i). Anything else runs sd_general.
    const uint32_t SIh = SI / P.KS;        // k columns per unit
    const uint32_t nkts = SIh / 32;        // k tiles per unit
    const uint32_t sd_units = w < P.NSD ? cdiv(P.NSD - w, G) : 0u;
    const bool sd_fast = sd_units <= 3u && nkts <= 8u * kSPU;
    const rsrc_t sd_rs = make_rsrc(a.sh_down, H * SI * 2u);
    const uint32_t sd_voff = (n * SI + 8u * g) * 2u;
    uint32_t sd_s[3], sd_a[3];
#pragma unroll
    for (int lu = 0; lu < 3; lu++) {
        const uint32_t vc = min(w + G * lu, P.NSD - 1u);
        const uint32_t tr = vc / P.KS, h = vc % P.KS;
        sd_s[lu] = uni((16u * tr * SI + h * SIh + kSPU * v * 32u) * 2u);
        sd_a[lu] = uni(h * SIh + kSPU * v * 32u);
    }
    auto sd_issue = [&](SdBatch& B) {
#pragma unroll
        for (int lu = 0; lu < 3; lu++) {
#pragma unroll
            for (int i = 0; i < (int)kSPU; i++) B.w[lu * kSPU + i] = bld16(sd_rs, sd_voff + i * 64u, sd_s[lu]);
        }
    };
    auto sd_consume_store = [&](const SdBatch& B) {
        f32x4 sacc[3];
#pragma unroll
        for (int lu = 0; lu < 3; lu++) {
            sacc[lu] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < (int)kSPU; i++) {
                const bool valid = (uint32_t)lu < sd_units && kSPU * v + i < nkts;
                const u32x4 z = {0u, 0u, 0u, 0u};
                sacc[lu] = mma(a_lds(smp, sps, n, sd_a[lu] + i * 32u + 8u * g, valid),
                               as_bf16x8(valid ? B.w[lu * kSPU + i] : z), sacc[lu]);
            }
        }
        if (lane < 16) {
#pragma unroll
            for (int lu = 0; lu < 3; lu++) red[v * 64 + lu * 16 + n] = sum3(sacc[lu]);
        }
        lds_barrier();
        if (tid < 48) {
            const uint32_t lu = tid / 16, row = tid % 16;
            const uint32_t vu = w + G * lu;
            if (lu < sd_units) {
                float s = 0.f;
#pragma unroll
                for (int wv = 0; wv < kWaves; wv++) s += red[wv * 64 + tid];
                const uint32_t tr = vu / P.KS, h = vu % P.KS;
                gst(a.sdpart + (size_t)h * H + 16u * tr + row, s);
            }
        }
        lds_barrier();
    };

    // ================= segment 0: norm, router row, shared gate/up ==============
    if (d.seg_lo == 0u) {
        // hidden state and norm weight first: they are consumed first
        constexpr int HV = 4;  // float4 per thread: H <= 8192
        float4 hv[HV];
        uint2 lv[HV];
        const rsrc_t hid_rs = make_rsrc(d.hidden, H * 4u);
        const rsrc_t ln_rs = make_rsrc(a.ln_w ? (const void*)a.ln_w : (const void*)d.hidden, H * 2u);
#pragma unroll
        for (int i = 0; i < HV; i++) {
            const uint32_t j = tid + kThreads * i;  // float4 j = elements [4j, 4j+4)
            hv[i] = __builtin_bit_cast(float4, bld16(hid_rs, 16u * j, 0u));
            lv[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ln_rs, (int)(8u * j), 0, 0));
        }
        // the first router row of this work-group
        constexpr int RCH = 2;  // 16-byte chunks per thread: H <= 8192
        const uint32_t nch = H / 8;
        const uint32_t r0 = min(w, E - 1u);
        const rsrc_t rt_rs = make_rsrc(a.router_w, E * H * 2u);
        u32x4 rw[RCH];
#pragma unroll
        for (int m = 0; m < RCH; m++) rw[m] = bld16(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), r0 * H * 2u);
        // shared gate/up: tiles t = w + G*i of SI/8; items are 32-wide k tiles
        const uint32_t nsg = SI / 8, nkt = H / 32;
        const uint32_t sg_per = cdiv(nkt, 8u);  // k tiles per wave: [v*sg_per, +sg_per)
        const uint32_t sg_nb = at_least2(cdiv(sg_per, (uint32_t)kNB));
        // gate and up are adjacent in the shared block: one resource covers both
        const rsrc_t sg_rs = make_rsrc(a.sh_gate, 2u * SI * H * 2u);
        auto sg_issue = [&](uint32_t tile, uint32_t b, Batch& B) {
            const uint32_t row = min(tile, nsg - 1u) * 8u + (n & 7u);
            const uint32_t voff = ((n < 8 ? 0u : SI * H) + row * H + 8u * g) * 2u;
            const uint32_t kt0 = v * sg_per + b * kNB;
#pragma unroll
            for (int i = 0; i < kNB; i++) B.w[i] = bld16(sg_rs, voff + i * 64u, kt0 * 64u);
        };
        f32x4 gacc;
        auto sg_consume = [&](uint32_t b, const Batch& B) {
#pragma unroll
            for (int i = 0; i < kNB; i++) {
                const uint32_t m = b * kNB + i, kt = v * sg_per + m;
                const bool valid = m < sg_per && kt < nkt;
                const u32x4 z = {0u, 0u, 0u, 0u};
                gacc = mma(a_lds(xp, xps, n, kt * 32u + 8u * g, valid), as_bf16x8(valid ? B.w[i] : z), gacc);
            }
        };
        sg_issue(w, 0, bA);
        sg_issue(w, 1, bB);

        // RMSNorm: w * (x * (1/sqrt(mean(x^2) + eps))) in fp32
        // (tools/ref_glm_chain.py:63-80; src/glm_primitives.cuh:35-62)
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < HV; i++) {
            ss = __fadd_rn(ss, __fmul_rn(hv[i].x, hv[i].x));
            ss = __fadd_rn(ss, __fmul_rn(hv[i].y, hv[i].y));
            ss = __fadd_rn(ss, __fmul_rn(hv[i].z, hv[i].z));
            ss = __fadd_rn(ss, __fmul_rn(hv[i].w, hv[i].w));
        }
        const float tot = block_sum(ss, red);
        const float rinv = 1.0f / sqrtf(tot / (float)H + a.eps);
#pragma unroll
        for (int i = 0; i < HV; i++) {
            const uint32_t j = tid + kThreads * i;
            if (j < H / 4) {
                const float xs[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
                const uint32_t ls[4] = {lv[i].x & 0xFFFFu, lv[i].x >> 16, lv[i].y & 0xFFFFu, lv[i].y >> 16};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    float x = __fmul_rn(xs[c], rinv);
                    if (a.ln_w) x = __fmul_rn(x, bf2f(ls[c]));
                    const uint32_t col = 4 * j + c;
                    xn[col] = x;
                    uint32_t ph, pm, pl;
                    split3(x, ph, pm, pl);
                    xp[col] = (uint16_t)ph;
                    xp[xps + col] = (uint16_t)pm;
                    xp[2 * xps + col] = (uint16_t)pl;
                    if (w == 0) gst(a.norm + col, x);
                }
            }
        }
        lds_barrier();

        // router rows r = w + G*i (bf16 x f32, fp32 accumulate)
        for (uint32_t r = w, first = 1; r < E; r += G, first = 0) {
            if (!first) {
#pragma unroll
                for (int m = 0; m < RCH; m++) rw[m] = bld16(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), r * H * 2u);
            }
            float pd = 0.f;
#pragma unroll
            for (int m = 0; m < RCH; m++) {
                const uint32_t c = tid + kThreads * m;
                if (c < nch) {
                    const float4 x0 = *(const float4*)(xn + 8 * c);
                    const float4 x1 = *(const float4*)(xn + 8 * c + 4);
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
            for (int o = 32; o > 0; o >>= 1) pd += __shfl_xor(pd, o, 64);
            if (lane == 0) red[v * 64 + 48] = pd;
            lds_barrier();
            if (tid == 0) {
                float s = 0.f;
#pragma unroll
                for (int wv = 0; wv < kWaves; wv++) s += red[wv * 64 + 48];
                gst(a.logits + r, s);
            }
            lds_barrier();
        }

        // shared gate/up tiles, SwiGLU of 8 rows each
        for (uint32_t tile = w; tile < nsg; tile += G) {
            if (tile != w) {
                sg_issue(tile, 0, bA);
                sg_issue(tile, 1, bB);
            }
            gacc = f32x4{0.f, 0.f, 0.f, 0.f};
            pingpong(sg_nb, bA, bB, [&](uint32_t b, Batch& B) { sg_issue(tile, b, B); }, sg_consume);
            if (lane < 16) red[v * 64 + n] = sum3(gacc);
            lds_barrier();
            if (tid < 8) {
                float gs = 0.f, us = 0.f;
#pragma unroll
                for (int wv = 0; wv < kWaves; wv++) {
                    gs += red[wv * 64 + tid];
                    us += red[wv * 64 + 8 + tid];
                }
                const float mid = silu_mul(gs, us);
                const uint32_t r = tile * 8 + tid;
                gst(a.smid + r, mid);
                uint32_t ph, pm, pl;
                split3(mid, ph, pm, pl);
                gst(a.smid_p + r, (uint16_t)ph);
                gst(a.smid_p + SI + r, (uint16_t)pm);
                gst(a.smid_p + 2 * SI + r, (uint16_t)pl);
            }
            lds_barrier();
        }

        if (d.seg_hi >= 1u) {
            if (!grid_barrier(a.sync, SM, 2u * d.epoch, w, G, misc, false)) return;
        }
    }

    // ================= segment 1: top-k, shared down, routed units ==============
    if (d.seg_lo <= 1u && d.seg_hi >= 1u) {
        // The top-k inputs, the slot table and the shared SwiGLU pieces are
        // loaded first and the first shared-down batch right after them, so
        // those weights stream while the top-k is computed.
        constexpr int TKV = 2, SMV = 2;  // per thread: E <= 1024, 3*SI/8 <= 1024 in registers
        const rsrc_t lg_rs = make_rsrc(a.logits, E * 4u), bs_rs = make_rsrc(a.bias, E * 4u);
        const rsrc_t sl_rs = make_rsrc(a.slot_tab, E * 8u), sm_rs = make_rsrc(a.smid_p, 3u * SI * 2u);
        uint32_t lgv[TKV], bsv[TKV];
        uint64_t slv[TKV];
        u32x4 smv[SMV];
#pragma unroll
        for (int i = 0; i < TKV; i++) {
            const uint32_t e = tid + kThreads * i;
            lgv[i] = __builtin_amdgcn_raw_buffer_load_b32(lg_rs, (int)(4u * e), 0, 0);
            bsv[i] = __builtin_amdgcn_raw_buffer_load_b32(bs_rs, (int)(4u * e), 0, 0);
            slv[i] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(sl_rs, (int)(8u * e), 0, 0));
        }
#pragma unroll
        for (int i = 0; i < SMV; i++) smv[i] = bld16(sm_rs, 16u * (tid + kThreads * i), 0u);
        if (sd_fast && sd_units) sd_issue(bP);
#pragma unroll
        for (int i = 0; i < TKV; i++) {
            const uint32_t e = tid + kThreads * i;
            if (e < E) topk_score(__uint_as_float(lgv[i]), __uint_as_float(bsv[i]), e, tk_sc, tk_ch);
            if (e < E) tk_blk[e] = (const uint8_t*)slv[i];
        }
        for (uint32_t e = tid + kThreads * TKV; e < E; e += kThreads) {
            topk_score(gld(a.logits + e), gld(a.bias + e), e, tk_sc, tk_ch);
            tk_blk[e] = gld(a.slot_tab + e);
        }
#pragma unroll
        for (int i = 0; i < SMV; i++) {
            const uint32_t c = tid + kThreads * i;
            if (c < 3u * SI / 8u) *(u32x4*)(smp + (c / (SI / 8u)) * sps + (c % (SI / 8u)) * 8u) = smv[i];
        }
        for (uint32_t c = tid + kThreads * SMV; c < 3u * SI / 8u; c += kThreads)
            *(u32x4*)(smp + (c / (SI / 8u)) * sps + (c % (SI / 8u)) * 8u) = gld16(a.smid_p + 8u * c);
        lds_barrier();
        topk_rank(E, K, tk_sc, tk_ch, tk_idx, tk_w);
        if (w == 0 && tid < K) {
            gst(a.idx + tid, (int32_t)tk_idx[tid]);
            gst(a.topw + tid, topk_weight(a, K, tk_w, tid));
        }

        // routed units u = w + G*i: items are gate/up k tiles (128 wide, this
        // wave's 8+8 row tile), then down row pairs (32 rows x the slice's 64
        // columns), each wave a contiguous range of them
        const uint32_t nkg = H / 128, nq = H / 32;
        const uint32_t dq_per = cdiv(nq, 8u);  // down row pairs per wave: [v*dq_per, +dq_per)
        const uint32_t nbg = cdiv(nkg, (uint32_t)kNB);
        const uint32_t nbd = cdiv(dq_per, (uint32_t)kNB);
        const uint32_t nbr = nbg + nbd;  // >= 2
        const uint8_t* blk = nullptr;
        uint32_t uk = 0, uj = 0, uu = 0;
        rsrc_t r_rs = make_rsrc(a.router_w, 16u);  // rebound per unit
        uint32_t gu_voff = 0, gu_soff = 0, dn_voff = 0, dn_soff = 0;
        // Branch-free: per-slot offsets are selected, then one block of loads
        // (loads on two paths would be joined by register copies that wait
        // for them).
        auto r_issue = [&](uint32_t b, Batch& B) {
            const bool gu = b < nbg;
            const uint32_t kt0 = b * kNB;
            const uint32_t q0 = v * dq_per + (b - nbg) * kNB;
#pragma unroll
            for (int i = 0; i < kNB; i++) {
                const uint32_t wv = gu ? gu_voff + i * 64u : dn_voff;
                const uint32_t ws = gu ? kt0 * 64u : (q0 + i) * 32u * (I / 2);
                const uint32_t sv = gu ? gu_soff + i * 4u : dn_soff;
                const uint32_t ss = gu ? kt0 * 4u : (q0 + i) * 32u * (I / 32);
                B.w[i] = bld16(r_rs, wv, ws);
                B.s[i] = bld1(r_rs, sv, ss);
            }
        };
        f32x4 racc;
        bf16x8 A0, A1;
        auto r_consume = [&](uint32_t b, const Batch& B) {
            if (b < nbg) {
#pragma unroll
                for (int i = 0; i < kNB; i++) {
                    const uint32_t kt = b * kNB + i;
                    const bool valid = kt < nkg;
                    // a masked item reads the next row (or zeros past the
                    // block): scale 0 makes its B operand exactly zero
                    const float sc = valid ? e8m0f(B.s[i]) : 0.f;
#pragma unroll
                    for (int jj = 0; jj < 4; jj++)
                        racc = mma(a_lds(xp, xps, n, kt * 128u + 32u * g + 8u * jj, valid),
                                   fp4x8_bf16(B.w[i][jj], sc), racc);
                }
                if (b == nbg - 1u) {
                    // SwiGLU of this wave's 8 rows: lane r < 8 holds gate row r,
                    // lane r + 8 the matching up row
                    const float val = sum3(racc);
                    const float up = __shfl(val, (lane + 8u) & 63u, 64);
                    if (lane < 8) {
                        const float mid = silu_mul(val, up);
                        const uint32_t col = v * 8u + lane;
                        gst(a.rmid + (size_t)uk * I + uj * kSlice + col, mid);
                        uint32_t ph, pm, pl;
                        split3(mid, ph, pm, pl);
                        rmp[col] = (uint16_t)ph;
                        rmp[rps + col] = (uint16_t)pm;
                        rmp[2 * rps + col] = (uint16_t)pl;
                    }
                    lds_barrier();
                    // down A operands: k groups of lane g hold slice columns
                    // {0,32,8,40}[g] (+16 for the second), matching the
                    // lane order the row-pair swap below produces
                    const uint32_t c0 = 32u * (g & 1u) + 8u * (g >> 1);
                    A0 = a_lds(rmp, rps, n, c0, true);
                    A1 = a_lds(rmp, rps, n, c0 + 16u, true);
                }
            } else {
                const uint32_t m0 = (b - nbg) * kNB;
#pragma unroll
                for (int i = 0; i < kNB; i++) {
                    // lane (n, g) holds 16 bytes of row n + 16*(g>>1): columns
                    // [32*(g&1), +32) of the slice, and that block's scale.
                    // One swap of lane halves turns dwords (0,1) into the B
                    // operand of rows n (lanes 0-31 keep theirs, lanes 32-63
                    // take the lower half's dword 1) and of rows n + 16.
                    const uint32_t m = m0 + i, q = v * dq_per + m;
                    const bool valid = m < dq_per && q < nq;
                    uint32_t sx, sy, x01, y01, x23, y23;
                    swap32(B.s[i], B.s[i], sx, sy);
                    swap32(B.w[i][0], B.w[i][1], x01, y01);
                    swap32(B.w[i][2], B.w[i][3], x23, y23);
                    const float scx = e8m0f(sx), scy = e8m0f(sy);
                    f32x4 d0 = mma(A0, fp4x8_bf16(x01, scx), f32x4{0.f, 0.f, 0.f, 0.f});
                    d0 = mma(A1, fp4x8_bf16(x23, scx), d0);
                    f32x4 d1 = mma(A0, fp4x8_bf16(y01, scy), f32x4{0.f, 0.f, 0.f, 0.f});
                    d1 = mma(A1, fp4x8_bf16(y23, scy), d1);
                    const float s0 = sum3(d0);
                    const float s1 = __shfl(sum3(d1), (lane - 16u) & 63u, 64);
                    if (valid && lane < 32) gst(a.part + (size_t)uu * H + q * 32u + lane, lane < 16 ? s0 : s1);
                }
            }
        };

        bool first_unit = true;
        for (uint32_t u = w; u < P.U; u += G) {
            uu = u;
            uk = u % K;
            uj = u / K;
            blk = uni_ptr(tk_blk[tk_idx[uk]]);
            if (blk == nullptr) {
                if (tid == 0) raise_error(a.sync, SM, E_NOT_RESIDENT);
                continue;
            }
            if (!first_unit) lds_barrier();  // rmp of the previous unit fully read
            {
                const uint32_t row = uj * kSlice + v * 8u + (n & 7u);
                const uint32_t drow = n + 16u * (g >> 1);
                // packed block: gate_w | gate_s | up_w | up_s | down_w | down_s
                // (reference ExpertLayout, src/glm_layer_runner.cuh:60-72)
                const uint32_t gw = 0, gs = gw + I * H / 2, uw = gs + I * H / 32, us = uw + I * H / 2;
                const uint32_t dw = us + I * H / 32, ds = dw + H * I / 2, total = ds + H * I / 32;
                r_rs = make_rsrc(blk, total);
                gu_voff = (n < 8 ? gw : uw) + row * (H / 2) + 16u * g;
                gu_soff = (n < 8 ? gs : us) + row * (H / 32) + g;
                dn_voff = dw + drow * (I / 2) + 32u * uj + 16u * (g & 1u);
                dn_soff = ds + drow * (I / 32) + 2u * uj + (g & 1u);
            }
            r_issue(0, bA);
            if (first_unit) {
                // shared down (its batch is in bP) while batch 0 flies
                if (sd_fast && sd_units) sd_consume_store(bP);
                first_unit = false;
            }
            r_issue(1, bB);
            racc = f32x4{0.f, 0.f, 0.f, 0.f};
            pingpong(nbr, bA, bB, r_issue, r_consume);
        }
        if (first_unit && sd_fast && sd_units) sd_consume_store(bP);  // no routed unit here
        if (!sd_fast) sd_general(a, P, smp, sps, red, H, SI, w, G);

        if (d.seg_hi >= 2u) {
            if (!grid_barrier(a.sync, SM, 2u * d.epoch + 1u, w, G, misc, true)) return;
        }
    }

    // ================= segment 2: combine ========================================
    if (d.seg_hi >= 2u) {
        if (d.seg_lo == 2u) {
            for (uint32_t e = tid; e < E; e += kThreads) topk_score(gld(a.logits + e), gld(a.bias + e), e, tk_sc, tk_ch);
            lds_barrier();
            topk_rank(E, K, tk_sc, tk_ch, tk_idx, tk_w);
        }
        const uint32_t RB = P.RB, r0 = w * RB;
        if (r0 >= H) return;
        const uint32_t nr = min(RB, H - r0);
        float* fsd = fin + P.U * RB;
        float* fe = fsd + P.KS * RB;
        for (uint32_t i = tid; i < P.U * RB; i += kThreads) {
            const uint32_t u = i / RB, rr = i % RB;
            fin[i] = rr < nr ? gld(a.part + (size_t)u * H + r0 + rr) : 0.f;
        }
        for (uint32_t i = tid; i < P.KS * RB; i += kThreads) {
            const uint32_t h = i / RB, rr = i % RB;
            fsd[i] = rr < nr ? gld(a.sdpart + (size_t)h * H + r0 + rr) : 0.f;
        }
        lds_barrier();
        for (uint32_t i = tid; i < K * RB; i += kThreads) {
            const uint32_t k = i / RB, rr = i % RB;
            float e = 0.f;
            for (uint32_t j = 0; j < P.S; j++) e += fin[(j * K + k) * RB + rr];
            fe[i] = e;
            if (rr < nr) gst(a.edown + (size_t)k * H + r0 + rr, e);
        }
        lds_barrier();
        for (uint32_t rr = tid; rr < nr; rr += kThreads) {
            float sh = 0.f;
            for (uint32_t h = 0; h < P.KS; h++) sh += fsd[h * RB + rr];
            float o = 0.f;
            for (uint32_t k = 0; k < K; k++) o = __fadd_rn(o, __fmul_rn(topk_weight(a, K, tk_w, k), fe[k * RB + rr]));
            o = __fadd_rn(o, sh);
            const uint32_t r = r0 + rr;
            gst(a.shared_out + r, sh);
            gst(d.out + r, d.resid ? __fadd_rn(gld(d.resid + r), o) : o);
        }
    }
}

// ---- standalone kernels: one MXFP4 matvec, one MXFP4 expert FFN -------------
// x (fp32) split into bf16 pieces in LDS by the whole work-group.
WL_DEV void pieces_to_lds(const float* x, uint32_t K, uint16_t* xp, uint32_t xps) {
    for (uint32_t i = threadIdx.x; i < K; i += kThreads) {
        uint32_t h, m, l;
        split3(x[i], h, m, l);
        xp[i] = (uint16_t)h;
        xp[xps + i] = (uint16_t)m;
        xp[2 * xps + i] = (uint16_t)l;
    }
    __syncthreads();
}

// Routed gate/up rows [0,16) of one MXFP4 expert (pointers at the tile's first
// row), full K = H, against the LDS norm pieces. Leaves red[wave][0..15] = gate,
// red[wave][16..31] = up.
template <int MAXT>
WL_DEV void fp4_gu_tile(const uint8_t* gw, const uint8_t* gs, const uint8_t* uw, const uint8_t* us, uint32_t H,
                        const uint16_t* xp, uint32_t xps, float* red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t rb = H / 2, rs = H / 32, nkt = H / 128;
    f32x4 dg = {0.f, 0.f, 0.f, 0.f}, du = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t base = 0; base < nkt; base += kWaves * MAXT) {
        u32x4 wg[MAXT], wu[MAXT];
        uint32_t sg[MAXT], su[MAXT];
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const uint32_t kt = min(base + wave + kWaves * i, nkt - 1);
            wg[i] = gld16(gw + (size_t)n * rb + kt * 64 + g * 16);
            wu[i] = gld16(uw + (size_t)n * rb + kt * 64 + g * 16);
            sg[i] = gld1(gs + (size_t)n * rs + kt * 4 + g);
            su[i] = gld1(us + (size_t)n * rs + kt * 4 + g);
        }
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const uint32_t ktr = base + wave + kWaves * i;
            const uint32_t kt = min(ktr, nkt - 1);
            const float scg = e8m0f(sg[i]), scu = e8m0f(su[i]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bf16x8 av = a_lds(xp, xps, n, kt * 128 + g * 32 + j * 8, ktr < nkt);
                dg = mma(av, fp4x8_bf16(wg[i][j], scg), dg);
                du = mma(av, fp4x8_bf16(wu[i][j], scu), du);
            }
        }
    }
    if (lane < 16) {
        red[wave * 64 + lane] = sum3(dg);
        red[wave * 64 + 16 + lane] = sum3(du);
    }
    __syncthreads();
}

// Routed down: RT row tiles (16 rows each, pointers at the block's first row)
// of one MXFP4 expert over K = I, against that expert's SwiGLU pieces ap
// [3][aps] (global or LDS). red[wave][t*16 + row].
template <int RT, int MAXT>
WL_DEV void fp4_down_block(const uint8_t* dw, const uint8_t* ds, uint32_t I, const uint16_t* ap, uint32_t aps,
                           float* red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t rb = I / 2, rs = I / 32, nkt = I / 128;
    f32x4 d[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) d[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t base = 0; base < nkt; base += kWaves * MAXT) {
        u32x4 wv[RT][MAXT];
        uint32_t sv[RT][MAXT];
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const uint32_t kt = min(base + wave + kWaves * i, nkt - 1);
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const size_t row = (size_t)t * 16 + n;
                wv[t][i] = gld16(dw + row * rb + kt * 64 + g * 16);
                sv[t][i] = gld1(ds + row * rs + kt * 4 + g);
            }
        }
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const uint32_t ktr = base + wave + kWaves * i;
            const uint32_t kt = min(ktr, nkt - 1);
            bf16x8 av[4];
#pragma unroll
            for (int j = 0; j < 4; j++) av[j] = a_any(ap, aps, n, kt * 128 + g * 32 + j * 8, ktr < nkt);
#pragma unroll
            for (int t = 0; t < RT; t++) {
                const float sc = e8m0f(sv[t][i]);
#pragma unroll
                for (int j = 0; j < 4; j++) d[t] = mma(av[j], fp4x8_bf16(wv[t][i][j], sc), d[t]);
            }
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int t = 0; t < RT; t++) red[wave * 64 + t * 16 + lane] = sum3(d[t]);
    }
    __syncthreads();
}

// Sum of red[0..kWaves)[col] in wave order.
WL_DEV float wave_total(const float* red, uint32_t col) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) s += red[w * 64 + col];
    return s;
}

constexpr uint32_t kDownRT = 4;  // row tiles per work-group of the standalone down kernel

// y[r] = sum_c e2m1(W[r,c]) * 2^(S[r,c/32]-127) * x[c]; one work-group per 16
// rows. Drop-in for launch_dequant_matvec_mxfp4 (src/glm_kernels.cuh:104-110).
__global__ void __launch_bounds__(kThreads)
dequant_matvec_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ S, const float* __restrict__ x,
                      float* __restrict__ y, uint32_t N, uint32_t K) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    uint16_t* xp = (uint16_t*)lds_raw;
    const uint32_t xps = K + 8;
    float* red = (float*)(lds_raw + (size_t)3 * xps * 2);
    pieces_to_lds(x, K, xp, xps);
    const size_t r0 = (size_t)blockIdx.x * 16;
    fp4_down_block<1, 1>(W + r0 * (K / 2), S + r0 * (K / 32), K, xp, xps, red);
    if (threadIdx.x < 16 && r0 + threadIdx.x < N) y[r0 + threadIdx.x] = wave_total(red, threadIdx.x);
}

// One expert, gate/up + SwiGLU: mid[r] for rows [16*blockIdx.x, +16).
__global__ void __launch_bounds__(kThreads)
ffn_gu_kernel(const uint8_t* __restrict__ blk, uint64_t gw_off, uint64_t gs_off, uint64_t uw_off, uint64_t us_off,
              const float* __restrict__ x, uint32_t H, uint32_t I, float* __restrict__ mid,
              uint16_t* __restrict__ mid_p) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    uint16_t* xp = (uint16_t*)lds_raw;
    const uint32_t xps = H + 8;
    float* red = (float*)(lds_raw + (size_t)3 * xps * 2);
    pieces_to_lds(x, H, xp, xps);
    const size_t r0 = (size_t)blockIdx.x * 16;
    fp4_gu_tile<3>(blk + gw_off + r0 * (H / 2), blk + gs_off + r0 * (H / 32), blk + uw_off + r0 * (H / 2),
                   blk + us_off + r0 * (H / 32), H, xp, xps, red);
    if (threadIdx.x < 16) {
        const float m = silu_mul(wave_total(red, threadIdx.x), wave_total(red, 16 + threadIdx.x));
        const size_t r = r0 + threadIdx.x;
        mid[r] = m;
        uint32_t h, mm, l;
        split3(m, h, mm, l);
        mid_p[r] = (uint16_t)h;
        mid_p[I + r] = (uint16_t)mm;
        mid_p[2 * I + r] = (uint16_t)l;
    }
}

// One expert, down: y[r] for rows [64*blockIdx.x, +64), optional bf16 copy.
__global__ void __launch_bounds__(kThreads)
ffn_down_kernel(const uint8_t* __restrict__ blk, uint64_t dw_off, uint64_t ds_off, const uint16_t* __restrict__ mid_p,
                uint32_t H, uint32_t I, float* __restrict__ y, uint16_t* __restrict__ y_bf16) {
    __shared__ float red[kWaves * 64];
    const size_t r0 = (size_t)blockIdx.x * 16 * kDownRT;
    fp4_down_block<kDownRT, 1>(blk + dw_off + r0 * (I / 2), blk + ds_off + r0 * (I / 32), I, mid_p, I, red);
    if (threadIdx.x < 16 * kDownRT) {
        const float v = wave_total(red, threadIdx.x);
        y[r0 + threadIdx.x] = v;
        if (y_bf16) y_bf16[r0 + threadIdx.x] = (uint16_t)f2bf(v);
    }
}

int launch_dequant_matvec(const uint8_t* W, const uint8_t* S, const float* x, float* y, uint32_t N, uint32_t K,
                          void* stream) {
    const size_t lds = (size_t)3 * (K + 8) * 2 + kWaves * 64 * 4;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)dequant_matvec_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(dequant_matvec_kernel, dim3(N / 16), dim3(kThreads), lds, (hipStream_t)stream, W, S, x, y,
                       N, K);
    return (int)hipGetLastError();
}

int launch_expert_ffn(const uint8_t* blk, uint64_t gw_off, uint64_t gs_off, uint64_t uw_off, uint64_t us_off,
                      uint64_t dw_off, uint64_t ds_off, const float* x, uint32_t H, uint32_t I, float* mid,
                      uint16_t* mid_p, float* y, uint16_t* y_bf16, void* stream) {
    const size_t lds = (size_t)3 * (H + 8) * 2 + kWaves * 64 * 4;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)ffn_gu_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(ffn_gu_kernel, dim3(I / 16), dim3(kThreads), lds, (hipStream_t)stream, blk, gw_off, gs_off,
                       uw_off, us_off, x, H, I, mid, mid_p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(ffn_down_kernel, dim3(H / (16 * kDownRT)), dim3(kThreads), 0, (hipStream_t)stream, blk,
                       dw_off, ds_off, mid_p, H, I, y, y_bf16);
    return (int)hipGetLastError();
}

static bool glm_shape(uint32_t H, uint32_t I, uint32_t SI, uint32_t E, uint32_t K) {
    return H == 6144 && I == 2048 && SI == 2048 && E == 256 && K == 8;
}

int decode_max_lds() { return 160 * 1024; }

int launch_decode(const DecodeArgs* d_args, const DecodeDyn& dyn, uint32_t H, uint32_t I, uint32_t SI, uint32_t E,
                  uint32_t K, uint32_t grid, void* stream) {
    const Plan p = Plan::make(H, I, SI, K, grid);
    const size_t lds = LdsMap::make(H, SI, E, K, p).bytes;
    const void* fn = glm_shape(H, I, SI, E, K) ? (const void*)moe_decode_kernel<true>
                                               : (const void*)moe_decode_kernel<false>;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    if (glm_shape(H, I, SI, E, K))
        hipLaunchKernelGGL(moe_decode_kernel<true>, dim3(grid), dim3(kThreads), lds, (hipStream_t)stream, d_args,
                           dyn);
    else
        hipLaunchKernelGGL(moe_decode_kernel<false>, dim3(grid), dim3(kThreads), lds, (hipStream_t)stream, d_args,
                           dyn);
    return (int)hipGetLastError();
}

}  // namespace wl
