// moe_decode.hip — gfx950 kernels of the bs=1 MoE decode layer.
//
// One layer is a fixed set of tasks, numbered in dependency order:
//
//   router   (E/16 row tiles x 4 k-quarters)   bf16 GEMV partial sums; the 4th
//            arrival of a tile writes its 16 logits; the last tile to finish runs
//            sigmoid / +bias / top-k / renorm / x scaling and publishes the ids,
//            weights and slot-table block pointers.
//            reference: matvec_bf16 + router_sigmoid_topk,
//            src/glm_primitives.cuh:87-116, src/glm_layer_runner.cuh:304-336,387-389
//   sgu      (SI/16 row tiles x 4 k-quarters)  shared-expert gate/up partials; the 4th
//            arrival applies SwiGLU. Independent of routing, so it fills the
//            machine while the router finishes.
//   rgu      (K experts x I/16 row tiles)      routed MXFP4 gate/up + SwiGLU.
//            reference: dequant_matvec_mxfp4 x2 + silu_mul, src/glm_kernels.cuh:63-110,
//            src/glm_layer_runner.cuh:338-341,424-426
//   sdown    (H/16 row tiles)                  shared-expert down projection (bf16).
//   rdown    (K experts x H/64 row blocks)     routed MXFP4 down projection; the K-th
//            arrival of a row block forms out = sum_k w_k e_k + shared in slot order.
//            reference: dequant_matvec_mxfp4 + axpy, src/glm_layer_runner.cuh:343-346,
//            427-436
//
// Work-groups (8 wave64s) claim tasks from a device-wide counter; a task only
// waits on tasks with smaller indices, and tasks are claimed in index order, so
// the lowest unfinished task can always run: the schedule cannot deadlock
// whatever the number of resident work-groups. Every wait is bounded and, on
// expiry, raises E_SPIN and lets the launch drain.
//
// Dot products run on the matrix cores. A 16-row weight tile is the B operand
// of v_mfma_f32_16x16x32_bf16 (lane n%16 holds row n, lane/16 selects a 16-byte
// slice of the row); the A operand carries the activation split into three
// bf16 pieces x = hi + mid + lo (exact for fp32 x), one piece per A row, so
// D[0..2][n] summed is the full-precision dot product of row n. MXFP4 weights
// are widened to bf16 with v_cvt_scalef32_pk_bf16_fp4, which applies the E8M0
// block scale exactly (e2m1 x 2^(s-127) is representable in bf16), low nibble =
// even column as in the reference (src/glm_kernels.cuh:4-33).
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
typedef __attribute__((address_space(3))) const u32x4 l_u32x4;
// 16-byte and 1-byte loads from global memory (never through the flat path).
WL_DEV u32x4 gld16(const void* p) { return *(g_u32x4*)p; }
WL_DEV uint32_t gld1(const uint8_t* p) { return *(g_u8*)p; }
// A operand: piece row r (< 3) of a [3][stride] bf16 array, 8 values at col;
// zero for the other rows and for k tiles past the end (valid == false).
WL_DEV bf16x8 a_lds(const uint16_t* base, uint32_t stride, uint32_t r, uint32_t col, bool valid) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < 3u && valid) v = *(const u32x4*)(base + r * stride + col);
    return as_bf16x8(v);
}
WL_DEV bf16x8 a_glb(const uint16_t* base, uint32_t stride, uint32_t r, uint32_t col, bool valid) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r < 3u && valid) v = gld16(base + r * stride + col);
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

// ---- device-wide synchronisation -----------------------------------------
// All words touched here are in uncached memory (see SyncMap). A barrier
// (which waits for every wave's outstanding stores) orders a work-group's
// results before the single store or RMW that announces them.
WL_DEV uint32_t ld_sync(uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
WL_DEV void st_sync(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Arrival: returns the counter value before this work-group's increment.
WL_DEV uint32_t arrive(uint32_t* c, uint32_t* s_bcast) {
    __syncthreads();
    if (threadIdx.x == 0) *s_bcast = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const uint32_t v = *s_bcast;
    __syncthreads();
    return v;
}
// Completion flag: set to this call's epoch once the work-group's stores are done.
WL_DEV void signal(uint32_t* flag, uint32_t epoch) {
    __syncthreads();
    if (threadIdx.x == 0) st_sync(flag, epoch);
}
// Invalidate the caches this work-group reads through (cheap on gfx950), so
// data read after a wait cannot come from a stale line.
WL_DEV void acquire_all() {
    if (threadIdx.x < 64) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __syncthreads();
}
WL_DEV void raise_error(uint32_t* sync, const SyncMap& m, uint32_t bits) {
    __hip_atomic_fetch_or(sync + m.error, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded wait until flags[0..n) all equal `epoch` (wave 0 polls, one flag per
// lane). Returns false, with E_SPIN raised, if the bound expires or another
// work-group already raised an error.
WL_DEV bool wait_flags(uint32_t* sync, const SyncMap& m, uint32_t first, uint32_t n, uint32_t epoch,
                       uint32_t* s_bcast) {
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x;
        uint32_t ok = 1u;
        for (uint32_t spins = 0;; spins++) {
            bool mine = true;
            for (uint32_t f = lane; f < n; f += 64) mine = mine && (ld_sync(sync + first + f) == epoch);
            if (__all(mine)) break;
            if (ld_sync(sync + m.error) != 0u || spins > (1u << 20)) {
                if (lane == 0 && spins > (1u << 20)) raise_error(sync, m, E_SPIN);
                ok = 0u;
                break;
            }
            __builtin_amdgcn_s_sleep(4);
        }
        if (lane == 0) *s_bcast = ok;
    }
    acquire_all();
    const bool ok = *s_bcast != 0u;
    __syncthreads();
    return ok;
}

// Sum over the 512 threads of the work-group (result in every thread).
WL_DEV float block_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; i++) s += red[i];
    __syncthreads();
    return s;
}

// post_attention_layernorm of the hidden state, split into three bf16 pieces
// in LDS. rms_norm: w * (x * (1/sqrt(mean(x^2) + eps))) in fp32
// (tools/ref_glm_chain.py:63-80; src/glm_primitives.cuh:35-62).
WL_DEV void norm_prologue(const DecodeArgs& a, const float* hidden, uint16_t* xp, uint32_t xps, float* red,
                          bool tap) {
    const uint32_t H = a.H;
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < H; i += kThreads) {
        const float x = hidden[i];
        ss = __fadd_rn(ss, __fmul_rn(x, x));
    }
    const float tot = block_sum(ss, red);
    const float r = 1.0f / sqrtf(tot / (float)H + a.eps);
    for (uint32_t i = threadIdx.x; i < H; i += kThreads) {
        float xn = __fmul_rn(hidden[i], r);
        if (a.ln_w) xn = __fmul_rn(xn, bf2f(a.ln_w[i]));
        if (tap) a.norm[i] = xn;
        uint32_t h, m, l;
        split3(xn, h, m, l);
        xp[i] = (uint16_t)h;
        xp[xps + i] = (uint16_t)m;
        xp[2 * xps + i] = (uint16_t)l;
    }
    __syncthreads();
}

// ---- tile kernels -----------------------------------------------------------
// All weight loads go through explicit global-address-space pointers and are
// issued unconditionally (k tiles past the end are clamped to the last valid
// tile and their A operand is zeroed), so a wave keeps its whole batch of
// loads in flight instead of waiting on each one.

// Rows [0,16) of NM bf16 matrices (row stride ld elements, pointers at the
// tile's first row), k in 32-wide tiles [kt0, kt0+nkt), against the LDS norm
// pieces. Leaves per-wave row sums in red[wave][mat*16 + row].
template <int NM, int MAXT>
WL_DEV void bf16_tile(const uint16_t* const (&W)[NM], uint32_t ld, uint32_t kt0, uint32_t nkt,
                      const uint16_t* xp, uint32_t xps, float* red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15, g = lane >> 4;
    f32x4 d[NM];
#pragma unroll
    for (int mt = 0; mt < NM; mt++) d[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t base = 0; base < nkt; base += kWaves * MAXT) {
        u32x4 wv[NM][MAXT];
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const uint32_t kt = min(base + wave + kWaves * i, nkt - 1);
#pragma unroll
            for (int mt = 0; mt < NM; mt++)
                wv[mt][i] = gld16(W[mt] + (size_t)n * ld + (kt0 + kt) * 32 + g * 8);
        }
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const uint32_t ktr = base + wave + kWaves * i;
            const uint32_t kt = min(ktr, nkt - 1);
            const bf16x8 av = a_lds(xp, xps, n, (kt0 + kt) * 32 + g * 8, ktr < nkt);
#pragma unroll
            for (int mt = 0; mt < NM; mt++) d[mt] = mma(av, as_bf16x8(wv[mt][i]), d[mt]);
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int mt = 0; mt < NM; mt++) red[wave * 64 + mt * 16 + lane] = sum3(d[mt]);
    }
    __syncthreads();
}

// Routed gate/up rows [0,16) of one MXFP4 expert (pointers at the tile's first
// row), full K = H, against the LDS norm pieces. Leaves red[wave][0..15] = gate,
// red[wave][16..31] = up.
template <int MAXT>
WL_DEV void fp4_gu_tile(const uint8_t* gw, const uint8_t* gs, const uint8_t* uw,
                        const uint8_t* us, uint32_t H, const uint16_t* xp, uint32_t xps,
                        float* red) {
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

// Shared-expert down rows [0,16) (bf16, row stride SI, pointer at the first
// row), against the global SwiGLU pieces ap [3][SI]. red[wave][0..15].
template <int MAXT>
WL_DEV void bf16_down_tile(const uint16_t* W, uint32_t SI, const uint16_t* ap, float* red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t nkt = SI / 32;
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t base = 0; base < nkt; base += kWaves * MAXT) {
        u32x4 wv[MAXT];
        bf16x8 av[MAXT];
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const uint32_t ktr = base + wave + kWaves * i;
            const uint32_t kt = min(ktr, nkt - 1);
            wv[i] = gld16(W + (size_t)n * SI + kt * 32 + g * 8);
            av[i] = a_glb(ap, SI, n, kt * 32 + g * 8, ktr < nkt);
        }
#pragma unroll
        for (int i = 0; i < MAXT; i++) d = mma(av[i], as_bf16x8(wv[i]), d);
    }
    if (lane < 16) red[wave * 64 + lane] = sum3(d);
    __syncthreads();
}

// Routed down: RT row tiles (16 rows each, pointers at the block's first row)
// of one MXFP4 expert over K = I, against that expert's SwiGLU pieces ap
// [3][aps] (global or LDS). red[wave][t*16 + row].
template <int RT, int MAXT>
WL_DEV void fp4_down_block(const uint8_t* dw, const uint8_t* ds, uint32_t I, const uint16_t* ap,
                           uint32_t aps, float* red) {
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


// ---- top-k (the last router tile's work-group) ------------------------------
// sigmoid, +e_score_correction_bias, top-K by biased score with ties to the
// lowest index (the reference's serial strict-> argmax, src/glm_layer_runner.cuh:
// 318-330), weight = unbiased score, / (sum + 1e-20), x routed_scaling
// (tools/ref_glm_chain.py:127-149). Slot order: descending biased score.
WL_DEV void topk_publish(const DecodeArgs& a, float* sc, float* ch, float* wsel) {
    const uint32_t E = a.E, K = a.K;
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        const float s = 1.0f / (1.0f + expf(-a.logits[e]));
        float c = s + a.bias[e];
        if (c != c) c = -INFINITY;  // a NaN choice never wins
        sc[e] = s;
        ch[e] = c;
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < E; e += kThreads) {
        const float c = ch[e];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < E; j++) {
            const float cj = ch[j];
            rank += (cj > c || (cj == c && j < e)) ? 1u : 0u;
        }
        if (rank < K) {
            a.idx[rank] = (int32_t)e;
            wsel[rank] = sc[e];  // unbiased score of slot `rank`
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.f;
        for (uint32_t k = 0; k < K; k++) sum += wsel[k];
        const float den = sum + 1e-20f;
        uint32_t bad = 0;
        for (uint32_t k = 0; k < K; k++) {
            float w = wsel[k];
            if (a.norm_topk) w = w / den;
            a.topw[k] = w * a.scaling;
            const uint8_t* blk = a.slot_tab[a.idx[k]];
            if (!blk) bad = 1;
            a.sel[k] = blk;
        }
        if (bad) raise_error(a.sync, SyncMap::make(a.H, a.I, a.E, a.K, a.SI), E_NOT_RESIDENT);
    }
    __syncthreads();
}

// ---- the persistent task kernel ----------------------------------------------
// Work-group b runs tasks b, b + G, b + 2G, ... (G = gridDim.x); tasks are
// numbered in dependency order, so each work-group meets its waits in the order
// the producers finish. With the fused schedule G is the number of work-groups
// the device holds at once, so every producer is resident; the waits are bounded
// regardless and report E_SPIN instead of hanging.
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
moe_decode_kernel(const DecodeArgs* __restrict__ pa, const DecodeDyn d) {
    const DecodeArgs& a = *pa;
    extern __shared__ __align__(16) uint8_t lds_raw[];
    const uint32_t xps = a.H + 8;
    uint16_t* xp = (uint16_t*)lds_raw;
    float* red = (float*)(lds_raw + decode_lds_xp_elems(a.H) * 2);
    float* ebuf = red + kWaves * 64;          // [32][16]
    float* tks = ebuf + 32 * 16;              // [2E + 32] top-k staging
    __shared__ uint32_t s_bcast;
    __shared__ const uint8_t* s_sel[32];
    __shared__ float s_w[32];

    const TaskMap tm = TaskMap::make(a.H, a.I, a.E, a.K, a.SI);
    const SyncMap sm = SyncMap::make(a.H, a.I, a.E, a.K, a.SI);
    uint32_t* sync = a.sync;
    const uint32_t ep = d.epoch;
    const uint32_t tid = threadIdx.x;
    bool have_norm = false, have_topk = false, have_sgu = false, ok_all = true;
    uint32_t have_rgu_k = 0xFFFFFFFFu;

    for (uint32_t t = d.task_lo + blockIdx.x; t < d.task_hi; t += gridDim.x) {
        if (t < tm.oSG) {
            // ---------------- router partial (16 rows, one k-quarter) -------------
            const uint32_t tile = t >> 2, q = t & 3u;
            const uint32_t nkt = a.H / 32 / 4;
            if (!have_norm) { norm_prologue(a, d.hidden, xp, xps, red, d.write_norm_tap && t == 0); have_norm = true; }
            const uint16_t* W[1] = {a.router_w + (size_t)tile * 16 * a.H};
            bf16_tile<1, 6>(W, a.H, q * nkt, nkt, xp, xps, red);
            if (tid < 16) a.part_r[(tile * 4 + q) * 16 + tid] = wave_total(red, tid);
            uint32_t* cnt = sync + sm.c_rtile + tile * kLineWords;
            if (arrive(cnt, &s_bcast) == 3u) {
                acquire_all();
                if (tid < 16) {
                    float sum = 0.f;
                    for (int qq = 0; qq < 4; qq++) sum += a.part_r[(tile * 4 + qq) * 16 + tid];
                    a.logits[tile * 16 + tid] = sum;
                }
                if (tid == 0) st_sync(cnt, 0u);
                uint32_t* done = sync + sm.c_router;
                if (arrive(done, &s_bcast) == a.E / 16 - 1) {
                    acquire_all();
                    topk_publish(a, tks, tks + a.E, tks + 2 * a.E);
                    if (tid == 0) st_sync(done, 0u);
                    signal(sync + sm.f_topk, ep);
                }
            }
        } else if (t < tm.oRG) {
            // ---------------- shared gate/up partial ------------------------------
            const uint32_t u = t - tm.oSG;
            const uint32_t tile = u >> 2, q = u & 3u;
            const uint32_t nkt = a.H / 32 / 4;
            if (!have_norm) { norm_prologue(a, d.hidden, xp, xps, red, false); have_norm = true; }
            const uint16_t* W[2] = {a.sh_gate + (size_t)tile * 16 * a.H,
                                    a.sh_up + (size_t)tile * 16 * a.H};
            bf16_tile<2, 6>(W, a.H, q * nkt, nkt, xp, xps, red);
            if (tid < 32) a.part_s[(tile * 4 + q) * 32 + tid] = wave_total(red, tid);
            uint32_t* cnt = sync + sm.c_sgtile + tile * kLineWords;
            if (arrive(cnt, &s_bcast) == 3u) {
                acquire_all();
                if (tid < 16) {
                    float gs = 0.f, us = 0.f;
                    for (int qq = 0; qq < 4; qq++) {
                        gs += a.part_s[(tile * 4 + qq) * 32 + tid];
                        us += a.part_s[(tile * 4 + qq) * 32 + 16 + tid];
                    }
                    const float mid = silu_mul(gs, us);
                    const uint32_t r = tile * 16 + tid;
                    a.smid[r] = mid;
                    uint32_t h, m, l;
                    split3(mid, h, m, l);
                    a.smid_p[r] = (uint16_t)h;
                    a.smid_p[a.SI + r] = (uint16_t)m;
                    a.smid_p[2 * a.SI + r] = (uint16_t)l;
                }
                if (tid == 0) st_sync(cnt, 0u);
                signal(sync + sm.f_sgu + tile, ep);
            }
        } else if (t < tm.oSD) {
            // ---------------- routed gate/up + SwiGLU -----------------------------
            const uint32_t u = t - tm.oRG;
            const uint32_t tiles = a.I / 16;
            const uint32_t k = u / tiles, tile = u % tiles;
            if (!have_norm) { norm_prologue(a, d.hidden, xp, xps, red, false); have_norm = true; }
            if (!have_topk) {
                if (d.wait_deps) ok_all = wait_flags(sync, sm, sm.f_topk, 1, ep, &s_bcast) && ok_all;
                if (tid < a.K) { s_sel[tid] = a.sel[tid]; s_w[tid] = a.topw[tid]; }
                __syncthreads();
                have_topk = true;
            }
            const uint8_t* blk = ok_all ? s_sel[k] : nullptr;
            if (blk) {
                const size_t r0 = (size_t)tile * 16;
                fp4_gu_tile<3>(blk + a.gw_off + r0 * (a.H / 2), blk + a.gs_off + r0 * (a.H / 32),
                               blk + a.uw_off + r0 * (a.H / 2), blk + a.us_off + r0 * (a.H / 32), a.H,
                               xp, xps, red);
                if (tid < 16) {
                    const float mid = silu_mul(wave_total(red, tid), wave_total(red, 16 + tid));
                    const uint32_t r = tile * 16 + tid;
                    a.rmid[(size_t)k * a.I + r] = mid;
                    uint32_t h, m, l;
                    split3(mid, h, m, l);
                    uint16_t* p = a.rmid_p + (size_t)k * 3 * a.I;
                    p[r] = (uint16_t)h;
                    p[a.I + r] = (uint16_t)m;
                    p[2 * a.I + r] = (uint16_t)l;
                }
                signal(sync + sm.f_rgu + k * tiles + tile, ep);
            }
        } else if (t < tm.oRD) {
            // ---------------- shared down -----------------------------------------
            const uint32_t tile = t - tm.oSD;
            if (!have_sgu) {
                if (d.wait_deps) ok_all = wait_flags(sync, sm, sm.f_sgu, a.SI / 16, ep, &s_bcast) && ok_all;
                have_sgu = true;
            }
            if (ok_all) {
                bf16_down_tile<8>(a.sh_down + (size_t)tile * 16 * a.SI, a.SI, a.smid_p, red);
                if (tid < 16) a.shared_out[tile * 16 + tid] = wave_total(red, tid);
                signal(sync + sm.f_sdown + tile, ep);
            }
        } else {
            // ---------------- routed down + combine -------------------------------
            const uint32_t u = t - tm.oRD;
            const uint32_t blocks = a.H / (16 * kDownRT);
            const uint32_t k = u / blocks, blkrow = u % blocks;
            if (!have_topk) {
                if (d.wait_deps) ok_all = wait_flags(sync, sm, sm.f_topk, 1, ep, &s_bcast) && ok_all;
                if (tid < a.K) { s_sel[tid] = a.sel[tid]; s_w[tid] = a.topw[tid]; }
                __syncthreads();
                have_topk = true;
            }
            if (have_rgu_k != k) {
                // this expert's SwiGLU output must be complete
                if (d.wait_deps)
                    ok_all = wait_flags(sync, sm, sm.f_rgu + k * (a.I / 16), a.I / 16, ep, &s_bcast) && ok_all;
                have_rgu_k = k;
            }
            const uint8_t* blk = ok_all ? s_sel[k] : nullptr;
            if (blk) {
                const size_t r0 = (size_t)blkrow * 16 * kDownRT;
                fp4_down_block<kDownRT, 1>(blk + a.dw_off + r0 * (a.I / 2), blk + a.ds_off + r0 * (a.I / 32),
                                           a.I, a.rmid_p + (size_t)k * 3 * a.I, a.I, red);
                if (tid < 16 * kDownRT) a.edown[(size_t)k * a.H + r0 + tid] = wave_total(red, tid);
                uint32_t* cnt = sync + sm.c_rdblk + blkrow * kLineWords;
                if (arrive(cnt, &s_bcast) == a.K - 1) {
                    acquire_all();
                    bool ok2 = true;
                    if (d.wait_deps)
                        ok2 = wait_flags(sync, sm, sm.f_sdown + blkrow * kDownRT, kDownRT, ep, &s_bcast);
                    if (ok2 && tid < 16 * kDownRT) {
                        const size_t r = r0 + tid;
                        float acc = 0.f;
                        for (uint32_t kk = 0; kk < a.K; kk++)
                            acc = __fadd_rn(acc, __fmul_rn(s_w[kk], a.edown[(size_t)kk * a.H + r]));
                        acc = __fadd_rn(acc, a.shared_out[r]);
                        d.out[r] = d.resid ? __fadd_rn(d.resid[r], acc) : acc;
                    }
                    if (tid == 0) st_sync(cnt, 0u);
                }
            }
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

// y[r] = sum_c e2m1(W[r,c]) * 2^(S[r,c/32]-127) * x[c]; one work-group per 16
// rows. Drop-in for launch_dequant_matvec_mxfp4 (src/glm_kernels.cuh:104-110).
__global__ void __launch_bounds__(kThreads)
dequant_matvec_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ S,
                      const float* __restrict__ x, float* __restrict__ y, uint32_t N, uint32_t K) {
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
ffn_gu_kernel(const uint8_t* __restrict__ blk, uint64_t gw_off, uint64_t gs_off, uint64_t uw_off,
              uint64_t us_off, const float* __restrict__ x, uint32_t H, uint32_t I,
              float* __restrict__ mid, uint16_t* __restrict__ mid_p) {
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
ffn_down_kernel(const uint8_t* __restrict__ blk, uint64_t dw_off, uint64_t ds_off,
                const uint16_t* __restrict__ mid_p, uint32_t H, uint32_t I, float* __restrict__ y,
                uint16_t* __restrict__ y_bf16) {
    __shared__ float red[kWaves * 64];
    const size_t r0 = (size_t)blockIdx.x * 16 * kDownRT;
    fp4_down_block<kDownRT, 1>(blk + dw_off + r0 * (I / 2), blk + ds_off + r0 * (I / 32), I, mid_p, I, red);
    if (threadIdx.x < 16 * kDownRT) {
        const float v = wave_total(red, threadIdx.x);
        y[r0 + threadIdx.x] = v;
        if (y_bf16) y_bf16[r0 + threadIdx.x] = (uint16_t)f2bf(v);
    }
}

int launch_dequant_matvec(const uint8_t* W, const uint8_t* S, const float* x, float* y, uint32_t N,
                          uint32_t K, void* stream) {
    const size_t lds = (size_t)3 * (K + 8) * 2 + kWaves * 64 * 4;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)dequant_matvec_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(dequant_matvec_kernel, dim3(N / 16), dim3(kThreads), lds, (hipStream_t)stream, W, S,
                       x, y, N, K);
    return (int)hipGetLastError();
}

int launch_expert_ffn(const uint8_t* blk, uint64_t gw_off, uint64_t gs_off, uint64_t uw_off,
                      uint64_t us_off, uint64_t dw_off, uint64_t ds_off, const float* x, uint32_t H,
                      uint32_t I, float* mid, uint16_t* mid_p, float* y, uint16_t* y_bf16,
                      void* stream) {
    const size_t lds = (size_t)3 * (H + 8) * 2 + kWaves * 64 * 4;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)ffn_gu_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
    }
    hipLaunchKernelGGL(ffn_gu_kernel, dim3(I / 16), dim3(kThreads), lds, (hipStream_t)stream, blk, gw_off,
                       gs_off, uw_off, us_off, x, H, I, mid, mid_p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(ffn_down_kernel, dim3(H / (16 * kDownRT)), dim3(kThreads), 0, (hipStream_t)stream,
                       blk, dw_off, ds_off, mid_p, H, I, y, y_bf16);
    return (int)hipGetLastError();
}

int launch_decode(const DecodeArgs* d_args, const DecodeDyn& dyn, uint32_t H, uint32_t E,
                  uint32_t grid, void* stream) {
    const size_t lds = decode_lds_bytes(H, E);
    hipLaunchKernelGGL(moe_decode_kernel, dim3(grid), dim3(kThreads), lds, (hipStream_t)stream, d_args,
                       dyn);
    return (int)hipGetLastError();
}

int decode_occupancy(uint32_t H, uint32_t E, int* blocks_per_cu) {
    const size_t lds = decode_lds_bytes(H, E);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)moe_decode_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
    }
    return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, moe_decode_kernel,
                                                             kThreads, lds);
}

}  // namespace wl
