// moe_batched.hip — the MoE layer for T tokens at once on gfx950 (the
// reference's run_moe_batched, src/glm_layer_runner.cuh:818-928, used by
// prefill): every expert's weights are streamed once per pass of up to kMT of
// its tokens instead of once per token.
//
//   bnorm    RMSNorm per token -> norm (f32, for the router) and norm3 (the
//            three bf16 pieces the GEMMs read)
//   broute   router logits, kTB tokens per work-group; norm and logits use the
//            arithmetic of the decode and routing kernels, so a token's ids
//            equal the ones wl_run_moe selects for it
//   btopk    sigmoid + bias, top-k, weights (one work-group per token)
//   bcount   per expert: its entries (token*K + slot) in ascending order
//            (wave ballots, deterministic) and their count
//   bscatter per expert: its compact range (prefix of the counts), ent/pos
//   bup      gate/up + SwiGLU: shared expert (unit = token pass x 64 rows),
//            routed experts (unit = expert pass x 4 x 64 rows); a routed
//            pass's activation DMAs read its tokens' norm3 rows in place,
//            through a per-work-group table of its units' tokens in LDS, so
//            no expert-major copy of the activations is made
//   bdown    down: shared expert (unit = token pass x 128 rows), routed
//            experts (unit = expert pass x 512 rows)
//   bcomb    out[t] = (resid[t] +) sum_k w[t][k] e_k[t] (slot order) + shared[t]
//
// The GEMMs run each activation as three bf16 pieces (x = p0 + p1 + p2 to f32
// precision) through v_mfma_f32_16x16x32_bf16; MXFP4 weights are converted
// exactly to bf16 (v_cvt_scalef32_pk_bf16_fp4), bf16 weights are used as they
// are. bup and bdown are persistent (one work-group per CU) and share one step
// pipeline: activations arrive in LDS by DMA, weights two steps ahead in
// registers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "dev_common.h"
#include "internal.h"

namespace wl {

#define WL_MEM __device__ __forceinline__  // member functions

constexpr uint32_t kMT = 32;         // tokens per pass: two MFMA row blocks of 16
constexpr uint32_t kMTW = 64;        // tokens per wide pass (more than kMT tokens): four row blocks
constexpr uint32_t kKCW = 128;       // activation columns staged per wide step
constexpr uint32_t kMTR = 48;        // tokens per wide pass of a routed expert (three row blocks)
constexpr uint32_t kKC = 256;        // activation columns staged per step
constexpr uint32_t kTB = 8;          // tokens per routing work-group

// Row layout of a pass's staged activations, chosen per pass from its token
// count nt (wave-uniform):
//   pieces in rows (nt <= kPR): plane 0, row 4m + pc holds piece pc of token
//     m (row 4m + 3 unused), so one MFMA covers 4 tokens; the three pieces of
//     token 4tb + g come out as elements 0..2 of lane group g of block tb and
//     are summed like the decode kernel's (sum3);
//   tokens in rows (nt > kPR): plane pc, row m holds piece pc of token m; the
//     three pieces accumulate into one tile by three MFMAs per 16 tokens.
// MFMA rows are independent, so rows of absent tokens may hold anything.
constexpr uint32_t kPR = 8;
struct PassShape {
    uint32_t nblk;  // 16-row blocks
    uint32_t npc;   // planes (MFMAs per block)
    bool pr;        // pieces in rows
};
WL_DEV PassShape pass_shape(uint32_t nt) {
    return nt <= kPR ? PassShape{cdiv(nt, 4u), 1u, true} : PassShape{cdiv(nt, 16u), 3u, false};
}
// The outputs of a tile: lane (n, g) calls f(m, value) for each live token m
// whose column-n value it holds. The epilogues pass the lane through
// opaque_lane, so the compiler cannot hoist their per-row addresses out of
// the step loop (where they would hold registers for the whole kernel).
WL_DEV uint32_t opaque_lane() {
    uint32_t l = threadIdx.x & 63u;
    asm volatile("" : "+v"(l));
    return l;
}
template <class F>
WL_DEV void tile_each(const f32x4 (&acc)[2], uint32_t nt, bool pr, uint32_t lane, F f) {
    const uint32_t g = lane >> 4;
#pragma unroll
    for (uint32_t tb = 0; tb < 2; tb++) {
        if (pr) {
            const uint32_t m = 4u * tb + g;
            if (m < nt) f(m, sum3(acc[tb]));
        } else {
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) {
                const uint32_t m = tb * 16u + 4u * g + i;
                if (m < nt) f(m, acc[tb][i]);
            }
        }
    }
}
// SwiGLU epilogue of a gate/up tile: columns n < 8 are gate rows, n + 8 the
// matching up rows. Calls put(m, n, value) for n < 8 and live tokens.
template <class PutF>
WL_DEV void swiglu_store(const f32x4 (&acc)[2], uint32_t nt, bool pr, uint32_t lane, PutF put) {
    const uint32_t n = lane & 15u, g = lane >> 4;
#pragma unroll
    for (uint32_t tb = 0; tb < 2; tb++) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            if (pr && i > 0) continue;
            const float v = pr ? sum3(acc[tb]) : acc[tb][i];
            // lane n < 8 takes lane n + 8 of its 16-lane row (DPP row_ror:8)
            const float up = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
            const uint32_t m = pr ? 4u * tb + g : tb * 16u + 4u * g + i;
            if (n < 8u && m < nt) put(m, n, silu_mul(v, up));
        }
    }
}
// The three bf16 pieces of 4 consecutive values at p, p + stride, p + 2 stride.
WL_DEV void store_pieces4(uint16_t* p, uint32_t stride, const float (&x)[4]) {
    uint32_t h[4], md[4], l[4];
#pragma unroll
    for (int q = 0; q < 4; q++) split3(x[q], h[q], md[q], l[q]);
    auto pack = [](const uint32_t (&x)[4]) {
        return (uint64_t)(x[0] | (x[1] << 16)) | ((uint64_t)(x[2] | (x[3] << 16)) << 32);
    };
    gst((uint64_t*)p, pack(h));
    gst((uint64_t*)(p + stride), pack(md));
    gst((uint64_t*)(p + 2u * stride), pack(l));
}

// ---- routing ------------------------------------------------------------------
// RMSNorm of token t = blockIdx.x (norm_rinv / norm_value: the decode kernel's
// arithmetic) into b.norm, and its three bf16 pieces into b.norm3.
__global__ void __launch_bounds__(kThreads) bnorm_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, tid = threadIdx.x, t = blockIdx.x;
    __shared__ float red[kWaves * 64];
    const rsrc_t hid_rs = make_rsrc(b.hidden + (size_t)t * H, H * 4u);
    const rsrc_t ln_rs = make_rsrc(a.ln_w ? (const void*)a.ln_w : (const void*)b.hidden, H * 2u);
    float4 hv[kHV];
    uint2 lv[kHV];
#pragma unroll
    for (int i = 0; i < kHV; i++) {
        const uint32_t j = tid + kThreads * i;
        hv[i] = __builtin_bit_cast(float4, bld16(hid_rs, 16u * j, 0u));
        lv[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ln_rs, (int)(8u * j), 0, 0));
    }
    const float rinv = norm_rinv(hv, red, H, a.eps);
#pragma unroll
    for (int i = 0; i < kHV; i++) {
        const uint32_t j = tid + kThreads * i;
        if (j < H / 4) {
            const float xs[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
            const uint32_t ls[4] = {lv[i].x & 0xFFFFu, lv[i].x >> 16, lv[i].y & 0xFFFFu, lv[i].y >> 16};
            float4 o;
            o.x = norm_value(xs[0], rinv, a.ln_w != nullptr, ls[0]);
            o.y = norm_value(xs[1], rinv, a.ln_w != nullptr, ls[1]);
            o.z = norm_value(xs[2], rinv, a.ln_w != nullptr, ls[2]);
            o.w = norm_value(xs[3], rinv, a.ln_w != nullptr, ls[3]);
            *(__attribute__((address_space(1))) u32x4*)(b.norm + (size_t)t * H + 4 * j) = __builtin_bit_cast(u32x4, o);
            const float os[4] = {o.x, o.y, o.z, o.w};
            store_pieces4(b.norm3 + (size_t)t * 3u * H + 4 * j, H, os);
        }
    }
}

// Wave sums of NV values per lane at once (NV a power of two <= 64), each
// summed over the 64 lanes by the same tree as router_partial_x's butterfly
// (x += shfl_xor(x, o), o = 32, 16, ..., 1): at each of the first log2(NV)
// levels a lane keeps half of its values and adds its partner's copy of them
// (the two operands the butterfly adds in this lane at this level), the
// levels after that are the butterfly itself. Afterwards lane l holds, in
// x[0], the sum of value l >> (6 - log2 NV) — bit for bit the butterfly's.
// (Levels are template parameters: every index into x is a constant, so x
// stays in registers without indexed moves.)
template <uint32_t N, uint32_t n, uint32_t o>  // values [0, 2n) -> [0, n) at offset o
WL_DEV void wave_levels(float (&x)[N]) {
    if constexpr (n >= 1u) {
        const bool up = (threadIdx.x & o) != 0u;
#pragma unroll
        for (uint32_t j = 0; j < n; j++) {
            const float keep = up ? x[j + n] : x[j];
            const float send = up ? x[j] : x[j + n];
            x[j] = keep + __shfl_xor(send, (int)o, 64);
        }
        wave_levels<N, n / 2u, o / 2u>(x);
    } else if constexpr (o >= 1u) {
        x[0] += __shfl_xor(x[0], (int)o, 64);
        wave_levels<N, 0u, o / 2u>(x);
    }
}
template <uint32_t NV>
WL_DEV void multi_wave_sum(float (&x)[NV]) {
    static_assert(NV >= 1u && NV <= 64u && (NV & (NV - 1u)) == 0u, "NV: a power of two <= 64");
    wave_levels<NV, NV / 2u, 32u>(x);
}

// Router logits of kTB tokens: each thread keeps its router_chain_x share of
// every token's normalised input in registers; the rows stream through, kRR
// at a time (rows r = x + gridDim.x (kRR i + q), q < kRR; the next group
// prefetched). The kRR x kTB wave sums of a group are taken together
// (multi_wave_sum), then summed over the waves in order from 0 — the
// arithmetic of router_partial and router_publish, so each logit equals the
// one the decode and routing kernels compute for the token.
constexpr uint32_t kRR = 4;  // router rows per group
__global__ void __launch_bounds__(kThreads) broute_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, E = a.E, tid = threadIdx.x, lane = tid & 63u, v = uni(tid >> 6);
    constexpr uint32_t NV = kRR * kTB;  // value q * kTB + tt: row q, token tt
    constexpr uint32_t SH = 6u - __builtin_ctz(NV);
    constexpr uint32_t kFL = 64;  // groups whose logits are buffered in LDS
    __shared__ float red[kWaves * 64];
    __shared__ float lgb[kFL * NV];
    const uint32_t t0 = blockIdx.y * kTB, nch = H / 8, gx = gridDim.x;
    float4 xr[kTB][kRCH][2];  // xn[8c .. 8c+8) of chunks c = tid + 512 m, per token
#pragma unroll
    for (uint32_t tt = 0; tt < kTB; tt++) {
        const bool live = t0 + tt < b.T;
        const rsrc_t nrs = make_rsrc(b.norm + (size_t)min(t0 + tt, b.T - 1u) * H, live ? H * 4u : 0u);
#pragma unroll
        for (int m = 0; m < kRCH; m++) {
            const uint32_t c = tid + kThreads * m;
            xr[tt][m][0] = __builtin_bit_cast(float4, bld16(nrs, 32u * c, 0u));
            xr[tt][m][1] = __builtin_bit_cast(float4, bld16(nrs, 32u * c + 16u, 0u));
        }
    }
    const rsrc_t rt_rs = make_rsrc(a.router_w, E * H * 2u);
    auto row_of = [&](uint32_t i, uint32_t q) { return blockIdx.x + gx * (kRR * i + q); };
    u32x4 rn[kRR][kRCH];
#pragma unroll
    for (uint32_t q = 0; q < kRR; q++)
#pragma unroll
        for (int m = 0; m < kRCH; m++)
            rn[q][m] = bld16(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), min(row_of(0u, q), E - 1u) * H * 2u);
    for (uint32_t i = 0; row_of(i, 0u) < E; i++) {
        u32x4 rw[kRR][kRCH];
#pragma unroll
        for (uint32_t q = 0; q < kRR; q++)
#pragma unroll
            for (int m = 0; m < kRCH; m++) {
                rw[q][m] = rn[q][m];
                rn[q][m] = bld16(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), min(row_of(i + 1u, q), E - 1u) * H * 2u);
            }
        // router_chain_x for every (row, token) value, its chunks in the same
        // order (m, then the 8 columns), with one branch per chunk instead of
        // one per value, so the NV independent chains interleave
        float x[NV];
#pragma unroll
        for (uint32_t j = 0; j < NV; j++) x[j] = 0.f;
#pragma unroll
        for (int m = 0; m < kRCH; m++) {
            if (tid + kThreads * m < nch) {
#pragma unroll
                for (uint32_t q = 0; q < kRR; q++) {
                    const u32x4 r = rw[q][m];
                    const float wv[8] = {bf2f(r.x & 0xFFFFu), bf2f(r.x >> 16), bf2f(r.y & 0xFFFFu), bf2f(r.y >> 16),
                                         bf2f(r.z & 0xFFFFu), bf2f(r.z >> 16), bf2f(r.w & 0xFFFFu), bf2f(r.w >> 16)};
#pragma unroll
                    for (uint32_t tt = 0; tt < kTB; tt++) {
                        const float4 x0 = xr[tt][m][0], x1 = xr[tt][m][1];
                        float pd = x[q * kTB + tt];
                        pd = fmaf(wv[0], x0.x, pd);
                        pd = fmaf(wv[1], x0.y, pd);
                        pd = fmaf(wv[2], x0.z, pd);
                        pd = fmaf(wv[3], x0.w, pd);
                        pd = fmaf(wv[4], x1.x, pd);
                        pd = fmaf(wv[5], x1.y, pd);
                        pd = fmaf(wv[6], x1.z, pd);
                        pd = fmaf(wv[7], x1.w, pd);
                        x[q * kTB + tt] = pd;
                    }
                }
            }
        }
        multi_wave_sum(x);
        if ((lane & ((1u << SH) - 1u)) == 0u) red[v * 64u + (lane >> SH)] = x[0];
        lds_barrier();
        if (tid < NV) {
            float sum = 0.f;  // the same order as router_publish
#pragma unroll
            for (int wv = 0; wv < kWaves; wv++) sum += red[wv * 64 + tid];
            lgb[(i % kFL) * NV + tid] = sum;
        }
        lds_barrier();
        // the logits go out kFL groups at a time: a store in the loop would be
        // waited for with the next group's rows (loads and stores share one
        // counter), i.e. every group would wait for a store's round trip
        if (i % kFL == kFL - 1u || row_of(i + 1u, 0u) >= E) {
            const uint32_t i0 = i - i % kFL, n = (i % kFL + 1u) * NV;
            for (uint32_t j = tid; j < n; j += kThreads) {
                const uint32_t q = (j % NV) / kTB, tt = j % kTB, r = row_of(i0 + j / NV, q);
                if (r < E && t0 + tt < b.T) gst(b.logits + (size_t)(t0 + tt) * E + r, lgb[j]);
            }
        }
    }
}

__global__ void __launch_bounds__(kThreads) btopk_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t E = a.E, K = a.K, t = blockIdx.x, tid = threadIdx.x;
    extern __shared__ __align__(16) uint8_t lds[];
    float* tk_sc = (float*)lds;
    float* tk_ch = tk_sc + E;
    uint32_t* tk_idx = (uint32_t*)(tk_ch + E);
    float* tk_w = (float*)(tk_idx + 32);
    for (uint32_t e = tid; e < E; e += kThreads)
        topk_score(gld(b.logits + (size_t)t * E + e), gld(a.bias + e), e, tk_sc, tk_ch);
    lds_barrier();
    if (E <= 256u) topk_argmax(E, K, tk_sc, tk_ch, tk_idx, tk_w);
    else topk_rank(E, K, tk_sc, tk_ch, tk_idx, tk_w);
    if (tid < K) {
        gst(b.idx + (size_t)t * K + tid, (int32_t)tk_idx[tid]);
        gst(b.wts + (size_t)t * K + tid, topk_weight(a, K, tk_w, tid));
    }
}

// Entries of expert e in ascending (token, slot) order: one wave, 64 entries
// per step, positions from a ballot prefix; the ids of kCB steps are loaded
// at once (one memory round trip per kCB steps).
constexpr uint32_t kCB = 8;
__global__ void __launch_bounds__(64) bcount_kernel(const BatchArgs b, uint32_t K) {
    const uint32_t e = blockIdx.x, lane = threadIdx.x, n = b.T * K;
    const rsrc_t ids = make_rsrc(b.idx, n * 4u);  // past n: zeros, masked by i < n
    uint32_t base = 0;
    for (uint32_t i0 = 0; i0 < n; i0 += 64u * kCB) {
        uint32_t id[kCB];
#pragma unroll
        for (uint32_t j = 0; j < kCB; j++)
            id[j] = __builtin_amdgcn_raw_buffer_load_b32(ids, (int)(4u * (i0 + 64u * j + lane)), 0, 0);
#pragma unroll
        for (uint32_t j = 0; j < kCB; j++) {
            const uint32_t i = i0 + 64u * j + lane;
            const bool hit = i < n && id[j] == e;
            const uint64_t bal = __builtin_amdgcn_ballot_w64(hit);
            const uint32_t below =
                __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            if (hit) gst(b.lists + (size_t)e * b.T + base + below, i);
            base += (uint32_t)__builtin_popcountll(bal);
        }
    }
    if (lane == 0) gst(b.counts + e, base);
}

// The compact range of expert e (exclusive prefix of the counts) and its
// entries' compact indices.
__global__ void __launch_bounds__(256) bscatter_kernel(const BatchArgs b, uint32_t E) {
    const uint32_t e = blockIdx.x, tid = threadIdx.x;
    __shared__ uint32_t s_off;
    if (tid < 64) {
        uint32_t s = 0;
        for (uint32_t f = tid; f < e; f += 64) s += gld(b.counts + f);
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        if (tid == 0) {
            s_off = s;
            gst(b.offsets + e, s);
            if (e == E - 1) gst(b.offsets + E, s + gld(b.counts + e));
        }
    }
    __syncthreads();
    const uint32_t off = s_off, ne = gld(b.counts + e);
    for (uint32_t i = tid; i < ne; i += blockDim.x) {
        const uint32_t en = gld(b.lists + (size_t)e * b.T + i);
        gst(b.ent + off + i, en);
        gst(b.pos + en, off + i);
    }
}

// ---- pass table ----------------------------------------------------------------
// Pass table of the routed GEMMs, in LDS: the experts' counts and offsets and
// the exclusive prefix pp of their passes (cdiv(count, kMT)), pp[E] = all
// passes. Units are numbered densely over the passes that exist (unit u =
// pass j * parts + part), so the grid-stride loop visits live units only and
// the passes of one expert sit next to each other.
// With wide passes on, an expert of more than kMT tokens runs as passes of
// kMTW tokens instead (their own prefix ppw, ppw[E] = all wide passes) and
// has no kMT passes.
struct PassTab {
    const uint32_t* cnt;
    const uint32_t* off;
    const uint32_t* pp;
    const uint32_t* ppw;
    uint32_t n;   // kMT passes
    uint32_t nw;  // kMTW passes
};
WL_DEV uint32_t passes_of(uint32_t c, bool wide) { return wide && c > kMT ? 0u : cdiv(c, kMT); }
WL_DEV uint32_t wide_passes_of(uint32_t c, bool wide) { return wide && c > kMT ? cdiv(c, kMTR) : 0u; }
// E counts the MXFP4 shared pseudo-expert (index E - 1) when there is one:
// all T tokens, compact rows from T*K on.
// wparts > 0: experts of more than kMT tokens run in wide passes if their
// wparts units per pass fill the grid (fewer wide units than work-groups
// leave the ones that hold one ending last: measured slower at T = 256).
// small > 0: routed experts of 1..small tokens are left out (their down
// projection runs in bdown_kernel's streaming pipeline, run_small_down).
WL_DEV PassTab load_pass_tab(const BatchArgs& b, uint32_t E, uint32_t K, uint32_t* s, const uint8_t* const* stab,
                             uint32_t wparts, uint32_t small = 0u) {
    const uint32_t tid = threadIdx.x;
    uint32_t *cnt = s, *off = s + E, *pp = s + 2u * E, *ppw = s + 3u * E + 1u;
    const bool skip = (b.flags & kBatchSkipUnbound) != 0u;
    const uint32_t esh = (b.flags & kBatchShared4) ? E - 1u : E;
    for (uint32_t f = tid; f < E; f += kThreads) {
        if (f == esh) {
            cnt[f] = (b.flags & kBatchNoShared) ? 0u : b.T;
            off[f] = b.T * K;
            continue;
        }
        // stab[f] was written by this thread (load_slot_tab, same stride)
        const uint32_t c = skip && stab[f] == nullptr ? 0u : gld(b.counts + f);
        cnt[f] = c <= small ? 0u : c;
        off[f] = gld(b.offsets + f);
    }
    lds_barrier();
    if (tid < 64u) {
        const uint32_t per = cdiv(E, 64u), e0 = tid * per;
        // inclusive scans over the wave of the kMT passes with and without
        // wide passes and of the wide passes; the wave then picks one form
        uint32_t mine0 = 0, mine1 = 0, minew = 0;
        for (uint32_t i = 0; i < per; i++)
            if (e0 + i < E) {
                mine0 += passes_of(cnt[e0 + i], false);
                mine1 += passes_of(cnt[e0 + i], true);
                minew += wide_passes_of(cnt[e0 + i], true);
            }
        uint32_t inc0 = mine0, inc1 = mine1, incw = minew;
#pragma unroll
        for (uint32_t o = 1; o < 64u; o <<= 1) {
            const uint32_t t0 = __shfl_up(inc0, o, 64), t1 = __shfl_up(inc1, o, 64), tw = __shfl_up(incw, o, 64);
            if (tid >= o) {
                inc0 += t0;
                inc1 += t1;
                incw += tw;
            }
        }
        const bool wide = wparts > 0u && __shfl(incw, 63, 64) * wparts >= gridDim.x;
        if (!wide) minew = incw = 0u;
        const uint32_t mine = wide ? mine1 : mine0, inc = wide ? inc1 : inc0;
        uint32_t run = inc - mine, runw = incw - minew;
        for (uint32_t i = 0; i < per; i++)
            if (e0 + i < E) {
                pp[e0 + i] = run;
                ppw[e0 + i] = runw;
                run += passes_of(cnt[e0 + i], wide);
                runw += wide_passes_of(cnt[e0 + i], wide);
            }
        if (tid == 63u) {
            pp[E] = inc;
            ppw[E] = incw;
        }
    }
    lds_barrier();
    return PassTab{cnt, off, pp, ppw, uni(pp[E]), uni(ppw[E])};
}
// Routed unit r (< n_passes * parts) -> (pass j, part). Units go in blocks
// of 8 passes x parts, ordered so that unit r has j % 8 == r % 8 in full
// blocks: with a grid of a multiple of 8 (work-group b runs on XCD b % 8),
// the units of one pass run on one XCD and share its L2 copy of the pass's
// activations.
struct PassPart {
    uint32_t j, part;
};
WL_DEV PassPart pass_part(uint32_t r, uint32_t parts, uint32_t npass) {
    const uint32_t blk = r / (8u * parts), l = r % (8u * parts);
    const uint32_t np = min(8u, npass - 8u * blk);
    return PassPart{8u * blk + l % np, l / np};
}
// Pass j (< n): its expert (the largest e with pp[e] <= j, which has a pass
// since pp[e + 1] > j), the pass within the expert, its token count and its
// first compact entry.
struct Pass {
    uint32_t e, nt, c0;
};
WL_DEV uint32_t expert_of_pass(const uint32_t* pp, uint32_t E, uint32_t j) {
    uint32_t lo = 0, hi = E;  // pp[lo] <= j < pp[hi]
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (uni(pp[mid]) <= j) lo = mid;
        else hi = mid;
    }
    return lo;
}
// kMT passes: full passes of kMT tokens, the remainder last.
WL_DEV Pass pass_at(const PassTab& pt, uint32_t E, uint32_t j) {
    const uint32_t e = expert_of_pass(pt.pp, E, j), p = j - uni(pt.pp[e]);
    return Pass{e, min(kMT, uni(pt.cnt[e]) - p * kMT), uni(pt.off[e]) + p * kMT};
}
// Wide passes: an expert's tokens split evenly over its cdiv(count, kMTR)
// passes (100 tokens: 34 + 33 + 33, not 48 + 48 + 4).
WL_DEV Pass pass_at_w(const PassTab& pt, uint32_t E, uint32_t j) {
    const uint32_t e = expert_of_pass(pt.ppw, E, j), p = j - uni(pt.ppw[e]);
    const uint32_t c = uni(pt.cnt[e]), np = cdiv(c, kMTR), q = c / np, r = c % np;
    return Pass{e, q + (p < r ? 1u : 0u), uni(pt.off[e]) + p * q + min(p, r)};
}

// ---- token table -------------------------------------------------------------
// A routed pass's activations are its tokens' rows of norm3, read in place by
// the DMAs. Before a gate/up pipeline runs, its work-group writes the tokens
// of its units' passes into LDS, tt[W i + m] = the token of row m of its unit
// i (W: the pipeline's largest pass), in one round of global loads for the
// whole pipeline; a unit's bind then reads its lane's two tokens there. (A
// prefetch into registers would cost a wait at every bind: the compiler does
// not know how many steps lie between a load and its use.) The host sizes
// the table (BatchArgs::tcap entries) for the most units a work-group can
// get (batched_tok_entries); past it, tokens read as 0 and E_TOKTAB is raised.
template <class Kn>
WL_DEV void fill_tokens(const Kn& k, uint16_t* tt, uint32_t W) {
    static_assert(kMT <= 64u && kMTR <= 64u, "one lane per pass row");
    if (k.nu * W > k.b.tcap && threadIdx.x == 0u) raise_error(k.a.sync, SyncMap::make(), E_TOKTAB, 0u);
    // wave v takes units v, v + kWaves, ...: unit() takes a uniform index (it
    // reads the pass table through readfirstlane), lane m the pass row m
    const uint32_t v = uni(threadIdx.x >> 6), m = threadIdx.x & 63u;
    constexpr uint32_t R = 4;  // units per wave whose loads are in flight together
    for (uint32_t i0 = 0; i0 < k.nu; i0 += R * kWaves) {
        uint32_t ent[R];
        bool has[R];
#pragma unroll
        for (uint32_t r = 0; r < R; r++) {
            const uint32_t i = i0 + v + kWaves * r;
            has[r] = false;
            ent[r] = 0u;
            if (i < k.nu) {
                const auto x = k.unit(i);
                has[r] = x.live && !x.sh && x.e != k.a.E && m < x.nt;
                if (has[r]) ent[r] = k.b.ent[x.row0 + m];
            }
        }
#pragma unroll
        for (uint32_t r = 0; r < R; r++) {
            const uint32_t i = i0 + v + kWaves * r;
            if (i < k.nu && m < W && W * i + m < k.b.tcap) tt[W * i + m] = (uint16_t)(has[r] ? ent[r] / k.K : 0u);
        }
    }
    lds_barrier();
}
// The token of row m (< nt) of this work-group's unit i.
WL_DEV uint32_t table_token(const uint16_t* tt, uint32_t cap, uint32_t W, uint32_t i, uint32_t m, uint32_t nt) {
    const uint32_t idx = W * i + min(m, nt - 1u);
    return idx < cap ? (uint32_t)tt[idx] : 0u;
}

// ---- grouped GEMMs ------------------------------------------------------------
// A unit is one token pass (up to kMT tokens: rows [row0, row0 + nt) of a
// [rows][3][kdim] bf16 piece array) times a block of weight rows, run in nst
// steps of kKC columns. A work-group walks its units u = blockIdx.x + G i as
// one flat sequence of steps z, so the pipeline runs across unit boundaries.
// Step z:
//   1. load the weights of step z + 2 into register buffer (z + 2) % 3;
//   2. wait until this wave's loads of step z (issued two steps ago) have
//      landed, barrier: every wave's activation DMAs of step z have landed,
//      and every wave is done with step z - 1;
//   3. DMA the activations of step z + 2 (buffer_load ... lds, no registers)
//      into slot (z + 2) % 3, the slot step z - 1 read;
//   4. compute step z from slot z % 3 and buffer z % 3; after a unit's last
//      step, its epilogue.
// Loads complete in issue order, so 2 is "at most kAfter loads outstanding":
// the weights of steps z + 1 and z + 2 and the activations of step z + 1 stay
// in flight (a load under full load takes several microseconds, a step
// less). The slots are separate LDS objects, so the compiler's own waits for
// DMA-written LDS stay per slot. (Spreading the loads through the compute
// instead, to avoid the eight waves issuing at once, makes the compiler wait
// for them early: it loses track of which buffer is outstanding.)
constexpr uint32_t kRows = 3u * kMT;            // LDS rows of a step
constexpr uint32_t kRowB = kKC * 2u;            // bytes of a staged row
constexpr uint32_t kSlotB = kRows * kRowB;      // 48 KB
constexpr uint32_t kDma = kRows / 2u / kWaves;  // DMA instructions per wave per step (1 KB = 2 rows each)
constexpr uint32_t kWL = 8;                     // 16-byte weight loads per step
constexpr uint32_t kSL = 1;                     // 8-byte scale loads per step (NativeLayout::bgus / bdns)
constexpr uint32_t kOOBV = 0x80000000u;  // a lane offset past every piece array (they stay below 2 GB)
static_assert(kRows % (2u * kWaves) == 0u, "DMA rows must split evenly over the waves");

// Slot layout: row R (512 bytes); its 16-byte group p holds columns
// [k0 + 8 (p ^ (R & 15)), +8) of the step, so the 16 rows an A fragment reads
// at one column fall in 16 different bank groups. Row R is (token m, piece
// pc): R = 4m + pc with pieces in rows, R = 32 pc + m with tokens in rows.
__shared__ __align__(16) uint8_t g_slot0[kSlotB];
__shared__ __align__(16) uint8_t g_slot1[kSlotB];
__shared__ __align__(16) uint8_t g_slot2[kSlotB];
template <int S>
WL_DEV uint8_t* slot() {
    return S == 0 ? g_slot0 : S == 1 ? g_slot1 : g_slot2;
}
// Lane (m, g) A fragment of row 32 pc + 16 tb + m at 16-byte column group
// cg = 16 hi + lo: the byte address splits into a uniform part and the lane
// part m * kRowB + 16 (lo ^ m) (lane_off), which the kernels precompute for
// the few lo they use.
WL_DEV uint32_t a_lane_off(uint32_t lo) {
    const uint32_t m = threadIdx.x & 15u;
    return m * kRowB + 16u * (lo ^ m);
}
WL_DEV bf16x8 afrag(const uint8_t* sl, uint32_t pc, uint32_t tb, uint32_t hi, uint32_t lane_off) {
    return as_bf16x8(*(const u32x4*)(sl + (pc * 32u + tb * 16u) * kRowB + 256u * hi + lane_off));
}

// Activation side of a unit: tokens [0, nt) of a pass, each a row of three
// pieces of kdim columns in a [rows][3][kdim] piece array (uniform values;
// dead: nt = 0). DMA instruction k of wave v writes slot rows 2j and 2j + 1
// (j = v + kWaves k; lanes 0-31 the first), so every row a lane writes has
// R & 15 = x = 2v + (lane >> 5): its 16-byte group (column group cg = p ^ x)
// is the same for every k, and per layout its token and piece are
//   pieces in rows: R = 4m + pc -> m = (x >> 2) + 4k, pc = x & 3 (a pass of
//                   at most kPR = 8 tokens: only k = 0, 1 have live rows);
//   tokens in rows: R = 32 pc + m -> m = x + 16 (k & 1), pc = k >> 1.
// Either way a lane's DMAs read two tokens' rows, at lane offsets base[k & 1]
// (the token's row, at piece x & 3 or 0), plus the uniform piece offset
// (k >> 1) kd2 with tokens in rows. The tokens' rows are consecutive rows of
// the array (a_bind) or any rows (a_bind_rows: a routed pass's tokens' rows
// of norm3, read in place).
struct AStream {
    rsrc_t rs;
    uint32_t base[2], nt, kd2;  // lane byte offsets of the two tokens' rows, tokens, bytes per piece row
    bool pr;
};
WL_DEV uint32_t a_x() { return 2u * uni(threadIdx.x >> 6) + ((threadIdx.x & 63u) >> 5); }
// The pass rows (tokens m0, m1 of the pass) this lane's DMAs write.
WL_DEV void a_rows(bool pr, uint32_t& m0, uint32_t& m1) {
    const uint32_t x = a_x();
    m0 = pr ? x >> 2 : x;
    m1 = pr ? (x >> 2) + 4u : x + 16u;
}
// row[j]: the array row of the lane's token m_j (a_rows).
WL_DEV void a_bind_rows(AStream& A, const uint16_t* base, uint64_t bytes, const uint32_t (&row)[2], uint32_t nt,
                        bool pr, uint32_t kdim) {
    A.rs = make_rsrc(base, (uint32_t)bytes);
    A.nt = nt;
    A.kd2 = 2u * kdim;
    A.pr = pr;
    const uint32_t x = a_x(), cg = (threadIdx.x & 31u) ^ x;
#pragma unroll
    for (uint32_t j = 0; j < 2; j++) A.base[j] = (row[j] * 3u + (pr ? x & 3u : 0u)) * A.kd2 + 16u * cg;
}
WL_DEV void a_bind(AStream& A, const uint16_t* base, uint64_t bytes, uint32_t row0, uint32_t nt, bool pr,
                   uint32_t kdim) {
    uint32_t m0, m1;
    a_rows(pr, m0, m1);
    const uint32_t row[2] = {row0 + m0, row0 + m1};
    a_bind_rows(A, base, bytes, row, nt, pr, kdim);
}
WL_DEV void a_none(AStream& A) { a_bind(A, nullptr, 0u, 0u, 0u, true, 0u); }
// DMA instruction k of one step (columns [k0, k0 + kKC)); absent rows
// (kOOBV) land as zeros.
template <int S>
WL_DEV void a_issue_one(const AStream& A, uint32_t k0, uint32_t k) {
    const uint32_t v = uni(threadIdx.x >> 6), x = a_x();
    const bool ok = A.pr ? (x >> 2) + 4u * k < A.nt && (x & 3u) < 3u : x + 16u * (k & 1u) < A.nt;
    const uint32_t so = 2u * k0 + (A.pr ? 0u : (k >> 1) * A.kd2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        A.rs, (__attribute__((address_space(3))) void*)(slot<S>() + (v + kWaves * k) * 2u * kRowB), 16u,
        ok ? A.base[k & 1u] : kOOBV, so, 0, 0);
}
template <int S>
WL_DEV void a_issue(const AStream& A, uint32_t k0) {
#pragma unroll
    for (uint32_t k = 0; k < kDma; k++) a_issue_one<S>(A, k0, k);
}

// ---- wide passes: 64 tokens, 128-column steps ----------------------------------
// The same slots hold 192 rows of 256 bytes: row R = 64 pc + m (token m,
// piece pc; tokens in rows only), its 16-byte group p holding columns
// [k0 + 8 (p ^ (R & 15)), +8). DMA instruction k of wave v writes rows 4j ..
// 4j + 3 (j = v + kWaves k; lanes 16r .. 16r + 15 row 4j + r), so a lane's
// rows are r0 + 32k with r0 = 4v + (lane >> 4) < 32: token r0 + 32 (k & 1),
// piece k >> 1, R & 15 = r0 & 15.
constexpr uint32_t kRowBW = 2u * kKCW;
static_assert(3u * kMTW * kRowBW == kSlotB, "a wide step fills one slot");
static_assert(3u * kMTW * kRowBW / 1024u / kWaves == kDma, "a wide step takes kDma DMAs per wave");
// A lane's two tokens r0 and r0 + 32 have lane offsets base[0], base[1]
// (their rows at piece 0: consecutive rows of the array, or any rows).
struct AStreamW {
    rsrc_t rs;
    uint32_t base[2], nt, kd2;  // lane byte offsets of the two tokens' rows, tokens, bytes per piece row
};
WL_DEV uint32_t aw_r0() { return 4u * uni(threadIdx.x >> 6) + ((threadIdx.x & 63u) >> 4); }
WL_DEV void aw_bind_rows(AStreamW& A, const uint16_t* base, uint64_t bytes, const uint32_t (&row)[2], uint32_t nt,
                         uint32_t kdim) {
    A.rs = make_rsrc(base, (uint32_t)bytes);
    A.nt = nt;
    A.kd2 = 2u * kdim;
    const uint32_t r0 = aw_r0(), cg = (threadIdx.x & 15u) ^ (r0 & 15u);
#pragma unroll
    for (uint32_t j = 0; j < 2; j++) A.base[j] = row[j] * 3u * A.kd2 + 16u * cg;
}
WL_DEV void aw_bind(AStreamW& A, const uint16_t* base, uint64_t bytes, uint32_t row0, uint32_t nt, uint32_t kdim) {
    const uint32_t r0 = aw_r0(), row[2] = {row0 + r0, row0 + r0 + 32u};
    aw_bind_rows(A, base, bytes, row, nt, kdim);
}
// The kDma DMAs of one wide step (columns [k0, k0 + kKCW)); absent rows land
// as zeros.
template <int S>
WL_DEV void aw_issue(const AStreamW& A, uint32_t k0) {
    const uint32_t v = uni(threadIdx.x >> 6), r0 = aw_r0();
#pragma unroll
    for (uint32_t k = 0; k < kDma; k++) {
        const bool ok = r0 + 32u * (k & 1u) < A.nt;
        const uint32_t so = 2u * k0 + (k >> 1) * A.kd2;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            A.rs, (__attribute__((address_space(3))) void*)(slot<S>() + (v + kWaves * k) * 1024u), 16u,
            ok ? A.base[k & 1u] : kOOBV, so, 0, 0);
    }
}
// Lane (m, g) A fragment of row 64 pc + 16 tb + m at column group cg (< 16):
// lane part m * kRowBW + 16 (cg ^ m).
WL_DEV uint32_t aw_lane_off(uint32_t cg) {
    const uint32_t m = threadIdx.x & 15u;
    return m * kRowBW + 16u * (cg ^ m);
}
// When cg = c0 | d with c0 per lane and d uniform in bits c0 never uses,
// aw_lane_off(cg) = aw_lane_off(c0) ^ 16 d: one base register per unit type
// and a constant per k step.
WL_DEV bf16x8 afragw(const uint8_t* sl, uint32_t pc, uint32_t tb, uint32_t lane_off) {
    return as_bf16x8(*(const u32x4*)(sl + (pc * kMTW + tb * 16u) * kRowBW + lane_off));
}
// The outputs of NB token blocks of a tile (tokens in rows): lane (n, g) calls
// f(m, value) for each live token m whose column-n value it holds.
template <uint32_t NB, class F>
WL_DEV void tile_each_w(const f32x4 (&acc)[NB], uint32_t nt, uint32_t lane, F f) {
    const uint32_t g = lane >> 4;
#pragma unroll
    for (uint32_t tb = 0; tb < NB; tb++) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t m = tb * 16u + 4u * g + i;
            if (m < nt) f(m, acc[tb][i]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}
// SwiGLU epilogue of a gate/up tile (columns n < 8 gate rows, n + 8 the
// matching up rows): put(m, n, value) for n < 8 and live tokens.
// One token block at a time (sched_barrier): interleaved over the blocks
// and tiles of a wide unit, the epilogue's temporaries do not fit beside the
// pipeline's registers.
template <uint32_t NB, class PutF>
WL_DEV void swiglu_store_w(const f32x4 (&acc)[NB], uint32_t nt, uint32_t lane, PutF put) {
    const uint32_t n = lane & 15u, g = lane >> 4;
#pragma unroll
    for (uint32_t tb = 0; tb < NB; tb++) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const float v = acc[tb][i];
            const float up = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
            const uint32_t m = tb * 16u + 4u * g + i;
            if (n < 8u && m < nt) put(m, n, silu_mul(v, up));
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}
// A value the compiler must treat as produced here: keeps the conversions of
// one k step in their iteration (pure conversions of a whole step are
// otherwise hoisted together, and their 64 results do not fit beside the
// wide units' accumulators).
WL_DEV uint32_t pinned(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}
struct WBufW {
    u32x4 w[8];
};

struct WBuf {
    u32x4 w[kWL];
    uint32_t s[2];  // the step's 8 scale bytes
};
WL_DEV void bld8(rsrc_t r, uint32_t voff, uint32_t soff, uint32_t (&s)[2]) {
    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0));
    s[0] = v.x;
    s[1] = v.y;
}

// Step 2: s_waitcnt vmcnt(N) (expcnt, lgkmcnt not waited on), barrier.
template <uint32_t N>
WL_DEV void step_barrier() {
    static_assert(N < 64u, "vmcnt is 6 bits");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((N & 15u) | ((N >> 4) << 14) | 0x0F70u);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Between two pipelines of one kernel: every load and DMA of the first has
// landed and every wave is done with its slots.
WL_DEV void pipeline_drain() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70u);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Position of a stream in the flat step sequence: my unit i, its step s.
struct Cursor {
    uint32_t i, s;
};
WL_DEV bool advance(Cursor& c, uint32_t nst) {
    if (++c.s < nst) return false;
    c.s = 0;
    c.i++;
    return true;
}
template <class Kn>
WL_DEV void issue_w(const Kn& k, uint32_t s, typename Kn::WB& W) {
#pragma unroll
    for (uint32_t j = 0; j < Kn::kLoads; j++) k.issue_w_one(s, W, j);
}
template <int S, class Kn>
WL_DEV void pipe_step(Kn& k, typename Kn::AS& A, const typename Kn::WB& cur, typename Kn::WB& nxt) {
    if (advance(k.cw, k.nst)) k.bind_w(k.cw.i);
    issue_w(k, k.cw.s, nxt);
    // loads issued after step z's activations: its weights' successors and
    // the activations of step z + 1
    step_barrier<kDma + 2u * Kn::kLoads>();
    // after the barrier every wave is done with step z - 1: its slot takes
    // the activations of step z + 2
    if (advance(k.ca, k.nst)) k.bind_a(k.ca.i, A);
    Kn::template issue_a<(S + 2) % 3>(A, k.ca.s);
    __builtin_amdgcn_sched_barrier(0);
    if (k.cc.i < k.nu) {
        if (k.cc.s == 0u) k.begin(k.cc.i);
        k.compute(k.cc.s, slot<S>(), cur);
        if (k.cc.s == k.nst - 1u) k.finish();
    }
    advance(k.cc, k.nst);
}
// Runs the pipeline over this work-group's nu units. Kn provides the types
// AS (activation stream) and WB (register buffer of one step's loads), kLoads
// (loads per step into a WB), nst, nu, the cursors ca/cw/cc and
// bind_a(i, A) / bind_w(i) (unit i >= nu: nothing to load),
// issue_w_one(s, W, j), issue_a<slot>(A, s) (kDma DMAs of step s),
// begin(i), compute(s, slot, W) and finish().
template <class Kn>
WL_DEV void run_steps(Kn& k) {
    if (k.nu == 0u) return;
    const uint32_t Z = k.nu * k.nst;
    typename Kn::AS A;
    typename Kn::WB B0, B1, B2;
    k.ca = k.cw = k.cc = Cursor{0u, 0u};
    k.bind_w(0u);
    issue_w(k, 0u, B0);
    k.bind_a(0u, A);
    Kn::template issue_a<0>(A, 0u);
    if (advance(k.cw, k.nst)) k.bind_w(k.cw.i);
    issue_w(k, k.cw.s, B1);
    if (advance(k.ca, k.nst)) k.bind_a(k.ca.i, A);
    Kn::template issue_a<1>(A, k.ca.s);
#pragma unroll 1
    for (uint32_t z = 0; z < Z; z += 3u) {
        pipe_step<0>(k, A, B0, B2);
        pipe_step<1>(k, A, B1, B0);
        pipe_step<2>(k, A, B2, B1);
    }
}

// Tables every GEMM work-group loads into LDS: the pass table and the
// layer's expert block pointers.
// With an MXFP4 shared expert, entry E is its block (NativeShared4::blk = 0).
WL_DEV const uint8_t* const* load_slot_tab(const DecodeArgs& a, uint32_t E, bool sh4, const uint8_t** s) {
    for (uint32_t f = threadIdx.x; f < E + (sh4 ? 1u : 0u); f += kThreads)
        s[f] = f < E ? gld(a.slot_tab + f) : a.sh_native;
    return s;  // visible after the barrier in load_pass_tab
}
// LDS of the tables for E experts and the MXFP4 shared pseudo-expert.
__host__ __device__ inline size_t gemm_tab_bytes(uint32_t E) { return 8u * (E + 1u) + 4u * (4u * (E + 1u) + 2u); }
// The gate/up kernel's token table follows them (16-byte aligned).
__host__ __device__ inline size_t tok_table_offset(uint32_t E) { return (gemm_tab_bytes(E) + 15u) & ~(size_t)15u; }
// The dynamic LDS of the kernel (every extern __shared__ array starts there).
WL_DEV uint8_t* dyn_lds() {
    extern __shared__ __align__(16) uint8_t dyn_base[];
    return dyn_base;
}

// Splits x into its three bf16 pieces at p[0], p[stride], p[2 stride].
WL_DEV void store3(uint16_t* p, uint32_t stride, float x) {
    uint32_t h, md, l;
    split3(x, h, md, l);
    gst(p, (uint16_t)h);
    gst(p + stride, (uint16_t)md);
    gst(p + 2u * stride, (uint16_t)l);
}

// A unit of a GEMM kernel: shared-expert units first (token passes of the
// batch), then the routed ones (expert passes of the pass table).
struct UnitInfo {
    bool live, sh;
    uint32_t e, part, nt, row0;
};

// ---- gate/up + SwiGLU ---------------------------------------------------------
// Shared unit (pass p, slice j): rows [64j, +64) of the shared gate and up
// (wave v: tile 8j + v, 8 bf16 per lane per 32-column k tile), K = H.
// Routed unit (expert pass, slice group sg): rows of kSG slices
// [64(kSG sg + i), +64) (wave v: tiles 8(kSG sg + i) + v, native gu chunks:
// 1 KB per 128-column k tile, one scale byte per k tile), K = H.
// Output: the SwiGLU values as pieces, smid3 / mid3 rows.
constexpr uint32_t kSG = 4;
static_assert(kWL == 2u * kSG && kSG == 4u, "gate/up step = 2 k tiles x 4 slices (one 8-byte scale word)");
struct UpK {
    using AS = AStream;
    using WB = WBuf;
    static constexpr uint32_t kLoads = kWL + kSL;
    template <int S>
    static __device__ __forceinline__ void issue_a(const AStream& A, uint32_t s) {
        a_issue<S>(A, s * kKC);
    }
    const DecodeArgs& a;
    const BatchArgs& b;
    uint32_t H, I, SI, E, K, nkg, nkt, S, NSG, Ssh, Us, nst, nu, v, lane, g;
    uint32_t uoff;  // unit u runs on work-group (u + uoff) % grid
    PassTab pt;
    const uint8_t* const* stab;
    NativeLayout NL;
    Cursor ca, cw, cc;
    // weight stream: the block and the scale stream's (null: none), kept as
    // pointers and sizes (see DownK)
    const uint8_t* wbase;
    const uint8_t* sbase;
    uint32_t wbytes, sbytes;
    bool wsh;
    uint32_t wpart, wvoff, vgu, vgus, vsh;
    // A fragment lane offsets: routed k step jj (cg = 16 q + 4 g + jj), shared
    // k tile k (cg = 4 k + g)
    uint32_t lo_r[4], lo_s[4];
    // compute unit
    UnitInfo cu;
    PassShape cps;
    uint32_t cvar;  // compute variant: 0/1 pieces in rows, 1/2 blocks; 2/3 tokens in rows, 1/2 blocks
    f32x4 acc[kSG][2];
    const uint16_t* tt;  // the token table (kMT entries per unit)

    WL_MEM UnitInfo unit(uint32_t i) const {
        UnitInfo x{false, false, 0u, 0u, 0u, 0u};
        if (i >= nu) return x;
        const uint32_t u = (blockIdx.x + gridDim.x - uoff) % gridDim.x + gridDim.x * i;
        x.live = true;
        if (u < Us) {
            const uint32_t p = u / Ssh;
            x.sh = true;
            x.part = u % Ssh;
            x.nt = min(kMT, b.T - p * kMT);
            x.row0 = p * kMT;
        } else {
            const PassPart jp = pass_part(u - Us, NSG, pt.n);
            const Pass ps = pass_at(pt, E, jp.j);
            x.part = jp.part;
            x.e = ps.e;
            x.nt = ps.nt;
            x.row0 = ps.c0;
        }
        return x;
    }
    WL_MEM void bind_a(uint32_t i, AStream& A) const {
        const UnitInfo x = unit(i);
        if (!x.live) return a_none(A);
        const bool pr = pass_shape(x.nt).pr;
        if (x.sh) a_bind(A, b.norm3, (uint64_t)b.T * 6u * H, x.row0, x.nt, pr, H);
        else if (x.e == a.E) a_bind(A, b.norm3, (uint64_t)b.T * 6u * H, x.row0 - b.T * K, x.nt, pr, H);  // MXFP4 shared
        else {
            uint32_t m0, m1;
            a_rows(pr, m0, m1);
            const uint32_t row[2] = {table_token(tt, b.tcap, kMT, i, m0, x.nt), table_token(tt, b.tcap, kMT, i, m1, x.nt)};
            a_bind_rows(A, b.norm3, (uint64_t)b.T * 6u * H, row, x.nt, pr, H);
        }
    }
    WL_MEM void bind_w(uint32_t i) {
        const UnitInfo x = unit(i);
        wsh = x.sh;
        wpart = x.part;
        const NativeShared NS = NativeShared::make(H, SI);
        const uint8_t* blk = x.live && !x.sh ? uni_ptr(stab[x.e]) : nullptr;
        wbase = !x.live ? nullptr : x.sh ? a.sh_native + NS.sgu : blk;
        wbytes = !x.live ? 0u : x.sh ? (uint32_t)(NS.sdn - NS.sgu) : blk ? (uint32_t)NL.total : 0u;
        sbase = x.live && !x.sh ? blk : nullptr;
        sbytes = x.live && !x.sh && blk ? (uint32_t)NL.total : 0u;
        wvoff = x.sh ? vsh : vgu;  // chosen here, not per load (see DownK::bind_w)
    }
    WL_MEM void issue_w_one(uint32_t s, WBuf& W, uint32_t j) const {
        if (j < kWL) {
            const uint32_t sl = min(wpart * kSG + j / 2u, S - 1u);
            const uint32_t ro = sl * 8u * nkg * 1024u + min(2u * s + j % 2u, nkg - 1u) * 1024u;
            const uint32_t so = wpart * 8u * nkt * 1024u + min(8u * s + j, nkt - 1u) * 1024u;
            W.w[j] = bld16_nt(make_rsrc(wbase, wbytes), wvoff, wsh ? so : ro);
        } else {
            bld8(make_rsrc(sbase, sbytes), vgus, (wpart * 8u * nst + s) * 512u, W.s);
        }
    }
    WL_MEM void begin(uint32_t i) {
        cu = unit(i);
        cps = pass_shape(cu.nt);
        cvar = (cps.pr ? 0u : 2u) + cps.nblk - 1u;
        if (!cu.sh && stab[cu.e] == nullptr && threadIdx.x == 0) raise_error(a.sync, SyncMap::make(), E_NOT_RESIDENT, 0u);  // no waits in this path: epoch 0 aborts nothing
#pragma unroll
        for (uint32_t j = 0; j < kSG; j++) acc[j][0] = acc[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // One step for a pass of NB row blocks and NP planes (shape-specialised
    // so the inner loops carry no branches).
    //
    // Shared: one MFMA per activation fragment, all on this wave's one weight
    // tile. MFMA it (k step k, plane pc, block tb) accumulates into
    // acc[(NP k + pc) % 4][tb], so consecutive MFMAs of a block do not wait on
    // each other; finish() adds the four. Fragments are read kSPD MFMAs ahead
    // (LDS latency is not hidden by the one other wave of the SIMD otherwise).
    static constexpr uint32_t kSPD = 6;
    template <uint32_t NB, uint32_t NP>
    WL_MEM void comp_shared(uint32_t s, const uint8_t* sl, const WBuf& W) {
        constexpr uint32_t N = 8u * NP * NB;
        bf16x8 af[kSPD + 1u];
        auto frag = [&](uint32_t it) {  // it = (k NP + pc) NB + tb
            const uint32_t tb = it % NB, pc = (it / NB) % NP, k = it / (NB * NP);
            return afrag(sl, pc, tb, k / 4u, lo_s[k % 4u]);
        };
#pragma unroll
        for (uint32_t it = 0; it < kSPD && it < N; it++) af[it] = frag(it);
#pragma unroll
        for (uint32_t it = 0; it < N; it++) {
            const uint32_t tb = it % NB, kp = it / NB, k = kp / NP;
            if (it + kSPD < N) af[(it + kSPD) % (kSPD + 1u)] = frag(it + kSPD);
            const u32x4 z = {0u, 0u, 0u, 0u};
            const bf16x8 bw = as_bf16x8(8u * s + k < nkt ? W.w[k] : z);
            acc[kp % 4u][tb] = mma(af[it % (kSPD + 1u)], bw, acc[kp % 4u][tb]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Routed: iteration it = NP (4 q + jj) + pc runs plane pc of k step
    // (q, jj) (columns q * 128 + 32 g + 8 jj) against the kSG slices; the
    // next iteration's NB fragments are read while this one's MFMAs run.
    template <uint32_t NB, uint32_t NP>
    WL_MEM void comp_routed(uint32_t s, const uint8_t* sl, const WBuf& W) {
        float sc[2][kSG];
#pragma unroll
        for (uint32_t q = 0; q < 2; q++)
#pragma unroll
            for (uint32_t i = 0; i < kSG; i++)
                sc[q][i] = e8m0f_if((W.s[i >> 1] >> (8u * (2u * (i & 1u) + q))) & 0xFFu, 2u * s + q < nkg);
        constexpr uint32_t N = 8u * NP;
        bf16x8 af[2][NB];
#pragma unroll
        for (uint32_t tb = 0; tb < NB; tb++) af[0][tb] = afrag(sl, 0u, tb, 0u, lo_r[0]);
        bf16x8 bw[kSG];
#pragma unroll
        for (uint32_t it = 0; it < N; it++) {
            const uint32_t pc = it % NP, ks = it / NP, q = ks / 4u, jj = ks % 4u, c = it % 2u;
            if (it + 1u < N) {
                const uint32_t n = it + 1u, nks = n / NP;
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) af[c ^ 1u][tb] = afrag(sl, n % NP, tb, nks / 4u, lo_r[nks % 4u]);
            }
            if (pc == 0u) {
#pragma unroll
                for (uint32_t i = 0; i < kSG; i++) bw[i] = fp4x8_bf16(W.w[2u * i + q][jj], sc[q][i]);
            }
#pragma unroll
            for (uint32_t i = 0; i < kSG; i++)
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) acc[i][tb] = mma(af[c][tb], bw[i], acc[i][tb]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    WL_MEM void compute(uint32_t s, const uint8_t* sl, const WBuf& W) {
        switch (cvar) {
            case 0: return cu.sh ? comp_shared<1, 1>(s, sl, W) : comp_routed<1, 1>(s, sl, W);
            case 1: return cu.sh ? comp_shared<2, 1>(s, sl, W) : comp_routed<2, 1>(s, sl, W);
            case 2: return cu.sh ? comp_shared<1, 3>(s, sl, W) : comp_routed<1, 3>(s, sl, W);
            default: return cu.sh ? comp_shared<2, 3>(s, sl, W) : comp_routed<2, 3>(s, sl, W);
        }
    }
    WL_MEM void finish() {
        const uint32_t ln = opaque_lane();
        if (cu.sh) {
#pragma unroll
            for (uint32_t tb = 0; tb < 2; tb++) acc[0][tb] = (acc[0][tb] + acc[1][tb]) + (acc[2][tb] + acc[3][tb]);
            swiglu_store(acc[0], cu.nt, cps.pr, ln, [&](uint32_t m, uint32_t n, float x) {
                store3(b.smid3 + (size_t)(cu.row0 + m) * 3u * SI + cu.part * kSlice + v * 8u + n, SI, x);
            });
            return;
        }
#pragma unroll
        for (uint32_t i = 0; i < kSG; i++) {
            const uint32_t sl = cu.part * kSG + i;
            if (sl >= S) continue;
            swiglu_store(acc[i], cu.nt, cps.pr, ln, [&](uint32_t m, uint32_t n, float x) {
                store3(b.mid3 + (size_t)(cu.row0 + m) * 3u * I + sl * kSlice + v * 8u + n, I, x);
            });
        }
    }
};
// Shared gate/up in wide passes (batches of more than kMT tokens): unit
// (pass p of kMTW tokens, slice pair j): wave v owns tiles T_i = 8 (2j + i) + v
// (i = 0, 1); step s covers columns [128 s, +128): per tile the native sgu
// chunks (T_i, 4s + k), k < 4 (lane (n, g): row n, columns [32 kt + 8 g, +8)).
// A work-group step moves 64 KB of weights and 48 KB of activations for 768
// MFMAs (a kMT unit: the same bytes for 384), and each A fragment feeds two
// tiles.
struct SharedUpW {
    using AS = AStreamW;
    using WB = WBufW;
    static constexpr uint32_t kLoads = 8;
    template <int S>
    static __device__ __forceinline__ void issue_a(const AStreamW& A, uint32_t s) {
        aw_issue<S>(A, s * kKCW);
    }
    const DecodeArgs& a;
    const BatchArgs& b;
    uint32_t H, SI, nkt, nsl, npair, npass, nst, nu, v, lane;
    Cursor ca, cw, cc;
    const uint8_t* wbase;  // the weight stream's block and size (see DownK)
    uint32_t wbytes;
    uint32_t wpair, vbase;
    uint32_t lob;  // A fragment lane offset of k step 0 (cg = g; k step k: ^ 64 k)
    uint32_t cpair, cnt, crow0, cnb;
    f32x4 acc[2][4];

    struct Unit {
        bool live;
        uint32_t pair, nt, row0;
    };
    WL_MEM Unit unit(uint32_t i) const {
        Unit x{false, 0u, 0u, 0u};
        if (i >= nu) return x;
        const PassPart jp = pass_part(blockIdx.x + gridDim.x * i, npair, npass);
        x.live = true;
        x.pair = jp.part;
        x.row0 = jp.j * kMTW;
        x.nt = min(kMTW, b.T - x.row0);
        return x;
    }
    WL_MEM void bind_a(uint32_t i, AStreamW& A) const {
        const Unit x = unit(i);
        if (!x.live) return aw_bind(A, nullptr, 0u, 0u, 0u, 0u);
        aw_bind(A, b.norm3, (uint64_t)b.T * 6u * H, x.row0, x.nt, H);
    }
    WL_MEM void bind_w(uint32_t i) {
        const Unit x = unit(i);
        const NativeShared NS = NativeShared::make(H, SI);
        wbase = x.live ? a.sh_native + NS.sgu : nullptr;
        wbytes = x.live ? (uint32_t)(NS.sdn - NS.sgu) : 0u;
        wpair = x.pair;
    }
    WL_MEM void issue_w_one(uint32_t s, WBufW& W, uint32_t j) const {
        const uint32_t T = 8u * min(2u * wpair + j / 4u, nsl - 1u) + v;
        W.w[j] = bld16(make_rsrc(wbase, wbytes), vbase, (T * nkt + 4u * s + j % 4u) * 1024u);  // re-read by every pass: cached
    }
    WL_MEM void begin(uint32_t i) {
        const Unit x = unit(i);
        cpair = x.pair;
        cnt = x.nt;
        crow0 = x.row0;
        cnb = cdiv(x.nt, 16u);
#pragma unroll
        for (uint32_t t = 0; t < 2; t++)
#pragma unroll
            for (uint32_t tb = 0; tb < 4; tb++) acc[t][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // Iteration it = 3 k + pc: plane pc of k step k against both tiles; the
    // next iteration's NB fragments are read while this one's MFMAs run.
    template <uint32_t NB>
    WL_MEM void comp(const uint8_t* sl, const WBufW& W) {
        bf16x8 af[2][NB];
#pragma unroll
        for (uint32_t tb = 0; tb < NB; tb++) af[0][tb] = afragw(sl, 0u, tb, lob);
#pragma unroll
        for (uint32_t it = 0; it < 12u; it++) {
            const uint32_t k = it / 3u, c = it & 1u;
            if (it + 1u < 12u) {
                const uint32_t nx = it + 1u;
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) af[c ^ 1u][tb] = afragw(sl, nx % 3u, tb, lob ^ (64u * (nx / 3u)));
            }
#pragma unroll
            for (uint32_t t = 0; t < 2; t++) {
                const bf16x8 bw = as_bf16x8(W.w[4u * t + k]);
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) acc[t][tb] = mma(af[c][tb], bw, acc[t][tb]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    WL_MEM void compute(uint32_t, const uint8_t* sl, const WBufW& W) {
        switch (cnb) {
            case 1: return comp<1>(sl, W);
            case 2: return comp<2>(sl, W);
            case 3: return comp<3>(sl, W);
            default: return comp<4>(sl, W);
        }
    }
    WL_MEM void finish() {
        const uint32_t ln = opaque_lane();
#pragma unroll
        for (uint32_t t = 0; t < 2; t++) {
            const uint32_t sl = 2u * cpair + t;
            if (sl >= nsl) continue;
            const uint32_t col = 8u * (8u * sl + v);
            swiglu_store_w(acc[t], cnt, ln, [&](uint32_t m, uint32_t n, float x) {
                store3(b.smid3 + (size_t)(crow0 + m) * 3u * SI + col + n, SI, x);
            });
        }
    }
};
// The shared expert's wide-pass units (kBatchWideSharedUp: launch_batched
// sets it when there are at least as many as work-groups; a wide unit is
// about three routed units of work, so with fewer of them than work-groups
// the ones that hold one end last: measured slower at T = 64 and 256, 3.8 %
// faster per call at T = 1024); returns their count.
template <bool GLM>
WL_DEV uint32_t run_shared_up_wide(const DecodeArgs& a, const BatchArgs& b) {
    if (!(b.flags & kBatchWideSharedUp)) return 0u;
    const uint32_t H_ = GLM ? 6144u : a.H, I_ = GLM ? 2048u : a.I, SI_ = GLM ? 2048u : a.SI, K_ = GLM ? 8u : a.K;
    (void)I_;
    (void)K_;
    SharedUpW w{a, b};
    w.H = H_;
    w.SI = SI_;
    w.nkt = H_ / 32u;
    w.nsl = SI_ / kSlice;
    w.npair = cdiv(w.nsl, 2u);
    w.npass = cdiv(b.T, kMTW);
    w.nst = H_ / kKCW;
    const uint32_t U = w.npass * w.npair;
    w.nu = U > blockIdx.x ? cdiv(U - blockIdx.x, gridDim.x) : 0u;
    w.lane = threadIdx.x & 63u;
    w.v = uni(threadIdx.x >> 6);
    w.vbase = 16u * w.lane;
    w.lob = aw_lane_off(w.lane >> 4);
    run_steps(w);
    return U;
}
// Routed gate/up in wide passes (an expert of more than kMT tokens): unit
// (pass of kMTW tokens, slice group sg): wave v owns the tiles of a kMT unit,
// 8 (kSG sg + i) + v (i < kSG); step s covers columns [128 s, +128): one
// native gu chunk (tile, s) per tile and the batched scale word of the
// 256-column step s / 2 (bytes 2i + (s & 1)). A work-group step moves 32 KB of
// weights and 48 KB of activations for 1536 MFMAs (a kMT unit: 64 + 48 KB),
// and an expert's weights are read once per 64 of its tokens.
struct RoutedUpW {
    using AS = AStreamW;
    struct WB {
        u32x4 w[kSG];
        uint32_t s[2];
    };
    static constexpr uint32_t kLoads = kSG + 1u;
    template <int S>
    static __device__ __forceinline__ void issue_a(const AStreamW& A, uint32_t s) {
        aw_issue<S>(A, s * kKCW);
    }
    const DecodeArgs& a;
    const BatchArgs& b;
    uint32_t H, I, E, K, nkg, S, NSG, nst, nst2, nu, v, lane, uoff;
    PassTab pt;
    const uint8_t* const* stab;
    NativeLayout NL;
    Cursor ca, cw, cc;
    const uint8_t* wbase;  // the weight stream's block and size (see DownK)
    uint32_t wbytes;
    uint32_t wpart, vgu, vgus;
    uint32_t lob;  // A fragment lane offset of k step 0 (cg = 4g; k step jj: ^ 16 jj)
    UnitInfo cu;
    uint32_t cnb;
    f32x4 acc[kSG][3];
    const uint16_t* tt;  // the token table (kMTR entries per unit)

    WL_MEM UnitInfo unit(uint32_t i) const {
        UnitInfo x{false, false, 0u, 0u, 0u, 0u};
        if (i >= nu) return x;
        const uint32_t r = (blockIdx.x + gridDim.x - uoff) % gridDim.x + gridDim.x * i;
        const PassPart jp = pass_part(r, NSG, pt.nw);
        const Pass ps = pass_at_w(pt, E, jp.j);
        x.live = true;
        x.part = jp.part;
        x.e = ps.e;
        x.nt = ps.nt;
        x.row0 = ps.c0;
        return x;
    }
    WL_MEM void bind_a(uint32_t i, AStreamW& A) const {
        const UnitInfo x = unit(i);
        if (!x.live) return aw_bind(A, nullptr, 0u, 0u, 0u, 0u);
        if (x.e == a.E) aw_bind(A, b.norm3, (uint64_t)b.T * 6u * H, x.row0 - b.T * K, x.nt, H);  // MXFP4 shared
        else {
            const uint32_t r0 = aw_r0();
            const uint32_t row[2] = {table_token(tt, b.tcap, kMTR, i, r0, x.nt),
                                     table_token(tt, b.tcap, kMTR, i, r0 + 32u, x.nt)};
            aw_bind_rows(A, b.norm3, (uint64_t)b.T * 6u * H, row, x.nt, H);
        }
    }
    WL_MEM void bind_w(uint32_t i) {
        const UnitInfo x = unit(i);
        const uint8_t* blk = x.live ? uni_ptr(stab[x.e]) : nullptr;
        wbase = blk;
        wbytes = blk ? (uint32_t)NL.total : 0u;
        wpart = x.part;
    }
    WL_MEM void issue_w_one(uint32_t s, WB& W, uint32_t j) const {
        if (j < kSG) {
            const uint32_t sl = min(wpart * kSG + j, S - 1u);
            W.w[j] = bld16_nt(make_rsrc(wbase, wbytes), vgu, sl * 8u * nkg * 1024u + s * 1024u);
        } else {
            bld8(make_rsrc(wbase, wbytes), vgus, (wpart * 8u * nst2 + s / 2u) * 512u, W.s);
        }
    }
    WL_MEM void begin(uint32_t i) {
        cu = unit(i);
        cnb = cdiv(cu.nt, 16u);
        if (stab[cu.e] == nullptr && threadIdx.x == 0) raise_error(a.sync, SyncMap::make(), E_NOT_RESIDENT, 0u);
#pragma unroll
        for (uint32_t t = 0; t < kSG; t++)
#pragma unroll
            for (uint32_t tb = 0; tb < 3; tb++) acc[t][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // Iteration it = NH (3 jj + pc) + hp: plane pc of k step jj (columns
    // 32 g + 8 jj of the step's k tile), token blocks 2 hp and 2 hp + 1,
    // against the kSG tiles; the next iteration's two fragments are read while
    // this one's MFMAs run (two at a time: four would not fit beside the 64
    // accumulator registers).
    template <uint32_t NB>
    WL_MEM void comp(uint32_t s, const uint8_t* sl, const WB& W) {
        constexpr uint32_t NH = (NB + 1u) / 2u, N = 12u * NH;
        float sc[kSG];
#pragma unroll
        for (uint32_t i = 0; i < kSG; i++) sc[i] = e8m0f((W.s[i >> 1] >> (8u * (2u * (i & 1u) + (s & 1u)))) & 0xFFu);
        auto frag = [&](uint32_t it, uint32_t t2) {
            const uint32_t kp = it / NH, tb = 2u * (it % NH) + t2;
            return afragw(sl, kp % 3u, tb < NB ? tb : NB - 1u, lob ^ (16u * (kp / 3u)));
        };
        bf16x8 af[2][2], bw[kSG];
        af[0][0] = frag(0u, 0u);
        af[0][1] = frag(0u, 1u);
#pragma unroll
        for (uint32_t it = 0; it < N; it++) {
            const uint32_t kp = it / NH, hp = it % NH, jj = kp / 3u, pc = kp % 3u, c = it & 1u;
            if (it + 1u < N) {
                af[c ^ 1u][0] = frag(it + 1u, 0u);
                af[c ^ 1u][1] = frag(it + 1u, 1u);
            }
            if (pc == 0u && hp == 0u) {
#pragma unroll
                for (uint32_t i = 0; i < kSG; i++) bw[i] = fp4x8_bf16(pinned(W.w[i][jj]), sc[i]);
            }
#pragma unroll
            for (uint32_t i = 0; i < kSG; i++)
#pragma unroll
                for (uint32_t t2 = 0; t2 < 2; t2++)
                    if (2u * hp + t2 < NB) acc[i][2u * hp + t2] = mma(af[c][t2], bw[i], acc[i][2u * hp + t2]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    WL_MEM void compute(uint32_t s, const uint8_t* sl, const WB& W) {
        switch (cnb) {
            case 1: return comp<1>(s, sl, W);
            case 2: return comp<2>(s, sl, W);
            default: return comp<3>(s, sl, W);
        }
    }
    WL_MEM void finish() {
        const uint32_t ln = opaque_lane();
#pragma unroll
        for (uint32_t i = 0; i < kSG; i++) {
            const uint32_t sl = cu.part * kSG + i;
            if (sl >= S) continue;
            swiglu_store_w(acc[i], cu.nt, ln, [&](uint32_t m, uint32_t n, float x) {
                store3(b.mid3 + (size_t)(cu.row0 + m) * 3u * I + sl * kSlice + v * 8u + n, I, x);
            });
        }
    }
};
// The wide passes of the routed experts, as one pipeline starting at work-group
// uoff; returns their unit count.
template <bool GLM>
WL_DEV uint32_t run_routed_up_wide(const DecodeArgs& a, const BatchArgs& b, const PassTab& pt,
                                   const uint8_t* const* stab, uint32_t E, uint32_t uoff) {
    if (pt.nw == 0u) return 0u;
    const uint32_t H_ = GLM ? 6144u : a.H, I_ = GLM ? 2048u : a.I, SI_ = GLM ? 2048u : a.SI, K_ = GLM ? 8u : a.K;
    (void)I_;
    (void)K_;
    RoutedUpW w{a, b};
    w.H = H_;
    w.I = I_;
    w.E = E;
    w.K = K_;
    w.nkg = H_ / 128u;
    w.S = I_ / kSlice;
    w.NSG = cdiv(w.S, kSG);
    w.nst = w.nkg;
    w.nst2 = cdiv(H_, kKC);
    w.uoff = uoff;
    const uint32_t U = pt.nw * w.NSG, b0 = (blockIdx.x + gridDim.x - uoff) % gridDim.x;
    w.nu = U > b0 ? cdiv(U - b0, gridDim.x) : 0u;
    w.lane = threadIdx.x & 63u;
    w.v = uni(threadIdx.x >> 6);
    w.pt = pt;
    w.stab = stab;
    w.NL = NativeLayout::make(H_, I_);
    w.vgu = (uint32_t)w.NL.gu + w.v * w.nkg * 1024u + 16u * w.lane;
    w.vgus = (uint32_t)w.NL.bgus + w.v * w.nst2 * 512u + 8u * w.lane;
    w.lob = aw_lane_off(4u * (w.lane >> 4));
    uint16_t* tt = (uint16_t*)(dyn_lds() + tok_table_offset(a.E));
    w.tt = tt;
    fill_tokens(w, tt, kMTR);
    run_steps(w);
    return U;
}
// ---- routed gate/up of small experts -----------------------------------------
// Experts with 1..kSmallUpT tokens run their gate/up as streaming units, like
// the decode kernel's gate/up phase: unit (expert, part of kSG slices), in two
// pipelines, NB = 1 for 1-4 tokens and NB = 2 for 5-8 (MFMA row blocks of
// pieces in rows: token m's pieces in rows 4m..4m+2). The three LDS slots
// hold the unit's tokens' pieces for K = H = 6144 in NCH chunks of CW
// columns, chunk c in slot c mod 3 (NB = 1: 3 chunks of 2048 columns, 12
// stored rows of 4 KB; NB = 2: 6 chunks of 1024 columns, 24 rows of 2 KB;
// either way 48 KB per slot). Stored row Rs = 3m + pc; its 16-byte group p
// holds logical group p ^ (Rs & 15), so the 16 rows an A fragment reads at
// one column fall in different bank groups. MFMA row 16 tb + n reads stored
// row 3m + min(pc, 2) for m = 4 tb + n / 4, pc = n % 4 (rows 4m + 3 and
// tokens past nt carry values no output reads). Each wave streams its tiles
// of the unit's kSG slices (the GEMM kernel's native gu chunks and batched
// scale words) two 256-column steps ahead with no barrier inside a chunk; at
// each chunk boundary the waves meet once, and the slot the last chunk used
// takes the chunk two ahead (of this unit or the next) by DMA, so a chunk's
// rows are in LDS at least two chunks before its steps read them. The
// per-step arithmetic is the GEMM kernel's for a pass of pieces in rows, so
// the results are the same bits. The lists (expert, its tokens, first
// compact entry, count) live where the pass table was, after the GEMM
// pipelines.
constexpr uint32_t kSmallUpT = 8;  // tokens of the largest expert the streaming units take (gate/up and down)
__host__ __device__ inline bool small_up_fits(uint32_t H, uint32_t I) {
    return H == 6144u && I % (kSlice * kSG) == 0u;
}
struct SmallExp {
    uint16_t tok[kSmallUpT];
    uint16_t c0, nt;
    uint32_t e;
};
static_assert(sizeof(SmallExp) == 24u, "24 bytes per small expert");
// LDS the small-expert list needs from the pass table's start (8 E bytes
// into the dynamic LDS), for E routed experts.
__host__ __device__ inline size_t small_list_end(uint32_t E) { return 8u * (E + 1u) + sizeof(SmallExp) * E + 64u; }
// The experts with lo..hi tokens (ascending), into se; returns their count.
// wcnt: kWaves words of LDS.
WL_DEV uint32_t small_list(const DecodeArgs& a, const BatchArgs& b, const uint8_t* const* stab, uint32_t lo,
                           uint32_t hi, uint32_t K, SmallExp* se, uint32_t* wcnt) {
    const uint32_t E = a.E, lane = threadIdx.x & 63u, v = uni(threadIdx.x >> 6);
    const bool skip = (b.flags & kBatchSkipUnbound) != 0u;
    auto is_small = [&](uint32_t e, uint32_t c) { return c >= lo && c <= hi && !(skip && stab[e] == nullptr); };
    // wave v takes experts v, v + 8, ... in blocks of 64 (ballot order within
    // a block), the blocks' counts summed in LDS
    uint32_t run = 0;
    for (uint32_t e0 = 64u * v; e0 < E; e0 += 64u * kWaves) {
        const uint32_t e = e0 + lane, c = e < E ? gld(b.counts + e) : 0u;
        run += (uint32_t)__popcll(__ballot(e < E && is_small(e, c)));
    }
    if (lane == 0u) wcnt[v] = run;
    lds_barrier();
    uint32_t base = 0, ns = 0;
    for (uint32_t w = 0; w < kWaves; w++) {
        const uint32_t c = uni(wcnt[w]);
        base += w < v ? c : 0u;
        ns += c;
    }
    run = base;
    for (uint32_t e0 = 64u * v; e0 < E; e0 += 64u * kWaves) {
        const uint32_t e = e0 + lane, c = e < E ? gld(b.counts + e) : 0u;
        const bool sm = e < E && is_small(e, c);
        const uint64_t bal = __ballot(sm);
        if (sm) {
            SmallExp x;
            const uint32_t c0 = gld(b.offsets + e);
#pragma unroll
            for (uint32_t m = 0; m < kSmallUpT; m++) x.tok[m] = (uint16_t)(gld(b.ent + c0 + min(m, c - 1u)) / K);
            x.c0 = (uint16_t)c0;
            x.nt = (uint16_t)c;
            x.e = e;
            se[run + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull))] = x;
        }
        run += (uint32_t)__popcll(bal);
    }
    lds_barrier();
    return ns;
}
// Units are taken from a work queue (b.wq[NB - 1], an agent-scope counter
// that every work-group increments): a work-group that ends its grouped
// passes early takes more units. Wave 0 takes the next unit at the current
// unit's first chunk boundary and publishes it in LDS (qs) at the boundary
// where the next unit's first DMA goes out, so the take's round trip is
// hidden behind a chunk of steps and no work-group holds more than one unit
// ahead when the queue runs dry.
// An agent-scope fetch-add through an address the compiler cannot tell is
// uniform: a uniform one is rewritten into a wave-level atomic whose result
// is waited for at once (vmcnt(0)), which would drain the weight stream.
WL_DEV uint32_t take_next(uint32_t* p) {
    uint32_t z = 0u;
    asm volatile("" : "+v"(z));
    return __hip_atomic_fetch_add((g_u32*)(p + z), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <uint32_t NB>
WL_DEV void run_small_up(const DecodeArgs& a, const BatchArgs& b, const SmallExp* se, uint32_t ns,
                         const uint8_t* const* stab, uint32_t* qs) {
    constexpr uint32_t H = 6144u, CW = NB == 1u ? 2048u : 1024u, NCH = H / CW, SPC = CW / kKC, RB = 2u * CW;
    constexpr uint32_t ROWS = 12u * NB, SEGS = RB / 1024u;
    static_assert(ROWS * RB == kSlotB && ROWS * SEGS == 6u * kWaves, "a chunk fills one slot in six DMAs per wave");
    static_assert(NCH * SPC == 24u && NCH >= 3u, "24 steps of 256 columns, at least three chunks");
    const uint32_t I = a.I;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, v = uni(tid >> 6), n = lane & 15u, g = lane >> 4;
    const uint32_t S = I / kSlice, NSG = cdiv(S, kSG), U = ns * NSG, G = gridDim.x;
    const uint32_t nkg = H / 128u, nst = H / kKC;  // 128-column k tiles, 256-column steps
    const NativeLayout NL = NativeLayout::make(H, I);
    const uint32_t vgu = (uint32_t)NL.gu + v * nkg * 1024u + 16u * lane;
    const uint32_t vgus = (uint32_t)NL.bgus + v * nst * 512u + 8u * lane;
    const rsrc_t nrs = make_rsrc(b.norm3, b.T * 6u * H);
    // A fragment of lane (n, g), row block tb: stored row of MFMA row
    // 16 tb + n, logical groups 32 s + 16 q + 4 g + jj of the chunk
    uint32_t lo[NB][4];
#pragma unroll
    for (uint32_t tb = 0; tb < NB; tb++) {
        const uint32_t rs = 3u * (4u * tb + (n >> 2)) + min(n & 3u, 2u);
#pragma unroll
        for (uint32_t jj = 0; jj < 4; jj++) lo[tb][jj] = rs * RB + 16u * ((4u * g + jj) ^ (rs & 15u));
    }
    struct Unit {
        const uint8_t* blk;
        uint32_t part, c0, nt;
        uint32_t tok[4u * NB];
        bool live;
    };
    auto unit = [&](uint32_t r, Unit& x) {
        x.blk = nullptr;
        x.part = 0u;
        x.c0 = 0u;
        x.nt = 0u;
        x.live = r < U;
        if (r >= U) return;
        const SmallExp* q = se + r / NSG;
        x.part = r % NSG;
        x.blk = uni_ptr(stab[uni(q->e)]);
        x.c0 = uni(q->c0);
        x.nt = uni(q->nt);
#pragma unroll
        for (uint32_t m = 0; m < 4u * NB; m++) x.tok[m] = uni(q->tok[m]);
    };
    auto slot_c = [](uint32_t C) { return C == 0u ? slot<0>() : C == 1u ? slot<1>() : slot<2>(); };
    // DMA of unit x's chunk c into slot c mod 3: instruction k of wave v
    // writes segment q = v + kWaves k (stored row q / SEGS, its 1 KB part
    // q % SEGS)
    auto dma = [&](uint32_t c, const Unit& x) {
#pragma unroll
        for (uint32_t k = 0; k < 6u; k++) {
            const uint32_t q = v + kWaves * k, rs = q / SEGS, seg = q % SEGS, m = rs / 3u, pc = rs % 3u;
            const bool ok = x.blk != nullptr && m < x.nt;
            uint32_t t = x.tok[0];
#pragma unroll
            for (uint32_t j = 1; j < 4u * NB; j++) t = m == j ? x.tok[j] : t;
            const uint32_t so = ((t * 3u + pc) * H + c * CW) * 2u + seg * 1024u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                nrs, (__attribute__((address_space(3))) void*)(slot_c(c % 3u) + rs * RB + seg * 1024u), 16u,
                ok ? 16u * (lane ^ (rs & 15u)) : kOOBV, ok ? so : 0u, 0, 0);
        }
    };
    struct WB {
        u32x4 w[kWL];
        uint32_t s[2];
    };
    auto issue = [&](const Unit& x, uint32_t st, WB& W) {
        const rsrc_t wr = make_rsrc(x.blk, x.blk ? (uint32_t)NL.total : 0u);
#pragma unroll
        for (uint32_t j = 0; j < kWL; j++) {
            const uint32_t sl = min(x.part * kSG + j / 2u, S - 1u);
            W.w[j] = bld16_nt(wr, vgu, sl * 8u * nkg * 1024u + (2u * st + j % 2u) * 1024u);
        }
        bld8(wr, vgus, (x.part * 8u * nst + st) * 512u, W.s);
    };
    f32x4 acc[kSG][NB];
    // step st (< SPC) of chunk c: the GEMM kernel's routed step, A from slot c mod 3
    auto consume = [&](uint32_t c, uint32_t st, const WB& W) {
        float sc[2][kSG];
#pragma unroll
        for (uint32_t q = 0; q < 2; q++)
#pragma unroll
            for (uint32_t i = 0; i < kSG; i++) sc[q][i] = e8m0f((W.s[i >> 1] >> (8u * (2u * (i & 1u) + q))) & 0xFFu);
        const uint8_t* sl = slot_c(c % 3u) + 512u * st;
        bf16x8 af[2][NB];
#pragma unroll
        for (uint32_t tb = 0; tb < NB; tb++) af[0][tb] = as_bf16x8(*(const u32x4*)(sl + lo[tb][0]));
        bf16x8 bw[kSG];
#pragma unroll
        for (uint32_t it = 0; it < 8u; it++) {
            const uint32_t q = it / 4u, jj = it % 4u, cc = it % 2u;
            if (it + 1u < 8u) {
                const uint32_t n2 = it + 1u;
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++)
                    af[cc ^ 1u][tb] = as_bf16x8(*(const u32x4*)(sl + 256u * (n2 / 4u) + lo[tb][n2 % 4u]));
            }
#pragma unroll
            for (uint32_t i = 0; i < kSG; i++) bw[i] = fp4x8_bf16(W.w[2u * i + q][jj], sc[q][i]);
#pragma unroll
            for (uint32_t i = 0; i < kSG; i++)
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) acc[i][tb] = mma(af[cc][tb], bw[i], acc[i][tb]);
        }
    };
    // chunk boundary: this wave's DMAs older than the two steps of weights in
    // flight have landed and its LDS writes are done, then every wave's are
    // and every wave is done with the slot the last chunk read
    auto boundary = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt((18u & 15u) | ((18u >> 4) << 14) | 0x0070u);  // vmcnt(18) lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    uint32_t* const q = b.wq + (NB - 1u);
    const bool taker = tid == 0u;
    if (taker) qs[0] = take_next(q);
    lds_barrier();
    Unit cur, nxt, done;
    unit(uni(qs[0]), cur);
    unit(U, nxt);
    done.blk = nullptr;
    done.live = false;
    if (!cur.live) return;
    dma(0u, cur);
    dma(1u, cur);
    WB B0, B1;
    issue(cur, 0u, B0);
    issue(cur, 1u, B1);
    // SwiGLU of unit x's kSG slices (pieces in rows: token m = 4 tb + g),
    // after the next unit's first boundary, so its stores do not count
    // against that boundary's wait
    auto epilogue = [&](const Unit& x) {
        const uint32_t ln = opaque_lane();
#pragma unroll
        for (uint32_t i = 0; i < kSG; i++) {
            const uint32_t sl = x.part * kSG + i;
            if (sl >= S) continue;
            const f32x4 two[2] = {acc[i][0], NB == 2u ? acc[i][NB - 1u] : f32x4{0.f, 0.f, 0.f, 0.f}};
            swiglu_store(two, x.nt, true, ln, [&](uint32_t m, uint32_t nn, float xv) {
                store3(b.mid3 + (size_t)(x.c0 + m) * 3u * I + sl * kSlice + v * 8u + nn, I, xv);
            });
        }
    };
    uint32_t taken = 0u;  // wave 0: the next unit (in flight from chunk 0 on)
    while (cur.live) {
        if (cur.blk == nullptr && threadIdx.x == 0u) raise_error(a.sync, SyncMap::make(), E_NOT_RESIDENT, 0u);
        // chunk c of unit cur: at its boundary the slot (c + 2) mod 3 takes
        // chunk c + 2 (of this unit, or the next unit's chunk c + 2 - NCH);
        // steps z + 2 >= 24 load the next unit's first steps (dead units
        // load nothing)
#pragma unroll
        for (uint32_t c = 0; c < NCH; c++) {
            if (c == NCH - 2u && taker) qs[2] = taken;  // published by this boundary
            boundary();
            if (c == 0u && taker) taken = take_next(q);
            if (c == NCH - 2u) unit(uni(qs[2]), nxt);
            if (c + 2u < NCH) dma(c + 2u, cur);
            else dma(c + 2u - NCH, nxt);
            if (c == 0u) {
                if (done.live && done.blk != nullptr) epilogue(done);
#pragma unroll
                for (uint32_t i = 0; i < kSG; i++)
#pragma unroll
                    for (uint32_t tb = 0; tb < NB; tb++) acc[i][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (uint32_t st = 0; st < SPC; st++) {
                const uint32_t z = SPC * c + st;
                WB& BUF = (z % 2u) ? B1 : B0;
                consume(c, st, BUF);
                __builtin_amdgcn_sched_barrier(0);
                if (z + 2u < 24u) issue(cur, z + 2u, BUF);
                else issue(nxt, z + 2u - 24u, BUF);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        done = cur;
        cur = nxt;
    }
    if (done.blk != nullptr) epilogue(done);
}
// After the streaming pipelines: the last work-group to get here resets the
// work-queue counters for the next launch (every other one has taken its
// last unit by then).
WL_DEV void wq_release(const BatchArgs& b) {
    if (threadIdx.x != 0u) return;
    if (rmw_inc(b.wq + kWqWords - 1u) != gridDim.x - 1u) return;
    for (uint32_t i = 0; i < kWqWords; i++) __hip_atomic_store(b.wq + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// SMALL = true (GLM shape only): the instantiation with the small-expert
// pipeline, taken with bdown_kernel's (launch_batched).
template <bool GLM, bool SMALL>
__global__ void __launch_bounds__(kThreads) bup_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    extern __shared__ __align__(16) uint8_t dyn[];
    const uint32_t H = a.H, I = a.I;
    const bool sh4 = (b.flags & kBatchShared4) != 0u;
    const uint32_t E = a.E + (sh4 ? 1u : 0u);  // experts in the pass table
    const uint8_t* const* stab = load_slot_tab(a, a.E, sh4, (const uint8_t**)dyn);
    const PassTab pt =
        load_pass_tab(b, E, a.K, (uint32_t*)(dyn + 8u * E), stab, cdiv(I / kSlice, kSG), SMALL ? kSmallUpT : 0u);
    // the wide units first (each a pipeline of its own), then the kMT units,
    // which start on the work-groups after the wide units' last ones
    const uint32_t Us = run_shared_up_wide<GLM>(a, b);
    if (Us) pipeline_drain();
    const uint32_t Ur = run_routed_up_wide<GLM>(a, b, pt, stab, E, Us % gridDim.x);
    if (Ur) pipeline_drain();
    UpK k{a, b};
    k.H = H;
    k.I = I;
    k.SI = a.SI;
    k.E = E;
    k.K = a.K;
    k.nkg = H / 128u;
    k.nkt = H / 32u;
    k.S = I / kSlice;
    k.NSG = cdiv(k.S, kSG);
    k.Ssh = a.SI / kSlice;
    k.Us = (b.flags & (kBatchNoShared | kBatchShared4 | kBatchWideSharedUp)) ? 0u : cdiv(b.T, kMT) * k.Ssh;
    k.nst = cdiv(H, kKC);
    const uint32_t U = k.Us + pt.n * k.NSG;
    k.uoff = (Us + Ur) % gridDim.x;
    const uint32_t b0 = (blockIdx.x + gridDim.x - k.uoff) % gridDim.x;
    k.nu = U > b0 ? cdiv(U - b0, gridDim.x) : 0u;
    k.lane = threadIdx.x & 63u;
    k.g = k.lane >> 4;
    k.v = uni(threadIdx.x >> 6);
    k.pt = pt;
    k.stab = stab;
    k.NL = NativeLayout::make(H, I);
    k.vgu = (uint32_t)k.NL.gu + k.v * k.nkg * 1024u + 16u * k.lane;
    k.vgus = (uint32_t)k.NL.bgus + k.v * k.nst * 512u + 8u * k.lane;
    k.vsh = k.v * k.nkt * 1024u + 16u * k.lane;
#pragma unroll
    for (uint32_t j = 0; j < 4; j++) {
        k.lo_r[j] = a_lane_off(4u * k.g + j);
        k.lo_s[j] = a_lane_off(4u * j + k.g);
    }
    uint16_t* tt = (uint16_t*)(dyn + tok_table_offset(a.E));
    k.tt = tt;
    fill_tokens(k, tt, kMT);
    run_steps(k);
    if constexpr (SMALL) {
        pipeline_drain();
        // the pass table's LDS (and on) holds the small-expert lists now
        // (the host sizes the dynamic LDS for them: small_list_end)
        SmallExp* se = (SmallExp*)(dyn + 8u * (a.E + 1u));
        uint32_t* wcnt = (uint32_t*)(se + a.E);
        const uint32_t K_ = GLM ? 8u : a.K;
        // the larger units first: the queue then evens the work-groups out
        // with the smaller ones (the other order left the work-groups that
        // took one of the last, larger units ending most of a unit late)
        uint32_t ns = small_list(a, b, stab, kSmallT + 1u, kSmallUpT, K_, se, wcnt);
        run_small_up<2>(a, b, se, ns, stab, wcnt);
        pipeline_drain();
        ns = small_list(a, b, stab, 1u, kSmallT, K_, se, wcnt);
        run_small_up<1>(a, b, se, ns, stab, wcnt);
        wq_release(b);
    }
}

// ---- down ---------------------------------------------------------------------
// Shared unit (pass p, row block rb): output rows r0 = 128 rb + 16 v .. +16
// per wave; native sdn: 16 bytes (8 bf16 columns of tile T) per row, lane
// (n, g) of k step ks reads tile 4 ks + g of row r0 + n. K = SI.
// Routed unit (expert pass, row block rb): wave v owns row pairs
// q = 16 rb + 2v + h (h = 0, 1; 32 rows each, native dn chunks: 1 KB per
// 64-column slice, v_permlane32_swap pairs the halves), K = I.
// Output: f32 rows of shout / expout.
static_assert(kWL == 8u && kSL == 1u, "down step = 4 slices x 2 row pairs (one 8-byte scale word)");
struct DownK {
    using AS = AStream;
    using WB = WBuf;
    static constexpr uint32_t kLoads = kWL + kSL;
    template <int S>
    static __device__ __forceinline__ void issue_a(const AStream& A, uint32_t s) {
        a_issue<S>(A, s * kKC);
    }
    const DecodeArgs& a;
    const BatchArgs& b;
    uint32_t H, I, SI, E, nq, NS, nks, RBs, RBr, Us, nst, nstd, nu, v, lane, n, g;
    uint32_t uoff;  // unit u runs on work-group (u + uoff) % grid
    PassTab pt;
    const uint8_t* const* stab;
    NativeLayout NL;
    Cursor ca, cw, cc;
    // the weight stream's block and the scale stream's (null: none), kept as
    // pointers: a buffer resource held in the struct went through scratch in
    // one instantiation, and its loads became per-lane resource loops
    const uint8_t* wbase;
    const uint8_t* sbase;
    uint32_t wbytes, sbytes;
    bool wsh;
    uint32_t wpart, wvoff, vdn, vdns;
    // A fragment lane offsets: routed slice s4, half f (cg = 8 s4 + 4 (g & 1)
    // + (g >> 1) + 2 f: lo_r[s4 & 1][f], hi = s4 >> 1); shared k tile k
    // (cg = 4 k + g)
    uint32_t lo_r[2][2], lo_s[4];
    UnitInfo cu;
    PassShape cps;
    uint32_t cvar;  // compute variant: 0/1 pieces in rows, 1/2 blocks; 2/3 tokens in rows, 1/2 blocks
    f32x4 d[2][2][2];  // [row pair h][x rows / y rows][row block tb]

    WL_MEM UnitInfo unit(uint32_t i) const {
        UnitInfo x{false, false, 0u, 0u, 0u, 0u};
        if (i >= nu) return x;
        const uint32_t u = (blockIdx.x + gridDim.x - uoff) % gridDim.x + gridDim.x * i;
        x.live = true;
        if (u < Us) {
            const uint32_t p = u / RBs;
            x.sh = true;
            x.part = u % RBs;
            x.nt = min(kMT, b.T - p * kMT);
            x.row0 = p * kMT;
        } else {
            const PassPart jp = pass_part(u - Us, RBr, pt.n);
            const Pass ps = pass_at(pt, E, jp.j);
            x.part = jp.part;
            x.e = ps.e;
            x.nt = ps.nt;
            x.row0 = ps.c0;
        }
        return x;
    }
    WL_MEM void bind_a(uint32_t i, AStream& A) const {
        const UnitInfo x = unit(i);
        if (!x.live) return a_none(A);
        const bool pr = pass_shape(x.nt).pr;
        if (x.sh) a_bind(A, b.smid3, (uint64_t)b.T * 6u * SI, x.row0, x.nt, pr, SI);
        else a_bind(A, b.mid3, (uint64_t)b.T * (a.K + ((b.flags & kBatchShared4) ? 1u : 0u)) * 6u * I, x.row0, x.nt, pr, I);
    }
    WL_MEM void bind_w(uint32_t i) {
        const UnitInfo x = unit(i);
        wsh = x.sh;
        wpart = x.part;
        const NativeShared NSh = NativeShared::make(H, SI);
        const uint8_t* blk = x.live && !x.sh ? uni_ptr(stab[x.e]) : nullptr;
        wbase = !x.live ? nullptr : x.sh ? a.sh_native + NSh.sdn : blk;
        wbytes = !x.live ? 0u : x.sh ? (uint32_t)(NSh.total - NSh.sdn) : blk ? (uint32_t)NL.total : 0u;
        sbase = x.live && !x.sh ? blk : nullptr;
        sbytes = x.live && !x.sh && blk ? (uint32_t)NL.total : 0u;
        // the lane's weight offset base, chosen here (a select between two
        // members at each load would take the members' addresses)
        wvoff = x.sh ? (g * H + min(x.part * 128u + 16u * v + n, H - 1u)) * 16u : vdn;
    }
    WL_MEM void issue_w_one(uint32_t st, WBuf& W, uint32_t j) const {
        const uint32_t q0 = wpart * 16u + 2u * v;
        if (j < kWL) {
            const uint32_t sj = min(st * 4u + j / 2u, NS - 1u), q = min(q0 + j % 2u, nq - 1u);
            const uint32_t ro = (sj * nq + q) * 1024u;
            const uint32_t so = min(8u * st + j, nks - 1u) * 4u * H * 16u;
            W.w[j] = bld16_nt(make_rsrc(wbase, wbytes), wvoff, wsh ? so : ro);
        } else {
            bld8(make_rsrc(sbase, sbytes), vdns, (wpart * 8u * nstd + min(st, nstd - 1u)) * 512u, W.s);
        }
    }
    WL_MEM void begin(uint32_t i) {
        cu = unit(i);
        cps = pass_shape(cu.nt);
        cvar = (cps.pr ? 0u : 2u) + cps.nblk - 1u;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++)
#pragma unroll
            for (uint32_t xy = 0; xy < 2; xy++) d[h][xy][0] = d[h][xy][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // Shared: as UpK::comp_shared, MFMA it (k step k, plane pc, block tb)
    // into accumulator j = (NP k + pc) % 4 of block tb (d[j >> 1][j & 1][tb]),
    // fragments read kSPD MFMAs ahead; finish() adds the four.
    static constexpr uint32_t kSPD = 6;
    template <uint32_t NB, uint32_t NP>
    WL_MEM void comp_shared(uint32_t st, const uint8_t* sl, const WBuf& W) {
        constexpr uint32_t N = 8u * NP * NB;
        bf16x8 af[kSPD + 1u];
        auto frag = [&](uint32_t it) {  // it = (k NP + pc) NB + tb
            const uint32_t tb = it % NB, pc = (it / NB) % NP, k = it / (NB * NP);
            return afrag(sl, pc, tb, k / 4u, lo_s[k % 4u]);
        };
#pragma unroll
        for (uint32_t it = 0; it < kSPD && it < N; it++) af[it] = frag(it);
#pragma unroll
        for (uint32_t it = 0; it < N; it++) {
            const uint32_t tb = it % NB, kp = it / NB, k = kp / NP, j = kp % 4u;
            if (it + kSPD < N) af[(it + kSPD) % (kSPD + 1u)] = frag(it + kSPD);
            const u32x4 z = {0u, 0u, 0u, 0u};
            const bf16x8 bw = as_bf16x8(8u * st + k < nks ? W.w[k] : z);
            d[j >> 1][j & 1u][tb] = mma(af[it % (kSPD + 1u)], bw, d[j >> 1][j & 1u][tb]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Routed: iteration it = NB NP (2 s4 + f) + NP tb + pc runs the fragment
    // of plane pc, block tb at column half f of slice s4 against both row
    // pairs; the next iteration's fragment is read while this one's four
    // MFMAs run.
    template <uint32_t NB, uint32_t NP>
    WL_MEM void comp_routed(uint32_t st, const uint8_t* sl, const WBuf& W) {
        constexpr uint32_t NI = NB * NP, N = 8u * NI;
        auto frag = [&](uint32_t it) {
            const uint32_t o = it / NI, in = it % NI, s4 = o / 2u, f = o % 2u;
            return afrag(sl, in % NP, in / NP, s4 / 2u, lo_r[s4 % 2u][f]);
        };
        bf16x8 af[2];
        af[0] = frag(0u);
        float scx[2], scy[2];
        bf16x8 bx[2], by[2];
#pragma unroll
        for (uint32_t it = 0; it < N; it++) {
            const uint32_t o = it / NI, in = it % NI, s4 = o / 2u, f = o % 2u, tb = in / NP;
            if (it + 1u < N) af[(it + 1u) % 2u] = frag(it + 1u);
            if (in == 0u) {
                if (f == 0u) {
                    const bool valid = st * 4u + s4 < NS;
#pragma unroll
                    for (uint32_t h = 0; h < 2; h++) {
                        // decoded once, then swapped like the weight dwords
                        const uint32_t sv = __float_as_uint(e8m0f((W.s[s4 >> 1] >> (8u * (2u * (s4 & 1u) + h))) & 0xFFu));
                        uint32_t sx, sy;
                        swap32(sv, sv, sx, sy);
                        scx[h] = valid ? __uint_as_float(sx) : 0.f;
                        scy[h] = valid ? __uint_as_float(sy) : 0.f;
                    }
                }
                // Column half f of the slice: lane group g's columns s4 * 64 +
                // 32 (g & 1) + 8 (g >> 1) + 16 f (the swap order), from dwords
                // 2f, 2f + 1 of each row pair's chunk.
#pragma unroll
                for (uint32_t h = 0; h < 2; h++) {
                    const u32x4 w = W.w[2u * s4 + h];
                    uint32_t x, y;
                    swap32(w[2u * f], w[2u * f + 1u], x, y);
                    bx[h] = fp4x8_bf16(x, scx[h]);
                    by[h] = fp4x8_bf16(y, scy[h]);
                }
            }
            const bf16x8 a = af[it % 2u];
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                d[h][0][tb] = mma(a, bx[h], d[h][0][tb]);
                d[h][1][tb] = mma(a, by[h], d[h][1][tb]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    WL_MEM void compute(uint32_t st, const uint8_t* sl, const WBuf& W) {
        switch (cvar) {
            case 0: return cu.sh ? comp_shared<1, 1>(st, sl, W) : comp_routed<1, 1>(st, sl, W);
            case 1: return cu.sh ? comp_shared<2, 1>(st, sl, W) : comp_routed<2, 1>(st, sl, W);
            case 2: return cu.sh ? comp_shared<1, 3>(st, sl, W) : comp_routed<1, 3>(st, sl, W);
            default: return cu.sh ? comp_shared<2, 3>(st, sl, W) : comp_routed<2, 3>(st, sl, W);
        }
    }
    WL_MEM void finish() {
        const uint32_t ln = opaque_lane(), nn = ln & 15u;
        if (cu.sh) {
#pragma unroll
            for (uint32_t tb = 0; tb < 2; tb++)
                d[0][0][tb] = (d[0][0][tb] + d[0][1][tb]) + (d[1][0][tb] + d[1][1][tb]);
            const uint32_t r = cu.part * 128u + 16u * v + nn;
            if (r < H)
                tile_each(d[0][0], cu.nt, cps.pr, ln,
                          [&](uint32_t m, float x) { gst(b.shout + (size_t)(cu.row0 + m) * H + r, x); });
            return;
        }
#pragma unroll
        for (uint32_t h = 0; h < 2; h++) {
            const uint32_t q = cu.part * 16u + 2u * v + h;
            if (q >= nq) continue;
            float* o = b.expout + (size_t)cu.row0 * H + 32u * q + nn;
            tile_each(d[h][0], cu.nt, cps.pr, ln, [&](uint32_t m, float x) { gst(o + (size_t)m * H, x); });
            tile_each(d[h][1], cu.nt, cps.pr, ln, [&](uint32_t m, float x) { gst(o + (size_t)m * H + 16u, x); });
        }
    }
};
// Shared down in wide passes (batches of more than kMT tokens): unit (pass p
// of kMTW tokens, row block rb of 256 output rows): wave v owns rows
// 256 rb + 32 v + 16 i + n (i = 0, 1); step st covers columns [128 st, +128)
// of SI: native sdn (16 bytes = 8 bf16 columns [8T, 8T + 8) of a row), lane
// (n, g) of k step k reads tile 4 (4 st + k) + g of its row.
struct SharedDownW {
    using AS = AStreamW;
    using WB = WBufW;
    static constexpr uint32_t kLoads = 8;
    template <int S>
    static __device__ __forceinline__ void issue_a(const AStreamW& A, uint32_t s) {
        aw_issue<S>(A, s * kKCW);
    }
    const DecodeArgs& a;
    const BatchArgs& b;
    uint32_t H, SI, nrb, npass, nst, nu, v, lane, n, g;
    Cursor ca, cw, cc;
    rsrc_t wrs;
    uint32_t wvoff[2];
    uint32_t lob;  // A fragment lane offset of k step 0 (cg = g; k step k: ^ 64 k)
    uint32_t crb, cnt, crow0, cnb;
    f32x4 d[2][4];

    struct Unit {
        bool live;
        uint32_t rb, nt, row0;
    };
    WL_MEM Unit unit(uint32_t i) const {
        Unit x{false, 0u, 0u, 0u};
        if (i >= nu) return x;
        const PassPart jp = pass_part(blockIdx.x + gridDim.x * i, nrb, npass);
        x.live = true;
        x.rb = jp.part;
        x.row0 = jp.j * kMTW;
        x.nt = min(kMTW, b.T - x.row0);
        return x;
    }
    WL_MEM void bind_a(uint32_t i, AStreamW& A) const {
        const Unit x = unit(i);
        if (!x.live) return aw_bind(A, nullptr, 0u, 0u, 0u, 0u);
        aw_bind(A, b.smid3, (uint64_t)b.T * 6u * SI, x.row0, x.nt, SI);
    }
    WL_MEM void bind_w(uint32_t i) {
        const Unit x = unit(i);
        const NativeShared NS = NativeShared::make(H, SI);
        wrs = x.live ? make_rsrc(a.sh_native + NS.sdn, (uint32_t)(NS.total - NS.sdn)) : make_rsrc(nullptr, 0u);
#pragma unroll
        for (uint32_t t = 0; t < 2; t++) wvoff[t] = (g * H + min(256u * x.rb + 32u * v + 16u * t + n, H - 1u)) * 16u;
    }
    WL_MEM void issue_w_one(uint32_t st, WBufW& W, uint32_t j) const {
        W.w[j] = bld16(wrs, wvoff[j / 4u], (16u * st + 4u * (j % 4u)) * H * 16u);  // re-read by every pass: cached
    }
    WL_MEM void begin(uint32_t i) {
        const Unit x = unit(i);
        crb = x.rb;
        cnt = x.nt;
        crow0 = x.row0;
        cnb = cdiv(x.nt, 16u);
#pragma unroll
        for (uint32_t t = 0; t < 2; t++)
#pragma unroll
            for (uint32_t tb = 0; tb < 4; tb++) d[t][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    template <uint32_t NB>
    WL_MEM void comp(const uint8_t* sl, const WBufW& W) {
        bf16x8 af[2][NB];
#pragma unroll
        for (uint32_t tb = 0; tb < NB; tb++) af[0][tb] = afragw(sl, 0u, tb, lob);
#pragma unroll
        for (uint32_t it = 0; it < 12u; it++) {
            const uint32_t k = it / 3u, c = it & 1u;
            if (it + 1u < 12u) {
                const uint32_t nx = it + 1u;
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) af[c ^ 1u][tb] = afragw(sl, nx % 3u, tb, lob ^ (64u * (nx / 3u)));
            }
#pragma unroll
            for (uint32_t t = 0; t < 2; t++) {
                const bf16x8 bw = as_bf16x8(W.w[4u * t + k]);
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) d[t][tb] = mma(af[c][tb], bw, d[t][tb]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    WL_MEM void compute(uint32_t, const uint8_t* sl, const WBufW& W) {
        switch (cnb) {
            case 1: return comp<1>(sl, W);
            case 2: return comp<2>(sl, W);
            case 3: return comp<3>(sl, W);
            default: return comp<4>(sl, W);
        }
    }
    WL_MEM void finish() {
        const uint32_t ln = opaque_lane(), nn = ln & 15u;
#pragma unroll
        for (uint32_t t = 0; t < 2; t++) {
            const uint32_t r = 256u * crb + 32u * v + 16u * t + nn;
            if (r < H)
                tile_each_w(d[t], cnt, ln, [&](uint32_t m, float x) { gst(b.shout + (size_t)(crow0 + m) * H + r, x); });
        }
    }
};
template <bool GLM>
WL_DEV uint32_t run_shared_down_wide(const DecodeArgs& a, const BatchArgs& b) {
    if (!(b.flags & kBatchWideSharedDown)) return 0u;
    const uint32_t H_ = GLM ? 6144u : a.H, I_ = GLM ? 2048u : a.I, SI_ = GLM ? 2048u : a.SI, K_ = GLM ? 8u : a.K;
    (void)I_;
    (void)K_;
    SharedDownW w{a, b};
    w.H = H_;
    w.SI = SI_;
    w.nrb = cdiv(H_, 256u);
    w.npass = cdiv(b.T, kMTW);
    w.nst = SI_ / kKCW;
    const uint32_t U = w.npass * w.nrb;
    w.nu = U > blockIdx.x ? cdiv(U - blockIdx.x, gridDim.x) : 0u;
    w.lane = threadIdx.x & 63u;
    w.n = w.lane & 15u;
    w.g = w.lane >> 4;
    w.v = uni(threadIdx.x >> 6);
    w.lob = aw_lane_off(w.g);
    run_steps(w);
    return U;
}
// Routed down in wide passes (an expert of more than kMT tokens): unit (pass
// of kMTW tokens, row block rb): wave v owns row pairs q = 16 rb + 2v + h
// (h = 0, 1), as in a kMT unit; step st covers columns [128 st, +128) of I:
// slices sj = 2 st + s4 (s4 = 0, 1), the native dn chunks (sj, q) and the
// batched scale word of the 256-column step st / 2 (bytes 2 (2 (st & 1) + s4)
// + h).
struct RoutedDownW {
    using AS = AStreamW;
    struct WB {
        u32x4 w[4];
        uint32_t s;  // the step's dword of its scale word
    };
    static constexpr uint32_t kLoads = 5;
    template <int S>
    static __device__ __forceinline__ void issue_a(const AStreamW& A, uint32_t s) {
        aw_issue<S>(A, s * kKCW);
    }
    const DecodeArgs& a;
    const BatchArgs& b;
    uint32_t H, I, E, nq, NS, RBr, nst, nstd, nu, v, lane, n, g, uoff;
    PassTab pt;
    const uint8_t* const* stab;
    NativeLayout NL;
    Cursor ca, cw, cc;
    rsrc_t wrs;
    uint32_t wpart, vdn, vdns;
    uint32_t lob;  // A fragment lane offset of slice 0, half 0 (cg = 4 (g & 1) + (g >> 1); ^ 16 (8 s4 + 2 f))
    UnitInfo cu;
    uint32_t cnb;
    f32x4 d[2][2][3];  // [row pair h][x rows / y rows][row block tb]

    WL_MEM UnitInfo unit(uint32_t i) const {
        UnitInfo x{false, false, 0u, 0u, 0u, 0u};
        if (i >= nu) return x;
        const uint32_t r = (blockIdx.x + gridDim.x - uoff) % gridDim.x + gridDim.x * i;
        const PassPart jp = pass_part(r, RBr, pt.nw);
        const Pass ps = pass_at_w(pt, E, jp.j);
        x.live = true;
        x.part = jp.part;
        x.e = ps.e;
        x.nt = ps.nt;
        x.row0 = ps.c0;
        return x;
    }
    WL_MEM void bind_a(uint32_t i, AStreamW& A) const {
        const UnitInfo x = unit(i);
        if (!x.live) return aw_bind(A, nullptr, 0u, 0u, 0u, 0u);
        aw_bind(A, b.mid3, (uint64_t)b.T * (a.K + ((b.flags & kBatchShared4) ? 1u : 0u)) * 6u * I, x.row0, x.nt, I);
    }
    WL_MEM void bind_w(uint32_t i) {
        const UnitInfo x = unit(i);
        const uint8_t* blk = x.live ? uni_ptr(stab[x.e]) : nullptr;
        wrs = make_rsrc(blk, blk ? (uint32_t)NL.total : 0u);
        wpart = x.part;
    }
    WL_MEM void issue_w_one(uint32_t st, WB& W, uint32_t j) const {
        if (j < 4u) {
            const uint32_t sj = min(2u * st + j / 2u, NS - 1u), q = min(wpart * 16u + 2u * v + j % 2u, nq - 1u);
            W.w[j] = bld16_nt(wrs, vdn, (sj * nq + q) * 1024u);
        } else {
            W.s = __builtin_amdgcn_raw_buffer_load_b32(wrs, (int)vdns, (int)((wpart * 8u * nstd + st / 2u) * 512u + 4u * (st & 1u)), 0);
        }
    }
    WL_MEM void begin(uint32_t i) {
        cu = unit(i);
        cnb = cdiv(cu.nt, 16u);
#pragma unroll
        for (uint32_t h = 0; h < 2; h++)
#pragma unroll
            for (uint32_t xy = 0; xy < 2; xy++)
#pragma unroll
                for (uint32_t tb = 0; tb < 3; tb++) d[h][xy][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // Iteration it = 3 NB (2 s4 + f) + 3 tb + pc runs the fragment of plane
    // pc, block tb at column half f of slice s4 against both row pairs; the
    // next iteration's fragment is read while this one's four MFMAs run.
    template <uint32_t NB>
    WL_MEM void comp(uint32_t st, const uint8_t* sl, const WB& W) {
        constexpr uint32_t NI = NB * 3u, N = 4u * NI;
        auto frag = [&](uint32_t it) {
            const uint32_t o = it / NI, in = it % NI;
            return afragw(sl, in % 3u, in / 3u, lob ^ (16u * (8u * (o / 2u) + 2u * (o % 2u))));
        };
        bf16x8 af[2];
        af[0] = frag(0u);
        float scx[2], scy[2];
        bf16x8 bx[2], by[2];
#pragma unroll
        for (uint32_t it = 0; it < N; it++) {
            const uint32_t o = it / NI, in = it % NI, s4 = o / 2u, f = o % 2u, tb = in / 3u;
            if (it + 1u < N) af[(it + 1u) % 2u] = frag(it + 1u);
            if (in == 0u) {
                if (f == 0u) {
                    const bool valid = 2u * st + s4 < NS;
#pragma unroll
                    for (uint32_t h = 0; h < 2; h++) {
                        // decoded once, then swapped like the weight dwords
                        const uint32_t sv = __float_as_uint(e8m0f((W.s >> (8u * (2u * s4 + h))) & 0xFFu));
                        uint32_t sx, sy;
                        swap32(sv, sv, sx, sy);
                        scx[h] = valid ? __uint_as_float(sx) : 0.f;
                        scy[h] = valid ? __uint_as_float(sy) : 0.f;
                    }
                }
#pragma unroll
                for (uint32_t h = 0; h < 2; h++) {
                    const u32x4 w = W.w[2u * s4 + h];
                    uint32_t x, y;
                    swap32(pinned(w[2u * f]), w[2u * f + 1u], x, y);
                    bx[h] = fp4x8_bf16(x, scx[h]);
                    by[h] = fp4x8_bf16(y, scy[h]);
                }
            }
            const bf16x8 av = af[it % 2u];
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                d[h][0][tb] = mma(av, bx[h], d[h][0][tb]);
                d[h][1][tb] = mma(av, by[h], d[h][1][tb]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    WL_MEM void compute(uint32_t st, const uint8_t* sl, const WB& W) {
        switch (cnb) {
            case 1: return comp<1>(st, sl, W);
            case 2: return comp<2>(st, sl, W);
            default: return comp<3>(st, sl, W);
        }
    }
    WL_MEM void finish() {
        const uint32_t ln = opaque_lane(), nn = ln & 15u;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++) {
            const uint32_t q = cu.part * 16u + 2u * v + h;
            if (q >= nq) continue;
            float* o = b.expout + (size_t)cu.row0 * H + 32u * q + nn;
            tile_each_w(d[h][0], cu.nt, ln, [&](uint32_t m, float x) { gst(o + (size_t)m * H, x); });
            tile_each_w(d[h][1], cu.nt, ln, [&](uint32_t m, float x) { gst(o + (size_t)m * H + 16u, x); });
        }
    }
};
template <bool GLM>
WL_DEV uint32_t run_routed_down_wide(const DecodeArgs& a, const BatchArgs& b, const PassTab& pt,
                                     const uint8_t* const* stab, uint32_t E, uint32_t uoff) {
    if (pt.nw == 0u) return 0u;
    const uint32_t H_ = GLM ? 6144u : a.H, I_ = GLM ? 2048u : a.I, SI_ = GLM ? 2048u : a.SI, K_ = GLM ? 8u : a.K;
    (void)I_;
    (void)K_;
    RoutedDownW w{a, b};
    w.H = H_;
    w.I = I_;
    w.E = E;
    w.nq = H_ / 32u;
    w.NS = I_ / kSlice;
    w.RBr = cdiv(w.nq, 16u);
    w.nst = I_ / kKCW;
    w.nstd = cdiv(I_, kKC);
    w.uoff = uoff;
    const uint32_t U = pt.nw * w.RBr, b0 = (blockIdx.x + gridDim.x - uoff) % gridDim.x;
    w.nu = U > b0 ? cdiv(U - b0, gridDim.x) : 0u;
    w.lane = threadIdx.x & 63u;
    w.n = w.lane & 15u;
    w.g = w.lane >> 4;
    w.v = uni(threadIdx.x >> 6);
    w.pt = pt;
    w.stab = stab;
    w.NL = NativeLayout::make(H_, I_);
    w.vdn = (uint32_t)w.NL.dn + 16u * w.lane;
    w.vdns = (uint32_t)w.NL.bdns + w.v * w.nstd * 512u + 8u * w.lane;
    w.lob = aw_lane_off(4u * (w.g & 1u) + (w.g >> 1));
    run_steps(w);
    return U;
}
// ---- routed down of small experts ---------------------------------------------
// Experts with 1..kSmallUpT tokens (at small T most of them: 64 tokens x 8
// slots over ~200 experts) run their down projection as streaming units,
// like the decode kernel's down phase: unit (expert, row block of 16 row
// pairs), in two pipelines, NB = 1 for 1-4 tokens and NB = 2 for 5-8 (MFMA
// row blocks of pieces in rows). The expert's SwiGLU pieces are staged once
// per unit in LDS, token m's three pieces in stored rows 3m..3m+2 (MFMA row
// 16 tb + n reads stored row 3m + min(n % 4, 2) for m = 4 tb + n / 4: rows
// 4m + 3 carry values no output reads), so NB v_mfma_f32_16x16x32_bf16 cover
// all of the expert's tokens; then each wave
// streams its 2 row pairs x I/64 slices (native 1 KB dn chunks, the batched
// scale words of bdns) two 256-column steps ahead, with no barrier between
// steps (the GEMM kernel stages 48 KB of activation rows and meets a barrier
// every step). The arithmetic per step is the GEMM kernel's (pieces in rows,
// one row block). It is the last pipeline of bdown_kernel: its units are
// 512 KB of weights each, so with the rotation (unit r on work-group (r +
// uoff) mod grid, uoff the units of the earlier pipelines) the work-groups
// end within about one unit of each other. LDS: stored rows 8s..8s+7 in slot
// s, the small-expert list where the pass table was.
// the shapes it runs: at least two 256-column steps, at most 2048 columns staged
__host__ __device__ inline bool small_down_fits(uint32_t H, uint32_t I) {
    return I % kKC == 0u && I >= 2u * kKC && I <= 2048u && H % 512u == 0u;
}
// Returns the pipeline's unit count (the next pipeline starts after it).
template <bool GLM, uint32_t NB>
WL_DEV uint32_t run_small_down(const DecodeArgs& a, const BatchArgs& b, const uint8_t* const* stab, uint32_t uoff,
                               uint32_t* se) {
    const uint32_t H = GLM ? 6144u : a.H, I = GLM ? 2048u : a.I, E = GLM ? 256u : a.E;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, v = uni(tid >> 6), n = lane & 15u, g = lane >> 4;
    // se: [E] the small experts, ascending; se[E] their count
    const uint32_t RS = I + 8u;  // staged row stride (bf16): rows 16 bytes apart in the bank groups
    constexpr uint32_t ROWS = 12u * NB;  // stored rows (token m, piece pc: 3m + pc)
    static_assert(ROWS <= 24u, "three slots of eight rows");
    auto xrow = [&](uint32_t R) {
        return (uint16_t*)(R < 8u ? slot<0>() : R < 16u ? slot<1>() : slot<2>()) + (R % 8u) * RS;
    };
    const uint32_t lo_t = NB == 1u ? 1u : kSmallT + 1u, hi_t = NB == 1u ? kSmallT : kSmallUpT;
    const bool skip = (b.flags & kBatchSkipUnbound) != 0u;
    if (v == 0u) {
        uint32_t run = 0;
        for (uint32_t e0 = 0; e0 < E; e0 += 64u) {
            const uint32_t e = e0 + lane;
            const uint32_t c = e < E ? gld(b.counts + e) : 0u;
            const bool sm = c >= lo_t && c <= hi_t && !(skip && stab[e] == nullptr);
            const uint64_t bal = __ballot(sm);
            if (sm) se[run + (uint32_t)__popcll(bal & ((1ull << lane) - 1ull))] = e;
            run += (uint32_t)__popcll(bal);
        }
        if (lane == 0u) se[E] = run;
    }
    lds_barrier();
    const uint32_t ns = uni(se[E]), nq = H / 32u, RBr = cdiv(nq, 16u), nstd = I / kKC;
    const uint32_t U = ns * RBr, G = gridDim.x;
    const NativeLayout NL = NativeLayout::make(H, I);
    const uint32_t vdn = (uint32_t)NL.dn + 16u * lane, vdns = (uint32_t)NL.bdns + v * nstd * 512u + 8u * lane;
    const rsrc_t mrs = make_rsrc(b.mid3, (uint32_t)((size_t)b.T * (a.K + ((b.flags & kBatchShared4) ? 1u : 0u)) * 6u * I));
    // A fragment of lane (n, g), row block tb: its stored row, columns
    // 256 st + 64 s4 + 32 (g & 1) + 8 (g >> 1) + 16 f
    const uint16_t* arow[NB];
#pragma unroll
    for (uint32_t tb = 0; tb < NB; tb++)
        arow[tb] = xrow(3u * (4u * tb + (n >> 2)) + min(n & 3u, 2u)) + 32u * (g & 1u) + 8u * (g >> 1);
    struct WB {
        u32x4 w[kWL];
        uint32_t s[2];
    };
    constexpr uint32_t kAV = ROWS * 256u / kThreads;  // 16-byte chunks of the stored rows per thread (I <= 2048)
    const uint32_t cpr = I / 8u;  // 16-byte chunks per staged row
    // the unit being loaded: its expert's tokens, first compact row, block, row block
    uint32_t nt = 0, c0 = 0, part = 0;
    rsrc_t wrs = make_rsrc(nullptr, 0u);
    u32x4 av[kAV];
    auto issue = [&](uint32_t st, WB& W) {
#pragma unroll
        for (uint32_t j = 0; j < kWL; j++) {
            const uint32_t sj = 4u * st + j / 2u, q = min(16u * part + 2u * v + j % 2u, nq - 1u);
            W.w[j] = bld16_nt(wrs, vdn, (sj * nq + q) * 1024u);
        }
        bld8(wrs, vdns, (part * 8u * nstd + st) * 512u, W.s);
    };
    // unit r's pieces (into av, issued first) and its first two steps
    WB B0, B1;
    auto start = [&](uint32_t r) {
        const PassPart jp = pass_part(r, RBr, ns);
        const uint32_t e = uni(se[jp.j]);
        part = jp.part;
        nt = uni(gld(b.counts + e));
        c0 = uni(gld(b.offsets + e));
        wrs = make_rsrc(uni_ptr(stab[e]), (uint32_t)NL.total);
#pragma unroll
        for (uint32_t k = 0; k < kAV; k++) {
            const uint32_t idx = tid + kThreads * k, row = idx / cpr, c8 = idx % cpr, m = row / 3u, pc = row % 3u;
            const bool ok = idx < ROWS * cpr && m < nt;
            av[k] = __builtin_amdgcn_raw_buffer_load_b128(mrs, (int)(ok ? (((c0 + m) * 3u + pc) * I + 8u * c8) * 2u : kOOB), 0, 0);
        }
        issue(0u, B0);
        issue(1u, B1);
    };
    f32x4 d[2][2][NB];
    auto consume = [&](uint32_t st, const WB& W) {
        auto frag = [&](uint32_t o, uint32_t tb) {  // o = 2 s4 + f
            return as_bf16x8(*(const u32x4*)(arow[tb] + 256u * st + 64u * (o / 2u) + 16u * (o % 2u)));
        };
        bf16x8 af[2][NB];
#pragma unroll
        for (uint32_t tb = 0; tb < NB; tb++) af[0][tb] = frag(0u, tb);
        float scx[2], scy[2];
#pragma unroll
        for (uint32_t o = 0; o < 8u; o++) {
            const uint32_t s4 = o / 2u, f = o % 2u;
            if (o + 1u < 8u)
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) af[(o + 1u) % 2u][tb] = frag(o + 1u, tb);
            if (f == 0u) {
#pragma unroll
                for (uint32_t h = 0; h < 2; h++) {
                    // decoded once, then swapped like the weight dwords
                    const uint32_t sv = __float_as_uint(e8m0f((W.s[s4 >> 1] >> (8u * (2u * (s4 & 1u) + h))) & 0xFFu));
                    uint32_t sx, sy;
                    swap32(sv, sv, sx, sy);
                    scx[h] = __uint_as_float(sx);
                    scy[h] = __uint_as_float(sy);
                }
            }
            // column half f of slice s4: lane group g's columns 64 s4 + 32 (g & 1)
            // + 8 (g >> 1) + 16 f, from dwords 2f, 2f + 1 of each row pair's chunk
            bf16x8 bx[2], by[2];
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                const u32x4 wv = W.w[2u * s4 + h];
                uint32_t x, y;
                swap32(wv[2u * f], wv[2u * f + 1u], x, y);
                bx[h] = fp4x8_bf16(x, scx[h]);
                by[h] = fp4x8_bf16(y, scy[h]);
            }
#pragma unroll
            for (uint32_t h = 0; h < 2; h++)
#pragma unroll
                for (uint32_t tb = 0; tb < NB; tb++) {
                    d[h][0][tb] = mma(af[o % 2u][tb], bx[h], d[h][0][tb]);
                    d[h][1][tb] = mma(af[o % 2u][tb], by[h], d[h][1][tb]);
                }
        }
    };
    const uint32_t r0 = (blockIdx.x + G - uoff % G) % G;
    if (r0 < U) start(r0);
    for (uint32_t r = r0; r < U; r += G) {
#pragma unroll
        for (uint32_t k = 0; k < kAV; k++) {
            const uint32_t idx = tid + kThreads * k;
            if (idx < ROWS * cpr) *(u32x4*)(xrow(idx / cpr) + 8u * (idx % cpr)) = av[k];
        }
        lds_barrier();
#pragma unroll
        for (uint32_t h = 0; h < 2; h++)
#pragma unroll
            for (uint32_t tb = 0; tb < NB; tb++) d[h][0][tb] = d[h][1][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
        pingpong(nstd, B0, B1, issue, consume);
        // the next unit's pieces and first steps go out before this unit's
        // epilogue, so the stream does not stop between units
        const uint32_t nt_u = nt, c0_u = c0, part_u = part;
        if (r + G < U) start(r + G);
        const uint32_t ln = opaque_lane(), nn = ln & 15u;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++) {
            const uint32_t q = 16u * part_u + 2u * v + h;
            if (q >= nq) continue;
            float* o = b.expout + (size_t)c0_u * H + 32u * q + nn;
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            const f32x4 ax[2] = {d[h][0][0], NB == 2u ? d[h][0][NB - 1u] : z};
            const f32x4 ay[2] = {d[h][1][0], NB == 2u ? d[h][1][NB - 1u] : z};
            tile_each(ax, nt_u, true, ln, [&](uint32_t m, float x) { gst(o + (size_t)m * H, x); });
            tile_each(ay, nt_u, true, ln, [&](uint32_t m, float x) { gst(o + (size_t)m * H + 16u, x); });
        }
        lds_barrier();  // every wave is done with the staged rows before the next unit's pieces
    }
    return U;
}

// SMALL = true: the instantiation with the small-expert pipeline (launch_batched
// takes it at the shapes small_down_fits allows); the other keeps the GEMM
// pipelines' code alone (with the small pipeline compiled into one kernel for
// every shape, T = 256 and 1024 ran 2-4 % slower).
template <bool GLM, bool SMALL>
__global__ void __launch_bounds__(kThreads) bdown_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    extern __shared__ __align__(16) uint8_t dyn[];
    const uint32_t H = a.H, I = a.I;
    const bool sh4 = (b.flags & kBatchShared4) != 0u;
    const uint32_t E = a.E + (sh4 ? 1u : 0u);  // experts in the pass table
    const uint8_t* const* stab = load_slot_tab(a, a.E, sh4, (const uint8_t**)dyn);
    // (5-8 token units at the GLM shape only: elsewhere the kernel's general
    // shape code leaves no registers for their second row block)
    const PassTab pt = load_pass_tab(b, E, a.K, (uint32_t*)(dyn + 8u * E), stab, cdiv(H / 32u, 16u),
                                     SMALL ? (GLM ? kSmallUpT : kSmallT) : 0u);
    const uint32_t Us = run_shared_down_wide<GLM>(a, b);
    if (Us) pipeline_drain();
    const uint32_t Ur = run_routed_down_wide<GLM>(a, b, pt, stab, E, Us % gridDim.x);
    if (Ur) pipeline_drain();
    DownK k{a, b};
    k.H = H;
    k.I = I;
    k.SI = a.SI;
    k.E = E;
    k.nq = H / 32u;
    k.NS = I / kSlice;
    k.nks = a.SI / 32u;
    k.RBs = cdiv(H, 128u);
    k.RBr = cdiv(k.nq, 16u);
    k.Us = (b.flags & (kBatchNoShared | kBatchShared4 | kBatchWideSharedDown)) ? 0u : cdiv(b.T, kMT) * k.RBs;
    k.nst = cdiv(max(I, a.SI), kKC);  // the shorter kind's extra steps are masked
    const uint32_t U = k.Us + pt.n * k.RBr;
    k.uoff = (Us + Ur) % gridDim.x;
    const uint32_t b0 = (blockIdx.x + gridDim.x - k.uoff) % gridDim.x;
    k.nu = U > b0 ? cdiv(U - b0, gridDim.x) : 0u;
    k.lane = threadIdx.x & 63u;
    k.n = k.lane & 15u;
    k.g = k.lane >> 4;
    k.v = uni(threadIdx.x >> 6);
    k.pt = pt;
    k.stab = stab;
    k.NL = NativeLayout::make(H, I);
    k.vdn = (uint32_t)k.NL.dn + 16u * k.lane;
    k.nstd = cdiv(I, kKC);
    k.vdns = (uint32_t)k.NL.bdns + k.v * k.nstd * 512u + 8u * k.lane;
#pragma unroll
    for (uint32_t j = 0; j < 4; j++) {
        k.lo_r[j / 2u][j % 2u] = a_lane_off(8u * (j / 2u) + 4u * (k.g & 1u) + (k.g >> 1) + 2u * (j % 2u));
        k.lo_s[j] = a_lane_off(4u * j + k.g);
    }
    run_steps(k);
    if constexpr (SMALL) {
        pipeline_drain();
        // the small-expert list where the pass table was (4 (E + 1) of its
        // 16 E + 8 bytes)
        uint32_t* se = (uint32_t*)(dyn + 8u * (a.E + 1u));
        // the larger units first, as in the gate/up kernel
        uint32_t u2 = 0;
        if constexpr (GLM) {
            u2 = run_small_down<GLM, 2>(a, b, stab, k.uoff + U, se);
            pipeline_drain();
        }
        run_small_down<GLM, 1>(a, b, stab, k.uoff + U + u2, se);
    }
}

// out[t] = (resid[t] +) sum_k w[t][k] e_k[t] in slot order + shared[t]
// (reference pass 3, src/glm_layer_runner.cuh:904-921).
// Thread: 4 consecutive rows (16-byte loads; H is a multiple of 128), each
// with the scalar sequence acc = fma(w_k, e_k, acc) over k, + shared, + resid.
__global__ void __launch_bounds__(256) bcomb_kernel(const BatchArgs b, uint32_t H, uint32_t K) {
    const uint32_t t = blockIdx.y;
    const uint32_t r = 4u * (blockIdx.x * blockDim.x + threadIdx.x);
    if (r >= H) return;
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t k = 0; k < K; k++) {
        const uint32_t c = gld(b.pos + (size_t)t * K + k);
        const float w = gld(b.wts + (size_t)t * K + k);
        const float4 x = *(const float4*)(b.expout + (size_t)c * H + r);
        acc.x = fmaf(w, x.x, acc.x);
        acc.y = fmaf(w, x.y, acc.y);
        acc.z = fmaf(w, x.z, acc.z);
        acc.w = fmaf(w, x.w, acc.w);
    }
    const float4 sh = (b.flags & kBatchShared4) ? *(const float4*)(b.expout + ((size_t)b.T * K + t) * H + r)
                                                : *(const float4*)(b.shout + (size_t)t * H + r);
    acc.x += sh.x;
    acc.y += sh.y;
    acc.z += sh.z;
    acc.w += sh.w;
    if (b.resid) {
        const float4 rs = *(const float4*)(b.resid + (size_t)t * H + r);
        acc.x = rs.x + acc.x;
        acc.y = rs.y + acc.y;
        acc.z = rs.z + acc.z;
        acc.w = rs.w + acc.w;
    }
    *(float4*)(b.out + (size_t)t * H + r) = acc;
}

// Token-table entries a work-group of the gate/up kernel can need for T
// tokens (an upper bound over every routing): the kMT pipeline's units are at
// most the shared passes' cdiv(T, kMT) x SI / kSlice plus P x NSG for
// P <= cdiv(T (K + 1), kMT) + E + 1 passes (each expert adds at most one
// partial pass; K + 1 counts an MXFP4 shared expert's rows), the wide
// pipeline's at most Pw x NSG for Pw <= R / kMTR + R / (kMT + 1) + 1 passes
// (R = T (K + 1) rows; only experts of more than kMT rows have wide passes,
// cdiv(c, kMTR) each); a work-group gets at most cdiv(units, grid).
static uint32_t batched_tok_entries(uint32_t T, uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid) {
    auto cd = [](uint64_t a, uint64_t b) { return (a + b - 1u) / b; };
    const uint64_t R = (uint64_t)T * (K + 1u), NSG = cd(I / kSlice, kSG);
    const uint64_t units = cd(T, kMT) * (SI / kSlice) + (cd(R, kMT) + E + 1u) * NSG;
    const uint64_t wunits = (R / kMTR + R / (kMT + 1u) + 1u) * NSG;
    return (uint32_t)std::max(cd(units, grid) * kMT, cd(wunits, grid) * kMTR);
}
static size_t bup_lds(uint32_t T, uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid) {
    return tok_table_offset(E) + 2u * (size_t)batched_tok_entries(T, I, SI, E, K, grid);
}
uint32_t batched_max_tokens(uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid) {
    const size_t room = (size_t)decode_max_lds() - 3u * (size_t)kSlotB;
    uint32_t lo = 0, hi = 1u << 16;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1u) / 2u;
        if (bup_lds(mid, I, SI, E, K, grid) <= room) lo = mid;
        else hi = mid - 1u;
    }
    return lo;
}

uint32_t batched_max_experts() {
    // the GEMM kernels' LDS: the three activation slots and the expert tables
    const size_t lds = (size_t)decode_max_lds(), ring = 3u * (size_t)kSlotB;
    uint32_t e = 0;
    while (ring + gemm_tab_bytes(e + 16u) <= lds) e += 16u;
    return e;
}

int launch_batched(const DecodeArgs* d_args, const BatchArgs& b, uint32_t H, uint32_t I, uint32_t SI, uint32_t E,
                   uint32_t K, uint32_t n_cu, uint32_t phases, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    const size_t topk_lds = 4u * (2u * E + 64u);
    const size_t gemm_lds = gemm_tab_bytes(E);
    // the gate/up kernel's token table, sized for this call and a grid of
    // n_cu or more work-groups
    BatchArgs bt = b;
    bt.tcap = batched_tok_entries(b.T, I, SI, E, K, n_cu);
    size_t up_lds = bup_lds(b.T, I, SI, E, K, n_cu);
    if (up_lds + 3u * (size_t)kSlotB > (size_t)decode_max_lds()) return (int)hipErrorInvalidValue;
    // the GEMM kernels' wide units take their shape parameters as constants
    // at the GLM shape
    const bool glm = H == 6144u && I == 2048u && SI == 2048u && K == 8u;
    // (decided below with the down kernel's small-expert instantiation)
    const void* up = nullptr;
    // routed experts of few tokens (up to kSmallT; kSmallUpT at the GLM
    // shape): their down projection as bdown_kernel's streaming pipelines,
    // for every batch the shape allows (measured at the GLM shape, per call,
    // with the 1-4 token units: T = 64 -3 %, 128 -5 %, 512 -4 %, 1024
    // unchanged, where no expert is that small)
    // (WL_BATCHED_SMALL=0 keeps every expert in the grouped passes: the
    // same results bit for bit, which a GPU test compares)
    const char* small_env = getenv("WL_BATCHED_SMALL");
    const bool small = small_down_fits(H, I) && !(small_env && small_env[0] == '0');
    const void* down = glm ? (small ? (const void*)bdown_kernel<true, true> : (const void*)bdown_kernel<true, false>)
                           : (small ? (const void*)bdown_kernel<false, true> : (const void*)bdown_kernel<false, false>);
    // the gate/up side (experts of up to kSmallUpT tokens; GLM shape, and
    // the lists must fit the dynamic LDS)
    const bool small_up = small && glm && small_up_fits(H, I) &&
                          small_list_end(E) + 3u * (size_t)kSlotB <= (size_t)decode_max_lds();
    if (small_up) up_lds = std::max(up_lds, small_list_end(E));
    up = glm ? (small_up ? (const void*)bup_kernel<true, true> : (const void*)bup_kernel<true, false>)
             : (const void*)bup_kernel<false, false>;
    const struct { const void* fn; size_t lds; } attrs[] = {
        {(const void*)btopk_kernel, topk_lds}, {up, up_lds}, {down, gemm_lds}};
    for (const auto& at : attrs)
        if ((e = hipFuncSetAttribute(at.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)at.lds)) != hipSuccess)
            return (int)e;
    // The GEMM kernels walk their units with a grid stride, so their grid is
    // what the chip holds at once (the LDS ring allows one work-group per CU);
    // a larger grid would leave its second part waiting for the first.
    auto resident = [&](const void* fn, size_t lds) {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, kThreads, lds) != hipSuccess || nb < 1) nb = 1;
        return n_cu * (uint32_t)nb;
    };
    if (phases & kPhaseRoute) {
        hipLaunchKernelGGL(bnorm_kernel, dim3(b.T), dim3(kThreads), 0, s, d_args, b);
        // router: ~one work-group per CU; each token block's rows split over gx
        // work-groups (each norm row is read gx times, the router once per block)
        const uint32_t nblk = (b.T + kTB - 1) / kTB;
        const uint32_t gx = std::max(1u, std::min(n_cu / nblk, (E + kRR - 1) / kRR));
        hipLaunchKernelGGL(broute_kernel, dim3(gx, nblk), dim3(kThreads), 0, s, d_args, b);
        hipLaunchKernelGGL(btopk_kernel, dim3(b.T), dim3(kThreads), topk_lds, s, d_args, b);
        hipLaunchKernelGGL(bcount_kernel, dim3(E), dim3(64), 0, s, b, K);
        hipLaunchKernelGGL(bscatter_kernel, dim3(E), dim3(256), 0, s, b, E);
    }
    if (phases & kPhaseGemm) {
        // the shared expert's wide units when they fill the grid, and at the
        // GLM shape from two wide passes on (measured, per call: T = 128
        // -1 %, 256 and 512 -2 %; at T = 64, one pass, +2 %)
        BatchArgs bw = bt;
        const uint32_t gu = resident(up, up_lds), gd = resident(down, gemm_lds);
        const bool bf16_sh = !(b.flags & (kBatchNoShared | kBatchShared4));
        const bool wide_sh = glm && b.T >= 2u * kMTW;
        if (bf16_sh && (wide_sh || (b.T + kMTW - 1u) / kMTW * ((SI / kSlice + 1u) / 2u) >= gu))
            bw.flags |= kBatchWideSharedUp;
        if (bf16_sh && (wide_sh || (b.T + kMTW - 1u) / kMTW * ((H + 255u) / 256u) >= gd))
            bw.flags |= kBatchWideSharedDown;
        if (glm) {
            if (small_up) hipLaunchKernelGGL((bup_kernel<true, true>), dim3(gu), dim3(kThreads), up_lds, s, d_args, bw);
            else hipLaunchKernelGGL((bup_kernel<true, false>), dim3(gu), dim3(kThreads), up_lds, s, d_args, bw);
            if (small) hipLaunchKernelGGL((bdown_kernel<true, true>), dim3(gd), dim3(kThreads), gemm_lds, s, d_args, bw);
            else hipLaunchKernelGGL((bdown_kernel<true, false>), dim3(gd), dim3(kThreads), gemm_lds, s, d_args, bw);
        } else {
            hipLaunchKernelGGL((bup_kernel<false, false>), dim3(gu), dim3(kThreads), up_lds, s, d_args, bw);
            if (small) hipLaunchKernelGGL((bdown_kernel<false, true>), dim3(gd), dim3(kThreads), gemm_lds, s, d_args, bw);
            else hipLaunchKernelGGL((bdown_kernel<false, false>), dim3(gd), dim3(kThreads), gemm_lds, s, d_args, bw);
        }
    }
    if (phases & kPhaseCombine)
        hipLaunchKernelGGL(bcomb_kernel, dim3((H + 1023) / 1024, b.T), dim3(256), 0, s, b, H, K);
    return (int)hipGetLastError();
}

}  // namespace wl
