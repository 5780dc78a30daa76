// moe_decode.hip — gfx950 kernels of the bs=1 MoE decode layer.
//
// One persistent launch of G work-groups (one per CU, 8 wave64s each) runs a
// layer in two segments (the phased schedule launches each on its own). No
// grid barrier: values another work-group needs are written with agent-scope
// stores and carry a tag of this call, and the reader polls, with a bounded
// wait, until it sees that tag: a logit is a 64-bit word epoch << 32 | f32
// bits; a partial sum is a 32-bit word, the f32 rounded to 21 stored mantissa
// bits with the call's 2-bit tag (1, 2 or 3) in the freed low bits.
//
//   0  every work-group normalises the hidden state (RMSNorm, redundantly),
//      computes its router row and publishes the logit, and streams one
//      8-gate + 8-up tile of the bf16 shared expert, whose batches also read
//      the published logits on the way. Then the top-k, on every work-group
//      (sigmoid, +e_score_correction_bias, top-K with ties to the lowest index,
//      renormalise, x routed_scaling; src/glm_layer_runner.cuh:304-336), the
//      tile's SwiGLU and its 8 columns of the shared down projection, and one
//      routed unit (expert slot k, slice j): the 64 SwiGLU rows [64j, 64j+64)
//      of expert k (MXFP4 gate/up) times the 64 matching columns of its MXFP4
//      down projection, i.e. a split-K partial of expert k's output over all H
//      rows, weighted by w_k and added to the shared columns' partial. The
//      work-group's partial vector is published as tagged words.
//      reference: rms_norm_bf16, matvec_bf16 (router), dequant_matvec_mxfp4 x3
//      + silu_mul, shared expert; src/glm_primitives.cuh:35-62,87-116,
//      src/glm_kernels.cuh:63-110, src/glm_layer_runner.cuh:338-341,370-436
//   1  work-groups combine blocks of 32 output rows: the sum of the G partials
//      (fixed order), + the residual when one is given (src/glm_layer_runner.cuh:
//      403,428,436,675). A work-group takes a ticket from this call's counter
//      as it gets here and combines blocks ticket, ticket + G, ...: the first
//      to finish their own work do the combining.
//
// Splitting the down projection by the SwiGLU slice a work-group computed
// means no work-group waits for another one's SwiGLU output: the only
// cross-work-group waits are the logits and the partials. Work-group w runs
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
// block scale exactly (e2m1 x 2^(s-127) is a bf16 value, subnormal at s = 1,
// except at s = 254 with |e2m1| >= 2, which overflows to inf and turns the
// 3-piece product into NaN where an f32 product would give inf), low nibble =
// even column as in the reference (src/glm_kernels.cuh:4-33).
//
// Weight loads are 16 bytes per lane (one 1 KB request per wave instruction)
// and are issued in batches of kNB, two batches in flight per wave: a wave
// issues batch b+2 right after it has consumed batch b. Every batch is issued
// unconditionally (indices past the end are clamped to a valid address and
// their contribution masked), so the compiler's wait counts stay exact.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <vector>
#include "dev_common.h"
#include "internal.h"

namespace wl {

// Diagnostic builds (-DWL_TIMELINE) record a 100 MHz timestamp per work-group
// at each phase boundary; product builds compile WL_TL to nothing.
// A kernel names its record slot tl_slot (the decode kernel: its call's epoch
// mod kTlCalls), so back-to-back calls keep their own records.
#ifdef WL_TIMELINE
constexpr uint32_t kTlCalls = 64;
__device__ uint64_t g_tl[kTlCalls * kMaxGrid * 16];
#define WL_TL(i)                                                                                  \
    do {                                                                                          \
        if (threadIdx.x == 0)                                                                     \
            g_tl[((size_t)tl_slot * kMaxGrid + blockIdx.x) * 16 + (i)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define WL_TL(i) \
    do {         \
    } while (0)
#endif


// A cross-work-group value with this call's epoch: one 8-byte agent-scope
// store, so a reader that sees the epoch sees the value.
WL_DEV void st_tag(uint64_t* p, uint32_t epoch, float x) {
    __hip_atomic_store((__attribute__((address_space(1))) uint64_t*)p, ((uint64_t)epoch << 32) | __float_as_uint(x),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A partial sum with this call's tag (1-3): the f32 rounded to nearest at 21
// stored mantissa bits (the combine's error grows from 2.0e-7 to 2.5e-7 of
// the output scale at the GLM shape), the tag in the two freed low bits; one
// 4-byte agent-scope store, so a reader that sees the tag sees the value.
// Every call writes every word of the partial arrays, so a word still holding
// an older call's tag is stale (consecutive calls' tags differ).
WL_DEV void st_part(uint32_t* p, uint32_t tag, float x) {
    __hip_atomic_store((__attribute__((address_space(1))) uint32_t*)p, ((__float_as_uint(x) + 2u) & ~3u) | tag,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The same tagged word for the first level of the two-level combine: a plain
// store, which stays in the writer's XCD L2. The XCD's other work-groups read
// it there with non-temporal loads (which never return a line kept in the
// reader's L1). Measured on MI355X while 240 MB stream: 8 MB of agent-scope
// (write-through) 4-byte stores cost 6.1 us, plain ones 1.7 us.
WL_DEV void st_l1(uint32_t* p, uint32_t tag, float x) {
    *(__attribute__((address_space(1))) uint32_t*)p = ((__float_as_uint(x) + 2u) & ~3u) | tag;
}
// This work-group's XCD (hardware register XCC_ID).
WL_DEV uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
    return x;
}

// ---- the decode kernel -------------------------------------------------------
// GLM = true compiles the GLM shape (H 6144, I 2048, SI 2048, E 256, K 8) with
// every shape constant known; GLM = false reads the shapes from the record.
// The hidden state of a layer inside one chain launch (moe_chain_kernel):
// the previous layer's output arrives as epoch-tagged words (epoch << 32 |
// f32 bits, agent scope) in hx, which is also the residual; a layer whose
// output feeds the next writes it there the same way. A single-layer launch
// passes {null, 0, null}: plain input d.hidden, plain output d.out.
struct ChainIO {
    const uint64_t* hx_in;  // tagged input (and residual), or null
    uint32_t in_epoch;      // the epoch its words must carry
    uint64_t* hx_out;       // tagged output, or null
};

// One layer on this work-group. Returns false when the work-group left an
// aborted call (its partial words are written as they stand).
// SH4 = true: the shared expert is MXFP4 (NativeShared4) instead of bf16.
// LOOP = true: the layer body of a multi-layer launch. Its work-group and
// thread indices are re-read opaquely per layer, so that nothing derived
// from them is computed once before the layer loop and held (spilled) across
// the whole body.
template <bool GLM, bool SH4, bool LOOP>
__device__ __forceinline__ bool decode_layer(const DecodeArgs& a, const DecodeDyn& d, const ChainIO ch) {
#ifdef WL_TIMELINE
    const uint32_t tl_slot = d.epoch % kTlCalls;
#endif
    const uint32_t H = GLM ? 6144u : a.H, I = GLM ? 2048u : a.I, SI = GLM ? 2048u : a.SI,
                   E = GLM ? 256u : a.E, K = GLM ? 8u : a.K;
    uint32_t G = gridDim.x, w = blockIdx.x, tid = threadIdx.x;
    if constexpr (LOOP) {
        asm volatile("" : "+s"(G), "+s"(w));
        asm volatile("" : "+v"(tid));
    }
    __builtin_assume(tid < (uint32_t)kThreads);
    const uint32_t v = uni(tid >> 6) & 7u, lane = tid & 63, n = lane & 15, g = lane >> 4;
    const Plan P = Plan::make(H, I, SI, K, G);
    const LdsMap L = LdsMap::make(H, SI, E, K, P);
    const SyncMap SM = SyncMap::make();
    extern __shared__ __align__(16) uint8_t lds[];
    uint16_t* xp = (uint16_t*)(lds + L.xp);
    const uint32_t xps = H + 8;
    float* pv = (float*)(lds + L.pv);  // normalised input, then this work-group's partial, then combine staging
    uint16_t* rmp = (uint16_t*)(lds + L.rmp);
    constexpr uint32_t rps = kSlice + 8;
    float* red = (float*)(lds + L.red);
    float* tk_sc = (float*)(lds + L.topk);
    float* tk_ch = tk_sc + E;
    uint32_t* tk_idx = (uint32_t*)(tk_ch + E);
    float* tk_w = (float*)(tk_idx + 32);
    const uint8_t** tk_blk = (const uint8_t**)(lds + L.slots);
    uint32_t* misc = (uint32_t*)(lds + L.misc);  // [0..8) vote flags, [8] barrier flag
    float* smf = (float*)(misc + 16);           // [8] this tile's shared SwiGLU values
    // Two-level combine: work-group w writes its partial rows into slot w/8
    // of XCD w mod 8's region ([8][H/32][G/8][32] words), which only that
    // XCD's work-groups read. Work-groups are dispatched to the XCDs round
    // robin; one that finds itself elsewhere raises E_XCD (checked below).
    const bool xl2 = d.xl2();
    // row r of block b of this work-group's partial: word b * pstride + r of
    // a partial array (one-level: slot w of [H/32][G][32]; two-level: slot
    // w/8 of XCD w mod 8's [H/32][G/8][32])
    const uint32_t pstride = (xl2 ? G >> 3 : G) * kRowBlock;
    const uint32_t pbase = (xl2 ? ((w & 7u) * P.NB * (G >> 3) + (w >> 3)) : w) * kRowBlock;
    // the next call's combine-ticket counter starts at zero: cleared first
    // thing by the launch that holds the combine (the counter was last used
    // two calls back, which has ended)
    if (d.seg_hi() >= 1u && w == 0 && tid == 0) st_sync(a.sync + SM.ticket + d.ptag() % 3u, 0u);

    Batch bA, bB;
    using SB = std::conditional_t<SH4, SBatch4, SBatch>;
    SB sA, sB;

    // ================= segment 0: everything but the combine ====================
    if (d.seg_lo() == 0u) {
        WL_TL(0);
        // hidden state and norm weight first: they are consumed first
        constexpr int HV = kHV;
        float4 hv[HV];
        uint2 lv[HV];
        u32x4 hq[2 * HV];  // tagged input: the 8-byte words of float4 j at 32j, 32j + 16
        // (no norm weight: the resource is empty and its loads read zeros)
        const rsrc_t ln_rs = make_rsrc(d.ln_w ? (const void*)d.ln_w : (const void*)d.lslot, d.ln_w ? H * 2u : 0u);
        if (ch.hx_in) {
            const rsrc_t hx_rs = make_rsrc(ch.hx_in, H * 8u);
#pragma unroll
            for (int i = 0; i < HV; i++) {
                const uint32_t j = tid + kThreads * i;
                hq[2 * i] = bld16_ag(hx_rs, 32u * j, 0u);
                hq[2 * i + 1] = bld16_ag(hx_rs, 32u * j + 16u, 0u);
            }
        } else {
            const rsrc_t hid_rs = make_rsrc(d.hidden, H * 4u);
#pragma unroll
            for (int i = 0; i < HV; i++) {
                const uint32_t j = tid + kThreads * i;  // float4 j = elements [4j, 4j+4)
                hv[i] = __builtin_bit_cast(float4, bld16(hid_rs, 16u * j, 0u));
            }
        }
#pragma unroll
        for (int i = 0; i < HV; i++) {
            const uint32_t j = tid + kThreads * i;
            lv[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ln_rs, (int)(8u * j), 0, 0));
        }
        // the first router row of this work-group
        constexpr int RCH = kRCH;
        const uint32_t nch = H / 8;
        const rsrc_t rt_rs = make_rsrc(d.router_w, E * H * 2u);
        u32x4 rw[RCH];
#pragma unroll
        for (int m = 0; m < RCH; m++) rw[m] = bld16_nt(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), min(w, E - 1u) * H * 2u);
        // routing inputs that do not depend on this call's data, for experts
        // e = tid (E <= 512; the rest later): consumed long after they land
        // (their addresses are not preloaded: issued after the loads above,
        // which the scheduling barrier keeps ahead of the wait for them)
        __builtin_amdgcn_sched_barrier(0);
        const rsrc_t bs_rs = make_rsrc(d.bias, E * 4u), sl_rs = make_rsrc(d.slot_tab, E * 8u);
        const uint32_t bias0 = __builtin_amdgcn_raw_buffer_load_b32(bs_rs, (int)(4u * tid), 0, 0);
        const uint64_t slot0 = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(sl_rs, (int)(8u * tid), 0, 0));

        // shared gate/up tiles (8 gate + 8 up rows). At G = SI/8 (GLM) the
        // tiles are mapped so that the 32 work-groups of one XCD hold 32
        // consecutive tiles: their down-projection columns share lines.
        const uint32_t nsg = SI / 8, nkt = H / 32;
        const bool xcd_map = nsg == G && (G & 7u) == 0u;
        auto tile_of = [&](uint32_t i) {  // i-th tile of this work-group
            const uint32_t t = w + G * i;
            return xcd_map ? (w & 7u) * (G / 8u) + (w >> 3) : t;
        };
        // bf16: 32-column k tiles (1 KB chunk T*(H/32)+kt of the native shared
        // expert); MXFP4: 128-column k tiles of the tile's gate/up chunks
        // (NativeLayout gu, 1 KB each, kSNB4 per batch, scales from gus)
        const uint32_t nkg = H / 128;
        const uint32_t sg_per = SH4 ? cdiv(nkg, 8u) : cdiv(nkt, 8u);  // k tiles per wave: [v*sg_per, +sg_per)
        const uint32_t sg_nb = at_least2(cdiv(sg_per, SH4 ? (uint32_t)kSNB4 : (uint32_t)kSNB));
        const NativeShared NS = NativeShared::make(H, SI);
        const NativeShared4 NS4 = NativeShared4::make(H, SI);
        const NativeLayout NL4 = NativeLayout::make(H, SI);
        const rsrc_t sg_rs = SH4 ? make_rsrc(d.sh_native + NS4.blk + NL4.gu, (uint32_t)(NL4.gus - NL4.gu))
                                 : make_rsrc(d.sh_native + NS.sgu, (uint32_t)(NS.sdn - NS.sgu));
        const rsrc_t sgs_rs = make_rsrc(d.sh_native + NS4.blk + NL4.gus, SH4 ? (uint32_t)(NL4.dn - NL4.gus) : 0u);
        // every shared batch also reads the logit slot of expert min(tid, E-1)
        // (agent scope): the logits published while the shared expert streams
        // are collected on the way, without a separate round trip
        const rsrc_t ls_rs = make_rsrc(d.lslot, E * 8u);
        const uint32_t pe = min(tid, E - 1u);
        auto sg_issue = [&](uint32_t tile, uint32_t b, SB& B) {
            if constexpr (SH4) {
                // items past this wave's share or past the tile read zeros
                // without touching memory: their lane offset lies past the
                // resource (the lane offset is what the range check sees)
                const uint32_t tl = min(tile, nsg - 1u);
                const uint32_t voff = tl * nkg * 1024u + 16u * lane;
                const uint32_t soff0 = tl * cdiv(nkg, 16u) * 1024u + 16u * lane;
#pragma unroll
                for (int i = 0; i < kSNB4; i++) {
                    const uint32_t m = b * kSNB4 + i, kt = v * sg_per + m;
                    const bool ok = m < sg_per && kt < nkg;
                    B.w[i] = bld16_nt(sg_rs, ok ? voff + kt * 1024u : kOOB, 0u);
                    B.s[i] = __builtin_amdgcn_raw_buffer_load_b32(
                        sgs_rs, (int)(ok ? soff0 + (kt / 16u) * 1024u + 4u * ((kt % 16u) / 4u) : kOOB), 0, 0);
                }
            } else {
                const uint32_t voff = min(tile, nsg - 1u) * nkt * 1024u + 16u * lane;
                const uint32_t kt0 = v * sg_per + b * kSNB;
#pragma unroll
                for (int i = 0; i < kSNB; i++) B.w[i] = bld16_nt(sg_rs, voff, (kt0 + i) * 1024u);
            }
            B.pl = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(ls_rs, (int)(8u * pe), 0, kSC1));
        };
        f32x4 gacc;
        bool seen = false;  // this call's logit of expert tid was read (only tid < E)
        uint32_t lbits = 0;
        auto sg_consume = [&](uint32_t b, const SB& B) {
            if constexpr (SH4) {
#pragma unroll
                for (int i = 0; i < kSNB4; i++) {
                    const uint32_t m = b * kSNB4 + i, kt = v * sg_per + m;
                    const bool valid = m < sg_per && kt < nkg;
                    // a masked item's nibbles are zero (read past the
                    // resource) and are selected as zero besides: +0 under any scale
                    const float sc = valid ? e8m0f((B.s[i] >> (8u * (kt % 4u))) & 0xFFu) : 0.f;
#pragma unroll
                    for (int jj = 0; jj < 4; jj++)
                        gacc = mma(a_rows3(xp, xps, n, kt * 128u + 32u * g + 8u * jj, valid),
                                   fp4x8_bf16(valid ? B.w[i][jj] : 0u, sc), gacc);
                }
            } else {
#pragma unroll
                for (int i = 0; i < kSNB; i++) {
                    const uint32_t m = b * kSNB + i, kt = v * sg_per + m;
                    const bool valid = m < sg_per && kt < nkt;
                    const u32x4 z = {0u, 0u, 0u, 0u};
                    gacc = mma(a_rows3(xp, xps, n, kt * 32u + 8u * g, valid), as_bf16x8(valid ? B.w[i] : z), gacc);
                }
            }
            // threads tid >= E read slot E - 1 only to keep every batch the
            // same shape; they own no expert and never record a logit
            if (tid < E && !seen && (uint32_t)(B.pl >> 32) == d.epoch) {
                seen = true;
                lbits = (uint32_t)B.pl;
            }
        };
        // shared down, columns [8t, 8t+8) of every row: thread tid takes rows
        // tid + 512*i, 16 bytes each (zero past the end)
        // rows per thread: H / 512 at the GLM shape, 16 (H <= 8192) otherwise;
        // the resource of a tile ends at its last row, so rows past H read
        // zeros without touching memory (the next tile's rows are not fetched)
        // MXFP4: 4 nibble bytes (dn8) and one scale byte (dns8) per row
        constexpr int SDV = GLM ? 12 : 16;
        u32x4 sdw[SH4 ? 1 : SDV];
        uint32_t sdq[SH4 ? SDV : 1], sdsc[SH4 ? SDV : 1];
        auto sd_issue = [&](uint32_t tile) {
            const uint32_t tl = min(tile, nsg - 1u);
            if constexpr (SH4) {
                const rsrc_t dq_rs = make_rsrc(d.sh_native + NS4.dn8 + (size_t)tl * H * 4u, H * 4u);
                const rsrc_t dsc_rs = make_rsrc(d.sh_native + NS4.dns8 + (size_t)(tl / 4u) * H, H);
#pragma unroll
                for (int i = 0; i < SDV; i++) {  // row r = tid + 512 i of the tile (zeros past H)
                    const uint32_t r = tid + kThreads * i;
                    sdq[i] = __builtin_amdgcn_raw_buffer_load_b32(dq_rs, (int)(r < H ? 4u * r : kOOB), 0, kNT);
                    sdsc[i] = bld1(dsc_rs, r < H ? r : kOOB, 0u);
                }
            } else {
                const rsrc_t sd_rs = make_rsrc(d.sh_native + NS.sdn + (size_t)tl * H * 16u, H * 16u);
#pragma unroll
                for (int i = 0; i < SDV; i++) {  // row r = tid + 512 i of the tile: 16 bytes (zeros past H)
                    const uint32_t r = tid + kThreads * i;
                    sdw[i] = bld16_nt(sd_rs, r < H ? 16u * r : kOOB, 0u);
                }
            }
        };
        const uint32_t tile0 = tile_of(0);
        sg_issue(tile0, 0, sA);
        sg_issue(tile0, 1, sB);
        if (xl2 && tid == 0 && xcc_id() != (w & 7u)) raise_error(a.sync, SM, E_XCD, d.epoch);

        if (ch.hx_in) {
            // the previous layer's output: every word of this thread's float4s
            // must carry its epoch; stale ones (its combine still running)
            // are read again, bounded, the error word ending the wait too
            const uint32_t e = ch.in_epoch;
            auto fresh = [&](int i) {
                return (hq[2 * i].y == e) & (hq[2 * i].w == e) & (hq[2 * i + 1].y == e) & (hq[2 * i + 1].w == e);
            };
            const rsrc_t hx_rs = make_rsrc(ch.hx_in, H * 8u);
            uint32_t stale = 0;
#pragma unroll
            for (int i = 0; i < HV; i++)
                if (tid + kThreads * i < H / 4u && !fresh(i)) stale |= 1u << i;
            for (uint32_t spins = 0; stale != 0u; spins++) {
                if (spins >= (1u << 20)) {
                    raise_error(a.sync, SM, E_SPIN, d.epoch);
                    break;
                }
                if ((spins & 63u) == 63u && aborted(a.sync, SM, d.epoch)) break;
                __builtin_amdgcn_s_sleep(2);
#pragma unroll
                for (int i = 0; i < HV; i++) {
                    if ((stale >> i) & 1u) {
                        const uint32_t j = tid + kThreads * i;
                        hq[2 * i] = bld16_ag(hx_rs, 32u * j, 0u);
                        hq[2 * i + 1] = bld16_ag(hx_rs, 32u * j + 16u, 0u);
                    }
                }
#pragma unroll
                for (int i = 0; i < HV; i++)
                    if (((stale >> i) & 1u) && fresh(i)) stale &= ~(1u << i);
            }
#pragma unroll
            for (int i = 0; i < HV; i++)
                hv[i] = make_float4(__uint_as_float(hq[2 * i].x), __uint_as_float(hq[2 * i].z),
                                    __uint_as_float(hq[2 * i + 1].x), __uint_as_float(hq[2 * i + 1].z));
        }
        // RMSNorm: w * (x * (1/sqrt(mean(x^2) + eps))) in fp32
        // (tools/ref_glm_chain.py:63-80; src/glm_primitives.cuh:35-62)
        const float rinv = norm_rinv(hv, red, H, a.eps);
        float* xn = pv;
#pragma unroll
        for (int i = 0; i < HV; i++) {
            const uint32_t j = tid + kThreads * i;
            if (j < H / 4) {
                const float xs[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
                const uint32_t ls[4] = {lv[i].x & 0xFFFFu, lv[i].x >> 16, lv[i].y & 0xFFFFu, lv[i].y >> 16};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float x = norm_value(xs[c], rinv, d.ln_w != nullptr, ls[c]);
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
        if (tid < E) {
            tk_ch[tid] = __uint_as_float(bias0);  // the bias until topk_score replaces it
            tk_blk[tid] = (const uint8_t*)slot0;
        }
        for (uint32_t e = tid + kThreads; e < E; e += kThreads) {
            tk_ch[e] = gld(d.bias + e);
            tk_blk[e] = gld(d.slot_tab + e);
        }
        lds_barrier();
        WL_TL(1);

        // router rows r = w + G*i (bf16 x f32, fp32 accumulate); each logit
        // is published as one 64-bit word (epoch << 32 | bits) with an
        // agent-scope store: a reader that sees this call's epoch has the value
        for (uint32_t r = w, first = 1; r < E; r += G, first = 0) {
            if (!first) {
#pragma unroll
                for (int m = 0; m < RCH; m++) rw[m] = bld16_nt(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), r * H * 2u);
            }
            router_publish(router_partial(rw, xn, nch), red, d.lslot, r, d.epoch);
        }
        WL_TL(2);

        // ---- top-k (runs after the first shared tile's gate/up, whose
        // batches collected most logits): every logit of this call must be
        // present; slots still holding an older epoch are re-read
        auto route = [&]() -> bool {
            if (tid < E && seen) {
                topk_score(__uint_as_float(lbits), tk_ch[tid], tid, tk_sc, tk_ch);
                if (w == 0) gst(a.logits + tid, __uint_as_float(lbits));
            }
            uint32_t done = seen ? 1u : 0u;  // bit i: expert tid + 512*i scored (tk_ch[e] then holds its choice)
            for (uint32_t spins = 0;; spins++) {
                bool mine = true;
                for (uint32_t i = 0, e = tid; e < E; i++, e += kThreads) {
                    if ((done >> i) & 1u) continue;
                    const uint64_t x = __hip_atomic_load((__attribute__((address_space(1))) uint64_t*)(d.lslot + e),
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((uint32_t)(x >> 32) == d.epoch) {
                        topk_score(__uint_as_float((uint32_t)x), tk_ch[e], e, tk_sc, tk_ch);
                        if (w == 0) gst(a.logits + e, __uint_as_float((uint32_t)x));
                        done |= 1u << i;
                    } else {
                        mine = false;
                    }
                }
                if (block_all(mine, misc)) break;
                // every lane of a wave sees the same abort word (one load);
                // a wave that leaves early drops out of the later barriers,
                // and the others leave at their next spin
                if (spins > (1u << 20) || aborted(a.sync, SM, d.epoch)) {
                    if (tid == 0 && spins > (1u << 20)) raise_error(a.sync, SM, E_SPIN, d.epoch);
                    return false;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            WL_TL(4);
            if (E <= 256u) topk_argmax(E, K, tk_sc, tk_ch, tk_idx, tk_w);
            else topk_rank(E, K, tk_sc, tk_ch, tk_idx, tk_w);
            WL_TL(5);
            if (w == 0 && tid < K) {
                gst(a.idx + tid, (int32_t)tk_idx[tid]);
                gst(a.topw + tid, topk_weight(a, K, tk_w, tid));
            }
            return true;
        };

        // pv -> rows [32b, 32b+32) into block b, slot w of dst ([H/32][G][32];
        // two-level: slot w/8 of XCD w mod 8's block b), tagged with this
        // call's tag (each thread stores the rows it wrote)
        auto publish = [&](uint32_t* dst) {
            for (uint32_t r = tid; r < H; r += kThreads) {
                uint32_t* const p = dst + pbase + (size_t)(r / kRowBlock) * pstride + r % kRowBlock;
                if (xl2) st_l1(p, d.ptag(), pv[r]);
                else st_part(p, d.ptag(), pv[r]);
            }
        };
        // A work-group that leaves an aborted call still writes its words (pv
        // as it stands), so the arrays keep holding one call's tags.
        auto leave = [&]() {
            publish(a.part);
            if (d.taps()) publish(a.tsh);
        };
        // shared expert: SwiGLU of each tile's 8 rows, then those 8 columns of
        // the down projection applied to every output row, into pv
        const uint32_t ntiles = w < nsg ? cdiv(nsg - w, G) : 0u;
        for (uint32_t i = tid; i < H; i += kThreads) pv[i] = 0.f;  // xn is no longer needed
        // the down columns of a tile: pv[r] += sum_c sdw[r][c] * smf[c]
        auto sd_compute = [&]() {
            const float4 m0 = *(const float4*)smf, m1 = *(const float4*)(smf + 4);
            if constexpr (SH4) {
#pragma unroll
                for (int i = 0; i < SDV; i++) {
                    const uint32_t r = tid + kThreads * i;
                    if (r < H) {
                        const bf16x8 wv = fp4x8_bf16(sdq[i], e8m0f(sdsc[i]));
                        float x = 0.f;
                        x = fmaf((float)wv[0], m0.x, x);
                        x = fmaf((float)wv[1], m0.y, x);
                        x = fmaf((float)wv[2], m0.z, x);
                        x = fmaf((float)wv[3], m0.w, x);
                        x = fmaf((float)wv[4], m1.x, x);
                        x = fmaf((float)wv[5], m1.y, x);
                        x = fmaf((float)wv[6], m1.z, x);
                        x = fmaf((float)wv[7], m1.w, x);
                        pv[r] += x;
                    }
                }
                return;
            }
#pragma unroll
            for (int i = 0; i < SDV; i++) {
                const uint32_t r = tid + kThreads * i;
                if (r < H) {
                    float x = 0.f;
                    x = fmaf(bf2f(sdw[i].x & 0xFFFFu), m0.x, x);
                    x = fmaf(bf2f(sdw[i].x >> 16), m0.y, x);
                    x = fmaf(bf2f(sdw[i].y & 0xFFFFu), m0.z, x);
                    x = fmaf(bf2f(sdw[i].y >> 16), m0.w, x);
                    x = fmaf(bf2f(sdw[i].z & 0xFFFFu), m1.x, x);
                    x = fmaf(bf2f(sdw[i].z >> 16), m1.y, x);
                    x = fmaf(bf2f(sdw[i].w & 0xFFFFu), m1.z, x);
                    x = fmaf(bf2f(sdw[i].w >> 16), m1.w, x);
                    pv[r] += x;
                }
            }
        };
        // The last tile's down columns are applied after the first routed
        // loads are issued: its rows stay in flight meanwhile, so HBM keeps
        // streaming through the top-k and into the routed units.
        bool sd_pending = false, routed = false;
        for (uint32_t ti = 0; ti < ntiles; ti++) {
            const uint32_t tile = tile_of(ti);
            if (ti != 0) {
                sg_issue(tile, 0, sA);
                sg_issue(tile, 1, sB);
            }
            gacc = f32x4{0.f, 0.f, 0.f, 0.f};
            pingpong(sg_nb, sA, sB, [&](uint32_t b, SB& B) { sg_issue(tile, b, B); }, sg_consume);
            // the tile's shared-down rows are issued only now: issued with the
            // last gate/up batch they delay it (the memory system serves both
            // together), and with it the top-k
            sd_issue(tile);
            if (lane < 16) red[v * 64 + n] = sum3(gacc);
            if (!routed) {
                if (!route()) {
                    leave();
                    return false;
                }
                routed = true;
            }
            lds_barrier();
            if (tid < 8) {
                float gs = 0.f, us = 0.f;
#pragma unroll
                for (int wv = 0; wv < kWaves; wv++) {
                    gs += red[wv * 64 + tid];
                    us += red[wv * 64 + 8 + tid];
                }
                const float mid = silu_mul(gs, us);
                smf[tid] = mid;
                gst(a.smid + tile * 8 + tid, mid);
            }
            lds_barrier();
            if (ti + 1u < ntiles) {
                sd_compute();
                lds_barrier();
            } else {
                sd_pending = true;
            }
        }
        if (!routed && !route()) {
            leave();
            return false;
        }
        // the deferred down columns, then (taps on) the shared-expert
        // contribution alone, published for the tap
        bool tsh_pending = d.taps() != 0;
        auto finish_shared = [&]() {
            if (sd_pending) {
                sd_compute();
                sd_pending = false;
            }
            if (tsh_pending) {
                lds_barrier();
                publish(a.tsh);
                tsh_pending = false;
            }
        };
        WL_TL(3);

        // ---- routed units u = w + G*i: items are gate/up k tiles (128 wide,
        // this wave's 8+8 row tile), then down row pairs (32 rows x the
        // slice's 64 columns), each wave a contiguous range of them
        const uint32_t nq = H / 32;
        const uint32_t dq_per = cdiv(cdiv(nq, 8u), (uint32_t)kNB) * kNB;  // row pairs per wave: [v*dq_per, +dq_per)
        const uint32_t nbg = cdiv(nkg, (uint32_t)kNB);
        const uint32_t nbd = cdiv(dq_per, (uint32_t)kNB);
        const uint32_t nbr = nbg + nbd;  // >= 2
        const uint8_t* blk = nullptr;
        uint32_t uk = 0, uj = 0;
        float wk = 0.f;
        // at most one routed unit per work-group (GLM: exactly one): its down
        // items publish the partial rows directly
        const bool direct = P.U <= G && w < P.U;
        rsrc_t r_rs = make_rsrc(d.router_w, 16u);  // rebound per unit
        const rsrc_t prs = make_rsrc(a.part, (uint32_t)(4u * part_words(H, G)));  // the partials (16-byte stores)
        uint32_t gu_voff = 0, gus_voff = 0, dn_voff = 0, dns_voff = 0;
        // Native block: the gate/up items of this wave are 1 KB chunks
        // [tile*(H/128) + kt], the down items [slice*(H/32) + q]; one 16-byte
        // scale chunk per batch. Branch-free: offsets are selected, then one
        // block of loads (loads on two paths would be joined by register copies
        // that wait for them).
        auto r_issue = [&](uint32_t b, Batch& B) {
            const bool gu = b < nbg;
            const uint32_t i0 = gu ? b * kNB : v * dq_per + (b - nbg) * kNB;
            const uint32_t wv = gu ? gu_voff : dn_voff;
#pragma unroll
            for (int i = 0; i < kNB; i++) B.w[i] = bld16_nt(r_rs, wv, (i0 + i) * 1024u);
            // a scale chunk serves 16 items, i.e. two batches: default policy
            // (not the streaming hint), so the second batch's load hits in L2
            B.sv = bld16(r_rs, gu ? gus_voff : dns_voff, (i0 / 16u) * 1024u);
        };
        f32x4 racc;
        bf16x8 A0, A1;
        auto r_consume = [&](uint32_t b, const Batch& B) {
            if (b < nbg) {
                const BatchScales bs = batch_scales(B, b * kNB);
#pragma unroll
                for (int i = 0; i < kNB; i++) {
                    const uint32_t kt = b * kNB + i;
                    const bool valid = kt < nkg;
                    // a masked item reads another tile (or zeros past the
                    // block): its nibbles are selected as zero, so its B
                    // operand is +0 under any scale (no item is masked at the
                    // GLM shape, where the select folds away)
                    const float sc = valid ? e8m0f(batch_scale8(bs, i)) : 0.f;
#pragma unroll
                    for (int jj = 0; jj < 4; jj++)
                        racc = mma(a_rows3(xp, xps, n, kt * 128u + 32u * g + 8u * jj, valid),
                                   fp4x8_bf16((GLM || valid) ? B.w[i][jj] : 0u, sc), racc);
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
                    WL_TL(7);
                    // down A operands: k groups of lane g hold slice columns
                    // {0,32,8,40}[g] (+16 for the second), matching the
                    // lane order the row-pair swap below produces
                    const uint32_t c0 = 32u * (g & 1u) + 8u * (g >> 1);
                    A0 = a_rows3(rmp, rps, n, c0, true);
                    A1 = a_rows3(rmp, rps, n, c0 + 16u, true);
                }
            } else {
                const uint32_t m0 = (b - nbg) * kNB;
                const BatchScales bs = batch_scales(B, v * dq_per + m0);
#pragma unroll
                for (int i = 0; i < kNB; i++) {
                    const uint32_t sbyte = batch_scale8(bs, i);
                    // lane (n, g) holds 16 bytes of row n + 16*(g>>1): columns
                    // [32*(g&1), +32) of the slice, and that block's scale.
                    // One swap of lane halves turns dwords (0,1) into the B
                    // operand of rows n (lanes 0-31 keep theirs, lanes 32-63
                    // take the lower half's dword 1) and of rows n + 16.
                    const uint32_t m = m0 + i, q = v * dq_per + m;
                    const bool valid = m < dq_per && q < nq;
                    uint32_t sx, sy, x01, y01, x23, y23;
                    const uint32_t sv = __float_as_uint(e8m0f(sbyte));
                    swap32(sv, sv, sx, sy);
                    swap32(B.w[i][0], B.w[i][1], x01, y01);
                    swap32(B.w[i][2], B.w[i][3], x23, y23);
                    const float scx = __uint_as_float(sx), scy = __uint_as_float(sy);
                    f32x4 d0 = mma(A0, fp4x8_bf16(x01, scx), f32x4{0.f, 0.f, 0.f, 0.f});
                    d0 = mma(A1, fp4x8_bf16(x23, scx), d0);
                    f32x4 d1 = mma(A0, fp4x8_bf16(y01, scy), f32x4{0.f, 0.f, 0.f, 0.f});
                    d1 = mma(A1, fp4x8_bf16(y23, scy), d1);
                    const float s0 = sum3(d0);
                    const float s1 = __shfl(sum3(d1), (lane - 16u) & 63u, 64);
                    // rows [32q, 32q+32): this unit's weighted contribution
                    if (valid && lane < 32) pv[q * 32u + lane] += wk * (lane < 16 ? s0 : s1);
                }
                if (direct) {
                    // with one unit per work-group the batch's rows are final:
                    // each lane publishes 4 consecutive rows of them with one
                    // 16-byte store (a wave's LDS accesses complete in order).
                    // Measured while 240 MB stream: 16-byte agent-scope stores
                    // cost a third as much per byte as 4-byte ones.
                    asm volatile("" ::: "memory");
                    const uint32_t mq = m0 + lane / 8u, q = v * dq_per + mq, c4 = 4u * (lane % 8u);
                    if (mq < dq_per && q < nq) {
                        const float4 x4 = *(const float4*)(pv + 32u * q + c4);
                        const uint32_t tag = d.ptag();
                        const u32x4 t4 = {((__float_as_uint(x4.x) + 2u) & ~3u) | tag, ((__float_as_uint(x4.y) + 2u) & ~3u) | tag,
                                          ((__float_as_uint(x4.z) + 2u) & ~3u) | tag, ((__float_as_uint(x4.w) + 2u) & ~3u) | tag};
                        const int off = (int)(4u * (pbase + q * pstride + c4));
                        if (xl2) __builtin_amdgcn_raw_buffer_store_b128(t4, prs, off, 0, 0);
                        else __builtin_amdgcn_raw_buffer_store_b128(t4, prs, off, 0, kSC1);
                    }
                }
            }
        };

        bool first_unit = true;
        bool ran = false;  // a unit's down items published this work-group's rows
        for (uint32_t u = w; u < P.U; u += G) {
            uk = u % K;
            uj = u / K;
            blk = uni_ptr(tk_blk[tk_idx[uk]]);
            wk = topk_weight(a, K, tk_w, uk);
            if (blk == nullptr) {
                if (tid == 0) raise_error(a.sync, SM, E_NOT_RESIDENT, d.epoch);
                continue;
            }
            if (!first_unit) lds_barrier();  // rmp of the previous unit fully read
            first_unit = false;
            ran = true;
            {
                const NativeLayout NL = NativeLayout::make(H, I);
                const uint32_t tile = uj * (kSlice / 8u) + v;  // this wave's 8+8 row tile
                r_rs = make_rsrc(blk, (uint32_t)NL.total);
                gu_voff = (uint32_t)NL.gu + tile * nkg * 1024u + 16u * lane;
                gus_voff = (uint32_t)NL.gus + tile * cdiv(nkg, 16u) * 1024u + 16u * lane;
                dn_voff = (uint32_t)NL.dn + uj * nq * 1024u + 16u * lane;
                dns_voff = (uint32_t)NL.dns + uj * cdiv(nq, 16u) * 1024u + 16u * lane;
            }
            r_issue(0, bA);
            r_issue(1, bB);
            finish_shared();  // pv is read by the down items, after the gate/up barrier
            racc = f32x4{0.f, 0.f, 0.f, 0.f};
            pingpong(nbr, bA, bB, r_issue, r_consume);
            WL_TL(8);
        }
        finish_shared();
        lds_barrier();

        // ---- publish this work-group's partial (the combine of block b reads
        // its G slots contiguously), unless the down items already did. No
        // barrier follows: the combine waits for the tags of the words it
        // reads.
        if (!(direct && ran)) publish(a.part);
        lds_barrier();  // pv is the combine's staging area
        WL_TL(9);
    }

    // ================= segment 1: combine ========================================
    // out[r] = sum over work-groups of their partials (fixed order), + resid.
    if (d.seg_hi() >= 1u) {
        constexpr uint32_t RB = kRowBlock;
        const uint32_t Gx = G >> 3, xw = w & 7u, iw = w >> 3;
        float* fin = pv;                   // [G][32]
        float* f2 = fin + (size_t)G * RB;  // [16][32]
        // Stages n 16-byte chunks (four tagged words each) into fin (chunk c
        // at fin + 4c): chunk c is read from byte offset off(c) of resource rs
        // with cache policy aux. All of a thread's chunks are issued at once;
        // a chunk whose words do not all carry this call's tag (their writers
        // have not finished: an older call's tag) is read again, all of a
        // thread's stale chunks in flight together, until the tag shows
        // (bounded; the error word ends the wait too). Ends with a barrier.
        auto gather = [&](rsrc_t rs, uint32_t n, auto off, int aux) {
            const uint32_t tag = d.ptag();
            constexpr uint32_t kGrp = 4;
            auto ld = [&](uint32_t ch) -> u32x4 {
                const uint32_t o = ch < n ? off(ch) : kOOB;
                return aux == kNT ? __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, kNT)
                                  : __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, kSC1);
            };
            for (uint32_t c0 = 0; c0 < n; c0 += kThreads * kGrp) {
                u32x4 q[kGrp];
#pragma unroll
                for (uint32_t i = 0; i < kGrp; i++) q[i] = ld(c0 + tid + kThreads * i);
                uint32_t stale = 0;  // bit i: chunk i still holds an older call's tag
                for (uint32_t spins = 0;; spins++) {
#pragma unroll
                    for (uint32_t i = 0; i < kGrp; i++) {
                        const uint32_t ch = c0 + tid + kThreads * i;
                        const bool mine = ch < n && (spins == 0 || ((stale >> i) & 1u));
                        if (!mine) continue;
                        if (((q[i].x & 3u) == tag) & ((q[i].y & 3u) == tag) & ((q[i].z & 3u) == tag) &
                            ((q[i].w & 3u) == tag)) {
                            *(float4*)(fin + 4u * ch) = make_float4(__uint_as_float(q[i].x & ~3u), __uint_as_float(q[i].y & ~3u),
                                                                    __uint_as_float(q[i].z & ~3u), __uint_as_float(q[i].w & ~3u));
                            stale &= ~(1u << i);
                        } else {
                            stale |= 1u << i;
                        }
                    }
                    if (stale == 0u) break;
                    if (spins >= (1u << 20)) {
                        raise_error(a.sync, SM, E_SPIN, d.epoch);
                        break;
                    }
                    if ((spins & 63u) == 63u && aborted(a.sync, SM, d.epoch)) break;
                    __builtin_amdgcn_s_sleep(2);
#pragma unroll
                    for (uint32_t i = 0; i < kGrp; i++)  // every stale chunk again, all in flight together
                        if ((stale >> i) & 1u) q[i] = ld(c0 + tid + kThreads * i);
                }
            }
            lds_barrier();
        };
        // one-level: sum of the G slots of block blkr of src ([H/32][G][32]);
        // the result is in threads 0..31
        auto block_total = [&](const uint32_t* src, uint32_t blkr) -> float {
            gather(make_rsrc(src + (size_t)blkr * G * RB, G * RB * 4u), G * RB / 4u,
                   [](uint32_t ch) { return 16u * ch; }, kSC1);
            {  // 16 groups of work-groups, then the 16 group sums
                const uint32_t rr = tid % RB, grp = tid / RB;
                float sum = 0.f;
                for (uint32_t ww = grp; ww < G; ww += 16u) sum += fin[ww * RB + rr];
                f2[grp * RB + rr] = sum;
            }
            lds_barrier();
            float o = 0.f;
            if (tid < RB) {
#pragma unroll
                for (int gi = 0; gi < 16; gi++) o += f2[gi * RB + tid];
            }
            lds_barrier();
            return o;
        };
        // two-level, first level: this work-group sums blocks iw + Gx*j of its
        // XCD (the G/8 slots of each, in slot order, read from the XCD's L2)
        // and publishes each sum with agent-scope tagged stores into slot xw
        // of the block's second-level words ([H/32][8][32] after the H x G
        // first-level words)
        auto xcd_level = [&](uint32_t* src) {
            const uint32_t nb1 = iw < P.NB ? cdiv(P.NB - iw, Gx) : 0u, cpb = Gx * (RB / 4u);
            const rsrc_t rs = make_rsrc(src + (size_t)xw * P.NB * Gx * RB, P.NB * Gx * RB * 4u);
            gather(rs, nb1 * cpb, [&](uint32_t ch) { return ((iw + Gx * (ch / cpb)) * Gx * RB + 4u * (ch % cpb)) * 4u; },
                   kNT);
            for (uint32_t t = tid; t < nb1 * RB; t += kThreads) {
                const uint32_t j = t / RB, rr = t % RB;
                float sum = 0.f;
                for (uint32_t sl = 0; sl < Gx; sl++) sum += fin[(j * Gx + sl) * RB + rr];
                st_part(src + (size_t)H * G + ((size_t)(iw + Gx * j) * 8u + xw) * RB + rr, d.ptag(), sum);
            }
            lds_barrier();  // fin is staged again next
        };
        // two-level, second level: the 8 XCD sums of block blkr, in XCD order;
        // the result is in threads 0..31
        auto xcd_total = [&](const uint32_t* src, uint32_t blkr) -> float {
            gather(make_rsrc(src + (size_t)H * G + (size_t)blkr * 8u * RB, 8u * RB * 4u), 8u * RB / 4u,
                   [](uint32_t ch) { return 16u * ch; }, kSC1);
            float o = 0.f;
            if (tid < RB) {
#pragma unroll
                for (int x = 0; x < 8; x++) o += fin[x * RB + tid];
            }
            lds_barrier();
            return o;
        };
        if (xl2) {
            if (d.seg_lo() >= 1u && tid == 0 && xcc_id() != xw) raise_error(a.sync, SM, E_XCD, d.epoch);
            xcd_level(a.part);
            if (d.taps()) xcd_level(a.tsh);
            WL_TL(6);
        }
        // blocks go to work-groups in the order they get here (one ticket
        // each), so the work-groups that finish their own work last do not
        // also combine: with H/32 <= G they take no block
        if (tid == 0) misc[9] = rmw_inc(a.sync + SM.ticket + d.ptag() - 1u);
        lds_barrier();
        const uint32_t t0 = uni(misc[9]);
        WL_TL(11);
        for (uint32_t blkr = t0; blkr < P.NB; blkr += G) {
            const uint32_t r = blkr * RB + tid;
            const float o = xl2 ? xcd_total(a.part, blkr) : block_total(a.part, blkr);
            if (tid < RB) {
                // + the residual: the layer's input (plain, or the tagged words it
                // was read from, which only this block's combine overwrites)
                float v = o;
                if (d.resid) v = __fadd_rn(gld(d.resid + r), o);
                else if (ch.hx_in)
                    v = __fadd_rn(__uint_as_float((uint32_t)__hip_atomic_load(
                                      (__attribute__((address_space(1))) const uint64_t*)(ch.hx_in + r),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
                                  o);
                if (d.out) gst(d.out + r, v);
                if (ch.hx_out) st_tag(ch.hx_out + r, d.epoch, v);
            }
            if (d.taps()) {
                const float sh = xl2 ? xcd_total(a.tsh, blkr) : block_total(a.tsh, blkr);
                if (tid < RB) gst(a.shared_out + r, sh);
            }
        }
        WL_TL(10);
    }
    return true;
}

// One layer per launch: the pointers its first loads need are preloaded
// kernel arguments (the record pointer, the five pointers up to lslot, seg
// and epoch).
static_assert(6 * sizeof(void*) / 4 + 2 == kPreloadDwords, "preloaded kernel arguments");
template <bool GLM, bool SH4>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
moe_decode_kernel(const DecodeArgs* __restrict__ pa, const float* hidden, const uint8_t* sh_native,
                  const uint16_t* router_w, const uint16_t* ln_w, uint64_t* lslot, uint32_t seg, uint32_t epoch,
                  const float* bias, const uint8_t* const* slot_tab, const float* resid, float* out) {
    const DecodeDyn d{hidden, sh_native, router_w, ln_w, lslot, seg, epoch, bias, slot_tab, resid, out};
    (void)decode_layer<GLM, SH4, false>(*pa, d, ChainIO{nullptr, 0u, nullptr});
}

// n consecutive resident layers in one launch, h <- h + moe(h) each: layer i
// uses record recs[i], epoch epoch0 + i and partial tag (tag0 - 1 + i) mod 3
// + 1. A work-group starts layer i + 1 as soon as it has finished its part
// of layer i (its own work and the combine blocks it took), so the next
// layer's weight loads overlap this layer's combine: the first layer reads h
// from d_h, every layer hands its output to the next through hx as tagged
// words (the reader polls), and the last writes d_h. Safe to reuse the
// per-layer arrays: a work-group stores layer i + 1's partials only after
// that layer's top-k, which needs every work-group's layer i + 1 logit, so
// every work-group has left layer i by then.
template <bool GLM, bool SH4>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
moe_chain_kernel(const DecodeArgs* __restrict__ recs, float* d_h, uint64_t* lslot, uint64_t* hx, uint32_t n,
                 uint32_t epoch0, uint32_t seg0) {
    const uint32_t tag0 = (seg0 >> 24) & 3u;
    for (uint32_t i = 0; i < n; i++) {
        const DecodeArgs& a = recs[i];
        const uint32_t seg = (seg0 & 0x00FFFFFFu) | ((((tag0 - 1u + i) % 3u) + 1u) << 24);
        const bool first = i == 0u, last = i + 1u == n;
        const DecodeDyn d{first ? d_h : nullptr, a.sh_native, a.router_w, a.ln_w, lslot, seg, epoch0 + i,
                          a.bias, a.slot_tab, first ? d_h : nullptr, last ? d_h : nullptr};
        if (!decode_layer<GLM, SH4, true>(a, d, ChainIO{first ? nullptr : hx, epoch0 + i - 1u, last ? nullptr : hx}))
            return;
        lds_barrier();  // the next layer's LDS writes follow every wave's last reads
    }
}

// ---- routing only (cache-backed layers) ------------------------------------
// RMSNorm, the router rows of this work-group (r = w + G*i, epoch-tagged
// logits, the same arithmetic as the decode kernel), then work-group 0 gathers
// every logit and writes the top-k ids and weights (idx, topw) and the logits.
// The host reads the ids, resolves the experts through its LRU slot pool, and
// only then runs the layer (reference run_moe's router + D2H staging,
// src/glm_layer_runner.cuh:386-396). LDS: xn [H] | red [8 x 64] | topk.
__global__ void __launch_bounds__(kThreads) route_kernel(const DecodeArgs* __restrict__ pa, const float* hidden,
                                                         uint32_t epoch) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, E = a.E, K = a.K;
    const uint32_t G = gridDim.x, w = blockIdx.x, tid = threadIdx.x;
    extern __shared__ __align__(16) uint8_t lds[];
    float* xn = (float*)lds;
    float* red = xn + ((H + 3u) & ~3u);
    float* tk_sc = red + kWaves * 64;
    float* tk_ch = tk_sc + E;
    uint32_t* tk_idx = (uint32_t*)(tk_ch + E);
    float* tk_w = (float*)(tk_idx + 32);
    uint32_t* flags = (uint32_t*)(tk_w + 32);
    const SyncMap SM = SyncMap::make();

    float4 hv[kHV];
    uint2 lv[kHV];
    const rsrc_t hid_rs = make_rsrc(hidden, H * 4u);
    const rsrc_t ln_rs = make_rsrc(a.ln_w ? (const void*)a.ln_w : (const void*)hidden, H * 2u);
#pragma unroll
    for (int i = 0; i < kHV; i++) {
        const uint32_t j = tid + kThreads * i;
        hv[i] = __builtin_bit_cast(float4, bld16(hid_rs, 16u * j, 0u));
        lv[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ln_rs, (int)(8u * j), 0, 0));
    }
    const uint32_t nch = H / 8;
    const rsrc_t rt_rs = make_rsrc(a.router_w, E * H * 2u);
    const float rinv = norm_rinv(hv, red, H, a.eps);
#pragma unroll
    for (int i = 0; i < kHV; i++) {
        const uint32_t j = tid + kThreads * i;
        if (j < H / 4) {
            const float xs[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
            const uint32_t ls[4] = {lv[i].x & 0xFFFFu, lv[i].x >> 16, lv[i].y & 0xFFFFu, lv[i].y >> 16};
#pragma unroll
            for (int c = 0; c < 4; c++) xn[4 * j + c] = norm_value(xs[c], rinv, a.ln_w != nullptr, ls[c]);
        }
    }
    lds_barrier();
    for (uint32_t r = w; r < E; r += G) {
        u32x4 rw[kRCH];
#pragma unroll
        for (int m = 0; m < kRCH; m++) rw[m] = bld16_nt(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), r * H * 2u);
        router_publish(router_partial(rw, xn, nch), red, a.lslot, r, epoch);
    }
    if (w != 0) return;

    // work-group 0: every logit of this call (bounded poll), then the top-k
    for (uint32_t e = tid; e < E; e += kThreads) tk_ch[e] = gld(a.bias + e);
    lds_barrier();
    uint32_t done = 0;  // bit i: expert tid + 512 i scored
    for (uint32_t spins = 0;; spins++) {
        bool mine = true;
        for (uint32_t i = 0, e = tid; e < E; i++, e += kThreads) {
            if ((done >> i) & 1u) continue;
            const uint64_t x = __hip_atomic_load((__attribute__((address_space(1))) uint64_t*)(a.lslot + e),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((uint32_t)(x >> 32) == epoch) {
                topk_score(__uint_as_float((uint32_t)x), tk_ch[e], e, tk_sc, tk_ch);
                gst(a.logits + e, __uint_as_float((uint32_t)x));
                done |= 1u << i;
            } else {
                mine = false;
            }
        }
        if (block_all(mine, flags)) break;
        if (spins > (1u << 20)) {
            if (tid == 0) raise_error(a.sync, SM, E_SPIN, epoch);
            return;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (E <= 256u) topk_argmax(E, K, tk_sc, tk_ch, tk_idx, tk_w);
    else topk_rank(E, K, tk_sc, tk_ch, tk_idx, tk_w);
    if (tid < K) {
        gst(a.idx + tid, (int32_t)tk_idx[tid]);
        gst(a.topw + tid, topk_weight(a, K, tk_w, tid));
    }
}

// Slot table of one layer: table[e] = the block of expert e if e is one of the
// n resolved ids, else null (an id the host did not resolve then raises
// E_NOT_RESIDENT instead of reading a stale slot).
struct SlotFill {
    int32_t ids[32];
    const uint8_t* ptrs[32];
    uint32_t n;
};
__global__ void __launch_bounds__(256) slot_fill_kernel(const uint8_t** table, uint32_t E, const SlotFill f) {
    for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < E; e += gridDim.x * blockDim.x) {
        const uint8_t* p = nullptr;
        for (uint32_t k = 0; k < f.n; k++)
            if ((uint32_t)f.ids[k] == e) p = f.ptrs[k];
        table[e] = p;
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

// ---- one expert FFN in one launch (config 0, wl_expert_ffn) --------------------
// A persistent launch of G work-groups (one per CU) over one reference-layout
// block: work-group w takes inter rows [RPW w, RPW w + RPW) of gate and up
// (wave v: rows RPW w + v + 8 j) and output rows [DPW w, DPW w + DPW) of down
// (wave v: rows DPW w + v + 8 j), and issues every weight load of both phases
// before it computes anything, so the whole block streams at once. Gate/up:
// lane l holds blocks l + 64 b of its row (16 bytes of nibbles, one E8M0
// byte), widened to f32 exactly (v_cvt_scalef32_pk_f32_fp4) and dotted with
// x in f32; a wave sum gives the row; SwiGLU; the value is published as an
// epoch-tagged word (epoch << 32 | f32 bits, agent scope). Down: every
// work-group reads the I tagged values (re-reading stale ones, bounded), then
// lane l dots block l of each of its rows with them. No partial sums: each
// output row is one work-group's. Reference: the per-expert sequence of
// run_moe, 3 x dequant_matvec_mxfp4 + silu_mul (src/glm_layer_runner.cuh:
// 424-427; src/glm_kernels.cuh:63-110).
typedef __attribute__((ext_vector_type(2))) float f32x2;
// acc + the 8 values of one dword (two per byte, low nibble first) times x[0..8)
WL_DEV float fp4x8_dot(uint32_t d, float sc, const float* x, float acc) {
    const f32x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, sc, 0);
    const f32x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, sc, 1);
    const f32x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, sc, 2);
    const f32x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, sc, 3);
    const float4 xa = *(const float4*)x, xb = *(const float4*)(x + 4);
    acc = fmaf(v0.x, xa.x, acc);
    acc = fmaf(v0.y, xa.y, acc);
    acc = fmaf(v1.x, xa.z, acc);
    acc = fmaf(v1.y, xa.w, acc);
    acc = fmaf(v2.x, xb.x, acc);
    acc = fmaf(v2.y, xb.y, acc);
    acc = fmaf(v3.x, xb.z, acc);
    return fmaf(v3.y, xb.w, acc);
}
// One 32-value block: 16 bytes of nibbles at scale sc against x[0..32).
WL_DEV float fp4_dot32(u32x4 w, float sc, const float* x) {
    float acc = fp4x8_dot(w.x, sc, x, 0.f);
    acc = fp4x8_dot(w.y, sc, x + 8, acc);
    acc = fp4x8_dot(w.z, sc, x + 16, acc);
    return fp4x8_dot(w.w, sc, x + 24, acc);
}
WL_DEV float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int NBL, int GJ, int NBD, int DJ>
__global__ void __launch_bounds__(kThreads) ffn1_kernel(FfnArgs a) {
    const uint32_t H = a.H, I = a.I, w = blockIdx.x, tid = threadIdx.x;
    const uint32_t v = uni(tid >> 6), lane = tid & 63;
    constexpr uint32_t RPW = 8u * GJ, DPW = 8u * DJ;
    extern __shared__ __align__(16) uint8_t lds[];
    float* xs = (float*)lds;    // [H]
    float* ms = xs + H;         // [I] the SwiGLU values
    uint32_t* flag = (uint32_t*)(ms + I);
    const SyncMap SM = SyncMap::make();
#ifdef WL_TIMELINE
    const uint32_t tl_slot = 0;
#endif
    WL_TL(12);
    // x first (it returns first: a wave's loads complete in order), then
    // every weight load of the work-group
    constexpr int XV = (int)(NBL * 64 * 32 / 4 / kThreads);  // float4 of x per thread (H = NBL * 2048)
    float4 xv[XV];
    const rsrc_t x_rs = make_rsrc(a.x, H * 4u);
#pragma unroll
    for (int i = 0; i < XV; i++) xv[i] = __builtin_bit_cast(float4, bld16(x_rs, 16u * (tid + kThreads * i), 0u));
    const rsrc_t gw_rs = make_rsrc(a.blk + a.gw_off, I * H / 2u), gs_rs = make_rsrc(a.blk + a.gs_off, I * H / 32u);
    const rsrc_t uw_rs = make_rsrc(a.blk + a.uw_off, I * H / 2u), us_rs = make_rsrc(a.blk + a.us_off, I * H / 32u);
    const rsrc_t dw_rs = make_rsrc(a.blk + a.dw_off, H * I / 2u), ds_rs = make_rsrc(a.blk + a.ds_off, H * I / 32u);
    u32x4 gw[GJ][NBL], uw[GJ][NBL], dw[DJ][NBD];
    uint32_t gs[GJ][NBL], us[GJ][NBL], dsc[DJ][NBD];
#pragma unroll
    for (int j = 0; j < GJ; j++) {
        const uint32_t r = RPW * w + v + 8u * j;
#pragma unroll
        for (int b = 0; b < NBL; b++) {
            const uint32_t blk = lane + 64u * b;
            gw[j][b] = bld16_nt(gw_rs, r * (H / 2u) + 16u * blk, 0u);
            uw[j][b] = bld16_nt(uw_rs, r * (H / 2u) + 16u * blk, 0u);
            gs[j][b] = bld1(gs_rs, r * (H / 32u) + blk, 0u);
            us[j][b] = bld1(us_rs, r * (H / 32u) + blk, 0u);
        }
    }
#pragma unroll
    for (int j = 0; j < DJ; j++) {
        const uint32_t r = DPW * w + v + 8u * j;
#pragma unroll
        for (int b = 0; b < NBD; b++) {
            const uint32_t blk = lane + 64u * b;
            dw[j][b] = bld16_nt(dw_rs, r * (I / 2u) + 16u * blk, 0u);
            dsc[j][b] = bld1(ds_rs, r * (I / 32u) + blk, 0u);
        }
    }
#pragma unroll
    for (int i = 0; i < XV; i++) *(float4*)(xs + 4u * (tid + kThreads * i)) = xv[i];
    lds_barrier();
    WL_TL(13);
    // gate / up rows, SwiGLU, published
#pragma unroll
    for (int j = 0; j < GJ; j++) {
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int b = 0; b < NBL; b++) {
            const float* xb = xs + 32u * (lane + 64u * b);
            g += fp4_dot32(gw[j][b], e8m0f(gs[j][b]), xb);
            u += fp4_dot32(uw[j][b], e8m0f(us[j][b]), xb);
        }
        g = wave_sum(g);
        u = wave_sum(u);
        if (lane == 0) {
            const uint32_t r = RPW * w + v + 8u * j;
            __hip_atomic_store((__attribute__((address_space(1))) uint64_t*)(a.tag + r),
                               ((uint64_t)a.epoch << 32) | __float_as_uint(silu_mul(g, u)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    WL_TL(14);
    // every SwiGLU value of this call, into LDS: each thread's 16-byte chunks
    // (two tagged words each) all in flight together, then the stale ones
    // again until this call's epoch shows (bounded)
    constexpr int MC = (int)(NBD * 64 * 32 / 2 / kThreads);  // chunks per thread (I = NBD * 2048)
    // (one round in flight at a time: measured, several rounds in flight
    // from every work-group hot-spot the channels holding the 16 KB array and
    // were slower, 16.9 against 13.3 us per expert)
    const rsrc_t tg_rs = make_rsrc(a.tag, I * 8u);
    u32x4 mc[MC];
#pragma unroll
    for (int i = 0; i < MC; i++) mc[i] = bld16_ag(tg_rs, 16u * (tid + kThreads * i), 0u);
    uint32_t stale = 0;
    for (uint32_t spins = 0;; spins++) {
#pragma unroll
        for (int i = 0; i < MC; i++) {
            if (spins != 0 && !((stale >> i) & 1u)) continue;
            if (mc[i].y == a.epoch && mc[i].w == a.epoch) {
                const uint32_t c = tid + kThreads * i;
                ms[2u * c] = __uint_as_float(mc[i].x);
                ms[2u * c + 1u] = __uint_as_float(mc[i].z);
                stale &= ~(1u << i);
            } else {
                stale |= 1u << i;
            }
        }
        if (block_all(stale == 0u, flag)) break;
        if (spins > (1u << 20) || aborted(a.sync, SM, a.epoch)) {
            if (tid == 0 && spins > (1u << 20)) raise_error(a.sync, SM, E_SPIN, a.epoch);
            return;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int i = 0; i < MC; i++)
            if ((stale >> i) & 1u) mc[i] = bld16_ag(tg_rs, 16u * (tid + kThreads * i), 0u);
    }
    WL_TL(15);
    // down rows
#pragma unroll
    for (int j = 0; j < DJ; j++) {
        float y = 0.f;
#pragma unroll
        for (int b = 0; b < NBD; b++) y += fp4_dot32(dw[j][b], e8m0f(dsc[j][b]), ms + 32u * (lane + 64u * b));
        y = wave_sum(y);
        if (lane == 0) {
            const uint32_t r = DPW * w + v + 8u * j;
            a.y[r] = y;
            if (a.y_bf16) a.y_bf16[r] = (uint16_t)f2bf(y);
        }
    }
}

// The one-launch expert FFN for the shapes it is instantiated for (GLM: H
// 6144, I 2048 on 256 work-groups); -1 for any other (the caller then runs
// launch_expert_ffn).
int launch_expert_ffn1(const FfnArgs& a, uint32_t grid, void* stream) {
    // more than half of a CU's 160 KB: one work-group per CU (the launch has
    // one per CU, and they wait for each other: two on one CU would share its
    // bandwidth while another CU idles)
    const size_t lds = std::max<size_t>(4u * ((size_t)a.H + a.I) + 64u, 84u * 1024u);
    if (!(a.H == 6144 && a.I == 2048 && grid == 256)) return -1;
    // every work-group must be resident at once (they wait for each other's
    // SwiGLU values): checked once per process (one launch shape)
    static const int per_cu = [&] {
        int n = 0;
        const void* fn = (const void*)ffn1_kernel<3, 1, 1, 3>;
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return 0;
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kThreads, lds) == hipSuccess ? n : 0;
    }();
    if (per_cu < 1) return -1;
    hipLaunchKernelGGL((ffn1_kernel<3, 1, 1, 3>), dim3(grid), dim3(kThreads), lds, (hipStream_t)stream, a);
    return (int)hipGetLastError();
}

static bool glm_shape(uint32_t H, uint32_t I, uint32_t SI, uint32_t E, uint32_t K) {
    return H == 6144 && I == 2048 && SI == 2048 && E == 256 && K == 8;
}

// The decode kernel instantiation for a shape and shared-expert format.
static const void* decode_fn(bool glm, bool sh4) {
    return glm ? (sh4 ? (const void*)moe_decode_kernel<true, true> : (const void*)moe_decode_kernel<true, false>)
               : (sh4 ? (const void*)moe_decode_kernel<false, true> : (const void*)moe_decode_kernel<false, false>);
}

int decode_max_lds() { return 160 * 1024; }

int decode_occupancy(uint32_t H, uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid, int* per_cu) {
    const Plan p = Plan::make(H, I, SI, K, grid);
    const size_t lds = LdsMap::make(H, SI, E, K, p).bytes;
    int lo = 1 << 30;
    for (bool sh4 : {false, true}) {  // the fewest of either shared-expert format
        const void* fn = decode_fn(glm_shape(H, I, SI, E, K), sh4);
        int n = 0;
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kThreads, lds);
        if (e != hipSuccess) return (int)e;
        lo = n < lo ? n : lo;
    }
    *per_cu = lo;
    return 0;
}

int route_occupancy(uint32_t H, uint32_t E, int* per_cu) {
    const size_t lds = route_lds_bytes(H, E);
    hipError_t e = hipFuncSetAttribute((const void*)route_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, (const void*)route_kernel, kThreads, lds);
    return (int)e;
}

size_t route_lds_bytes(uint32_t H, uint32_t E) {
    return 4u * (((H + 3u) & ~3u) + kWaves * 64u + 2u * E + 64u + 8u);
}

int launch_route(const DecodeArgs* d_args, const float* hidden, uint32_t epoch, uint32_t H, uint32_t E,
                 uint32_t grid, void* stream) {
    const size_t lds = route_lds_bytes(H, E);
    hipError_t e = hipFuncSetAttribute((const void*)route_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(route_kernel, dim3(grid), dim3(kThreads), lds, (hipStream_t)stream, d_args, hidden, epoch);
    return (int)hipGetLastError();
}

int launch_slot_fill(const uint8_t** table, uint32_t E, const int32_t* ids, const uint8_t* const* ptrs, uint32_t n,
                     void* stream) {
    if (n > 32) return (int)hipErrorInvalidValue;
    SlotFill f{};
    for (uint32_t k = 0; k < n; k++) {
        f.ids[k] = ids[k];
        f.ptrs[k] = ptrs[k];
    }
    f.n = n;
    hipLaunchKernelGGL(slot_fill_kernel, dim3((E + 255) / 256), dim3(256), 0, (hipStream_t)stream, table, E, f);
    return (int)hipGetLastError();
}

int launch_decode(const DecodeArgs* d_args, const DecodeDyn& dyn, uint32_t H, uint32_t I, uint32_t SI, uint32_t E,
                  uint32_t K, uint32_t grid, bool sh4, void* stream) {
    const Plan p = Plan::make(H, I, SI, K, grid);
    const size_t lds = LdsMap::make(H, SI, E, K, p).bytes;
    const bool glm = glm_shape(H, I, SI, E, K);
    hipError_t e = hipFuncSetAttribute(decode_fn(glm, sh4), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
#define WL_DECODE_ARGS                                                                                        \
    d_args, dyn.hidden, dyn.sh_native, dyn.router_w, dyn.ln_w, dyn.lslot, dyn.seg, dyn.epoch, dyn.bias, dyn.slot_tab, \
        dyn.resid, dyn.out
    const dim3 gr(grid), bl(kThreads);
    hipStream_t st = (hipStream_t)stream;
    if (glm && sh4) hipLaunchKernelGGL((moe_decode_kernel<true, true>), gr, bl, lds, st, WL_DECODE_ARGS);
    else if (glm) hipLaunchKernelGGL((moe_decode_kernel<true, false>), gr, bl, lds, st, WL_DECODE_ARGS);
    else if (sh4) hipLaunchKernelGGL((moe_decode_kernel<false, true>), gr, bl, lds, st, WL_DECODE_ARGS);
    else hipLaunchKernelGGL((moe_decode_kernel<false, false>), gr, bl, lds, st, WL_DECODE_ARGS);
#undef WL_DECODE_ARGS
    return (int)hipGetLastError();
}

__global__ void xcd_map_kernel(uint32_t* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

int probe_xcd_map(uint32_t grid, bool* ok) {
    *ok = false;
    uint32_t* d = nullptr;
    hipError_t e = hipMalloc(&d, 4 * (size_t)grid);
    if (e != hipSuccess) return (int)e;
    std::vector<uint32_t> h(grid, ~0u);
    hipLaunchKernelGGL(xcd_map_kernel, dim3(grid), dim3(64), 0, 0, d);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpy(h.data(), d, 4 * (size_t)grid, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return (int)e;
    bool all = true;
    for (uint32_t w = 0; w < grid; w++) all = all && h[w] == (w & 7u);
    *ok = all;
    return 0;
}

static const void* chain_fn(bool glm, bool sh4) {
    return glm ? (sh4 ? (const void*)moe_chain_kernel<true, true> : (const void*)moe_chain_kernel<true, false>)
               : (sh4 ? (const void*)moe_chain_kernel<false, true> : (const void*)moe_chain_kernel<false, false>);
}

int launch_chain(const DecodeArgs* recs, float* d_h, uint64_t* lslot, uint64_t* hx, uint32_t n, uint32_t epoch0,
                 uint32_t seg0, uint32_t H, uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid, bool sh4,
                 void* stream) {
    const Plan p = Plan::make(H, I, SI, K, grid);
    const size_t lds = LdsMap::make(H, SI, E, K, p).bytes;
    const bool glm = glm_shape(H, I, SI, E, K);
    const void* fn = chain_fn(glm, sh4);
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    const dim3 gr(grid), bl(kThreads);
    hipStream_t st = (hipStream_t)stream;
    if (glm && sh4) hipLaunchKernelGGL((moe_chain_kernel<true, true>), gr, bl, lds, st, recs, d_h, lslot, hx, n, epoch0, seg0);
    else if (glm) hipLaunchKernelGGL((moe_chain_kernel<true, false>), gr, bl, lds, st, recs, d_h, lslot, hx, n, epoch0, seg0);
    else if (sh4) hipLaunchKernelGGL((moe_chain_kernel<false, true>), gr, bl, lds, st, recs, d_h, lslot, hx, n, epoch0, seg0);
    else hipLaunchKernelGGL((moe_chain_kernel<false, false>), gr, bl, lds, st, recs, d_h, lslot, hx, n, epoch0, seg0);
    return (int)hipGetLastError();
}

#ifdef WL_TIMELINE
extern "C" int wl_dbg_timeline(void* host, size_t bytes) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_tl), bytes, 0, hipMemcpyDeviceToHost);
}
#endif

}  // namespace wl
