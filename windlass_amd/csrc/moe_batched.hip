// moe_batched.hip — the MoE layer for T tokens at once on gfx950 (the
// reference's run_moe_batched, src/glm_layer_runner.cuh:818-928, used by
// prefill): every expert's weights are streamed once per pass of up to kMT of
// its tokens instead of once per token.
//
//   bnorm    RMSNorm per token
//   broute   router logits, kTB tokens per work-group; norm and logits use the
//            arithmetic of the decode and routing kernels, so a token's ids
//            equal the ones wl_run_moe selects for it
//   btopk    sigmoid + bias, top-k, weights (one work-group per token)
//   bcount   per expert: its entries (token*K + slot) in ascending order
//            (wave ballots, deterministic) and their count
//   bscatter per expert: its compact range (prefix of the counts), ent/pos
//   bgu      routed gate/up + SwiGLU: unit = (token pass, expert, 4 slices of 64 rows)
//   bdn      routed down: unit = (token pass, expert, 256 output rows)
//   bsgu     shared gate/up + SwiGLU: unit = (token pass, 64-row slice)
//   bsdn     shared down: unit = (token pass, 128 output rows)
//   bcomb    out[t] = (resid[t] +) sum_k w[t][k] e_k[t] (slot order) + shared[t]
//
// The GEMMs put tokens on the MFMA's 16 rows (v_mfma_f32_16x16x32_bf16) and
// each activation as three bf16 pieces (x = p0 + p1 + p2 to f32 precision)
// accumulated by three MFMAs; MXFP4 weights are converted exactly to bf16
// (v_cvt_scalef32_pk_bf16_fp4), bf16 weights are used as they are. The
// activations of a pass are staged in LDS kKC columns at a time.
#include <hip/hip_runtime.h>

#include "dev_common.h"
#include "internal.h"

namespace wl {

constexpr uint32_t kMT = 32;         // tokens per pass: two MFMA row blocks of 16
constexpr uint32_t kKC = 256;        // activation columns staged per step
constexpr uint32_t kAS = kKC + 8;    // LDS row stride (bf16) of a staged piece
constexpr uint32_t kALds = 3u * kMT * kAS * 2u;
constexpr uint32_t kTB = 8;          // tokens per routing work-group
constexpr uint32_t kRouteGX = 16;    // routing work-groups per token block (router rows r = x + 16 i)

// A operand of token block tb, piece pc: lane (m, g) holds the 8 columns
// [col, col + 8) of token tb*16 + m (col already includes the lane group's
// offset).
WL_DEV bf16x8 afrag(const uint16_t* A, uint32_t pc, uint32_t tb, uint32_t col) {
    const uint32_t m = threadIdx.x & 15u;
    return as_bf16x8(*(const u32x4*)(A + (pc * kMT + tb * 16u + m) * kAS + col));
}
// acc[tb] += x[tokens of block tb] . b for every live block (3 pieces).
WL_DEV void mma_blocks(f32x4 (&acc)[2], const uint16_t* A, uint32_t nblk, uint32_t col, bf16x8 b) {
#pragma unroll
    for (uint32_t tb = 0; tb < 2; tb++) {
        if (tb < nblk) {
#pragma unroll
            for (uint32_t pc = 0; pc < 3; pc++) acc[tb] = mma(afrag(A, pc, tb, col), b, acc[tb]);
        }
    }
}
// SwiGLU epilogue of a gate/up tile: lane (n, g), element i of acc[tb] is
// token tb*16 + 4g + i; columns n < 8 are gate rows, n + 8 the matching up
// rows. Calls put(m, n, value) for n < 8 and live tokens.
template <class PutF>
WL_DEV void swiglu_store(const f32x4 (&acc)[2], uint32_t nt, PutF put) {
    const uint32_t lane = threadIdx.x & 63u, n = lane & 15u, g = lane >> 4;
#pragma unroll
    for (uint32_t tb = 0; tb < 2; tb++) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const float v = acc[tb][i];
            const float up = __shfl(v, (lane + 8u) & 63u, 64);
            const uint32_t m = tb * 16u + 4u * g + i;
            if (n < 8u && m < nt) put(m, n, silu_mul(v, up));
        }
    }
}

// ---- routing ------------------------------------------------------------------
// RMSNorm of token t = blockIdx.x (norm_rinv / norm_value: the decode kernel's
// arithmetic) into b.norm.
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
        }
    }
}

// Router logits of kTB tokens: each thread keeps its router_partial share of
// every token's normalised input in registers; the rows r = x + gridDim.x i
// stream through (next row prefetched). The per-row arithmetic and the
// summation over waves are router_partial's and router_publish's.
__global__ void __launch_bounds__(kThreads) broute_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, E = a.E, tid = threadIdx.x;
    __shared__ float red[kWaves * 64];
    const uint32_t t0 = blockIdx.y * kTB, nch = H / 8;
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
    u32x4 rn[kRCH];
#pragma unroll
    for (int m = 0; m < kRCH; m++)
        rn[m] = bld16(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), min(blockIdx.x, E - 1u) * H * 2u);
    for (uint32_t r = blockIdx.x; r < E; r += gridDim.x) {
        u32x4 rw[kRCH];
#pragma unroll
        for (int m = 0; m < kRCH; m++) {
            rw[m] = rn[m];
            rn[m] = bld16(rt_rs, 16u * min(tid + kThreads * m, nch - 1u), min(r + gridDim.x, E - 1u) * H * 2u);
        }
#pragma unroll
        for (uint32_t tt = 0; tt < kTB; tt++) {
            const float pd = router_partial_x(rw, [&](int m, int h) { return xr[tt][m][h]; }, nch);
            if ((tid & 63u) == 0) red[(tid >> 6) * 64 + 48 + tt] = pd;
        }
        lds_barrier();
        if (tid < kTB && t0 + tid < b.T) {
            float sum = 0.f;  // the same order as router_publish
#pragma unroll
            for (int wv = 0; wv < kWaves; wv++) sum += red[wv * 64 + 48 + tid];
            gst(b.logits + (size_t)(t0 + tid) * E + r, sum);
        }
        lds_barrier();
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
// per step, positions from a ballot prefix.
__global__ void __launch_bounds__(64) bcount_kernel(const BatchArgs b, uint32_t K) {
    const uint32_t e = blockIdx.x, lane = threadIdx.x, n = b.T * K;
    uint32_t base = 0;
    for (uint32_t i0 = 0; i0 < n; i0 += 64) {
        const uint32_t i = i0 + lane;
        const bool hit = i < n && (uint32_t)gld(b.idx + i) == e;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(hit);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (hit) gst(b.lists + (size_t)e * b.T + base + below, i);
        base += (uint32_t)__builtin_popcountll(bal);
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

// ---- grouped GEMMs ------------------------------------------------------------
// Loads complete in issue order, so a wave cannot wait for its activation
// loads of one step without also waiting for every weight load issued before
// them. Each step therefore issues, in order: the activations of this step,
// then the weights of the NEXT step, then consumes the activations (split
// into LDS) and computes with the weights loaded one step earlier. A step
// carries many weight tiles per activation stage (kSG slices per unit), so
// the weights in flight during the wait are large.
constexpr uint32_t kSG = 4;  // gate/up slices (64 rows each) per unit

// Activation loads of one step (issued before the next step's weights).
struct AStage {
    float4 x[kMT * kKC / 4u / kThreads];
};
template <class RowF>
WL_DEV void a_load(AStage& S, RowF row, uint32_t nt, uint32_t k0, uint32_t kmax) {
    constexpr uint32_t kPer = kMT * kKC / 4u / kThreads;
#pragma unroll
    for (uint32_t i = 0; i < kPer; i++) {
        const uint32_t it = threadIdx.x + kThreads * i;
        const uint32_t m = it / (kKC / 4u), c = (it % (kKC / 4u)) * 4u;
        S.x[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m < nt && k0 + c < kmax) S.x[i] = __builtin_bit_cast(float4, gld16(row(m) + k0 + c));
    }
}
WL_DEV void a_store(uint16_t* A, const AStage& S) {
    constexpr uint32_t kPer = kMT * kKC / 4u / kThreads;
#pragma unroll
    for (uint32_t i = 0; i < kPer; i++) {
        const uint32_t it = threadIdx.x + kThreads * i;
        const uint32_t m = it / (kKC / 4u), c = (it % (kKC / 4u)) * 4u;
        const float xs[4] = {S.x[i].x, S.x[i].y, S.x[i].z, S.x[i].w};
        uint32_t h[4], md[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; q++) split3(xs[q], h[q], md[q], l[q]);
        *(uint2*)(A + (0u * kMT + m) * kAS + c) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
        *(uint2*)(A + (1u * kMT + m) * kAS + c) = make_uint2(md[0] | (md[1] << 16), md[2] | (md[3] << 16));
        *(uint2*)(A + (2u * kMT + m) * kAS + c) = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
    }
}
// Two-deep step pipeline over nst steps with weight buffers W0/W1: W0 holds
// step 0 on entry. step(s, cur, nxt) must issue the activations of step s,
// then issue(s + 1, nxt), then consume.
template <class W, class StepF>
WL_DEV void steps2(uint32_t nst, W& W0, W& W1, StepF step) {
    uint32_t s = 0;
#pragma unroll 1
    for (; s + 2 <= nst; s += 2) {
        step(s, W0, W1);
        step(s + 1, W1, W0);
    }
    if (s < nst) step(s, W0, W1);
}
// An offset no buffer reaches: loads of steps past the end return zeros
// without a memory access.
constexpr uint32_t kOOB = 0x7FFFFFF0u;

// Routed gate/up + SwiGLU. Unit u = (pass p, expert e, slice group sg):
// tokens [p*kMT, +kMT) of expert e, rows of kSG slices [64(kSG sg + i), +64)
// of gate and up (wave v: tiles 8(kSG sg + i) + v, native gu chunks), K = H in
// steps of kKC columns (2 k tiles).
struct GuW {
    u32x4 w[kSG][2];
    u32x4 sv[kSG];
};
__global__ void __launch_bounds__(kThreads) bgu_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, I = a.I, E = a.E, K = a.K;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, g = lane >> 4;
    const uint32_t v = uni(tid >> 6) & 7u;
    extern __shared__ __align__(16) uint8_t lds[];
    uint16_t* A = (uint16_t*)lds;
    uint32_t* tok = (uint32_t*)(lds + kALds);
    uint32_t* s_cnt = tok + kMT;  // [E] counts, then [E] offsets
    const NativeLayout NL = NativeLayout::make(H, I);
    const uint32_t S = I / kSlice, NSG = cdiv(S, kSG), nkg = H / 128, P = cdiv(b.T, kMT);
    const uint32_t nst = cdiv(H, kKC);
    const SyncMap SM = SyncMap::make();
    for (uint32_t f = tid; f < E; f += kThreads) {
        s_cnt[f] = gld(b.counts + f);
        s_cnt[E + f] = gld(b.offsets + f);
    }
    lds_barrier();
    for (uint32_t u = blockIdx.x; u < P * E * NSG; u += gridDim.x) {
        const uint32_t p = u / (E * NSG), e = (u / NSG) % E, sg = u % NSG;
        const uint32_t ne = uni(s_cnt[e]);
        if (p * kMT >= ne) continue;
        const uint32_t nt = min(kMT, ne - p * kMT), c0 = uni(s_cnt[E + e]) + p * kMT;
        const uint8_t* blk = uni_ptr(gld(a.slot_tab + e));
        if (blk == nullptr) {
            if (tid == 0) raise_error(a.sync, SM, E_NOT_RESIDENT);
            continue;
        }
        lds_barrier();  // the previous unit's readers of tok are done
        if (tid < nt) tok[tid] = gld(b.ent + c0 + tid) / K;
        lds_barrier();
        const rsrc_t rs = make_rsrc(blk, (uint32_t)NL.total);
        uint32_t gu_voff[kSG], gus_voff[kSG];
        bool sl_ok[kSG];
#pragma unroll
        for (uint32_t i = 0; i < kSG; i++) {
            const uint32_t sl = min(sg * kSG + i, S - 1u);
            sl_ok[i] = sg * kSG + i < S;
            const uint32_t tile = sl * (kSlice / 8u) + v;
            gu_voff[i] = (uint32_t)NL.gu + tile * nkg * 1024u + 16u * lane;
            gus_voff[i] = (uint32_t)NL.gus + tile * cdiv(nkg, 16u) * 1024u + 16u * lane;
        }
        const uint32_t nblk = cdiv(nt, 16u);
        f32x4 acc[kSG][2];
#pragma unroll
        for (uint32_t i = 0; i < kSG; i++) acc[i][0] = acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto row = [&](uint32_t m) { return b.norm + (size_t)tok[m] * H; };
        auto issue = [&](uint32_t s, GuW& W) {
            const bool live = s < nst;
            const uint32_t kt0 = min(s * 2u, nkg - 1u), kt1 = min(s * 2u + 1u, nkg - 1u);
#pragma unroll
            for (uint32_t i = 0; i < kSG; i++) {
                W.w[i][0] = bld16_nt(rs, gu_voff[i], live ? kt0 * 1024u : kOOB);
                W.w[i][1] = bld16_nt(rs, gu_voff[i], live ? kt1 * 1024u : kOOB);
                W.sv[i] = bld16_nt(rs, gus_voff[i], live ? (kt0 / 16u) * 1024u : kOOB);
            }
        };
        GuW W0, W1;
        issue(0, W0);
        steps2(nst, W0, W1, [&](uint32_t s, const GuW& cur, GuW& nxt) {
            AStage as;
            a_load(as, row, nt, s * kKC, H);
            issue(s + 1u, nxt);
            lds_barrier();  // the previous step's readers of A are done
            a_store(A, as);
            lds_barrier();
#pragma unroll
            for (uint32_t q = 0; q < 2; q++) {
                const uint32_t kt = s * 2u + q, o = kt % 16u;
                float sc[kSG];
#pragma unroll
                for (uint32_t i = 0; i < kSG; i++) {
                    const u32x4 sv = cur.sv[i];
                    const uint32_t sw = (o / 4u == 0u) ? sv.x : (o / 4u == 1u) ? sv.y : (o / 4u == 2u) ? sv.z : sv.w;
                    sc[i] = kt < nkg ? e8m0f((sw >> (8u * (o % 4u))) & 0xFFu) : 0.f;
                }
#pragma unroll
                for (uint32_t jj = 0; jj < 4; jj++) {
                    // the activation fragments of this k step, shared by the kSG slices
                    const uint32_t col = q * 128u + 32u * g + 8u * jj;
                    bf16x8 af[2][3];
#pragma unroll
                    for (uint32_t tb = 0; tb < 2; tb++)
#pragma unroll
                        for (uint32_t pc = 0; pc < 3; pc++) af[tb][pc] = afrag(A, pc, tb, col);
#pragma unroll
                    for (uint32_t i = 0; i < kSG; i++) {
                        const bf16x8 bw = fp4x8_bf16(cur.w[i][q][jj], sc[i]);
#pragma unroll
                        for (uint32_t tb = 0; tb < 2; tb++) {
                            if (tb < nblk) {
#pragma unroll
                                for (uint32_t pc = 0; pc < 3; pc++) acc[i][tb] = mma(af[tb][pc], bw, acc[i][tb]);
                            }
                        }
                    }
                }
            }
        });
#pragma unroll
        for (uint32_t i = 0; i < kSG; i++) {
            if (!sl_ok[i]) continue;
            const uint32_t sl = sg * kSG + i;
            swiglu_store(acc[i], nt, [&](uint32_t m, uint32_t n, float x) {
                gst(b.mid + (size_t)(c0 + m) * I + sl * kSlice + v * 8u + n, x);
            });
        }
    }
}

struct DnW {
    u32x4 w[4];
    u32x4 sv[4];
};
// Routed down. Unit u = (pass p, expert e, row block rb): tokens as in
// bgu_kernel, output rows [256rb, 256rb + 256) (wave v: row pair q = 8rb + v,
// rows 32q..32q+32, native dn chunks), K = I.
__global__ void __launch_bounds__(kThreads) bdn_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, I = a.I, E = a.E;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, n = lane & 15u, g = lane >> 4;
    const uint32_t v = uni(tid >> 6) & 7u;
    extern __shared__ __align__(16) uint8_t lds[];
    uint16_t* A = (uint16_t*)lds;
    uint32_t* s_cnt = (uint32_t*)(lds + kALds) + kMT;  // [E] counts, then [E] offsets
    const NativeLayout NL = NativeLayout::make(H, I);
    const uint32_t nq = H / 32u, RB = cdiv(nq, 8u), P = cdiv(b.T, kMT);
    for (uint32_t f = tid; f < E; f += kThreads) {
        s_cnt[f] = gld(b.counts + f);
        s_cnt[E + f] = gld(b.offsets + f);
    }
    lds_barrier();
    for (uint32_t u = blockIdx.x; u < P * E * RB; u += gridDim.x) {
        const uint32_t p = u / (E * RB), e = (u / RB) % E, rb = u % RB;
        const uint32_t ne = uni(s_cnt[e]);
        if (p * kMT >= ne) continue;
        const uint32_t nt = min(kMT, ne - p * kMT), c0 = uni(s_cnt[E + e]) + p * kMT;
        const uint8_t* blk = uni_ptr(gld(a.slot_tab + e));
        if (blk == nullptr) continue;  // reported by bgu_kernel
        const rsrc_t rs = make_rsrc(blk, (uint32_t)NL.total);
        const uint32_t q = rb * 8u + v;
        const bool qv = q < nq;
        const uint32_t qq = qv ? q : nq - 1u;
        const uint32_t nblk = cdiv(nt, 16u);
        f32x4 d0[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        f32x4 d1[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        auto row = [&](uint32_t m) { return b.mid + (size_t)(c0 + m) * I; };
        const uint32_t ca = 32u * (g & 1u) + 8u * (g >> 1);  // this lane group's slice columns (the swap order)
        const uint32_t nst = cdiv(I, kKC), NS = I / kSlice;
        auto issue = [&](uint32_t st, DnW& W) {
            const bool live = st < nst;
#pragma unroll
            for (uint32_t s4 = 0; s4 < 4; s4++) {
                const uint32_t j = min(st * 4u + s4, NS - 1u);
                W.w[s4] = bld16_nt(rs, (uint32_t)NL.dn + j * nq * 1024u + 16u * lane, live ? qq * 1024u : kOOB);
                W.sv[s4] = bld16_nt(rs, (uint32_t)NL.dns + j * cdiv(nq, 16u) * 1024u + 16u * lane,
                                    live ? (qq / 16u) * 1024u : kOOB);
            }
        };
        DnW W0, W1;
        issue(0, W0);
        steps2(nst, W0, W1, [&](uint32_t st, const DnW& cur, DnW& nxt) {
            AStage as;
            a_load(as, row, nt, st * kKC, I);
            issue(st + 1u, nxt);
            lds_barrier();
            a_store(A, as);
            lds_barrier();
#pragma unroll
            for (uint32_t s4 = 0; s4 < 4; s4++) {
                const bool valid = st * 4u + s4 < NS;
                const uint32_t o = qq % 16u;
                const u32x4 sv = cur.sv[s4];
                const uint32_t sw = (o / 4u == 0u) ? sv.x : (o / 4u == 1u) ? sv.y : (o / 4u == 2u) ? sv.z : sv.w;
                const uint32_t sbyte = (sw >> (8u * (o % 4u))) & 0xFFu;
                uint32_t sx, sy, x01, y01, x23, y23;
                swap32(sbyte, sbyte, sx, sy);
                swap32(cur.w[s4][0], cur.w[s4][1], x01, y01);
                swap32(cur.w[s4][2], cur.w[s4][3], x23, y23);
                const float scx = valid ? e8m0f(sx) : 0.f, scy = valid ? e8m0f(sy) : 0.f;
                const uint32_t col = s4 * kSlice + ca;
                const bf16x8 bx01 = fp4x8_bf16(x01, scx), bx23 = fp4x8_bf16(x23, scx);
                const bf16x8 by01 = fp4x8_bf16(y01, scy), by23 = fp4x8_bf16(y23, scy);
#pragma unroll
                for (uint32_t tb = 0; tb < 2; tb++) {
                    if (tb < nblk) {
#pragma unroll
                        for (uint32_t pc = 0; pc < 3; pc++) {
                            const bf16x8 a0 = afrag(A, pc, tb, col), a1 = afrag(A, pc, tb, col + 16u);
                            d0[tb] = mma(a0, bx01, d0[tb]);
                            d0[tb] = mma(a1, bx23, d0[tb]);
                            d1[tb] = mma(a0, by01, d1[tb]);
                            d1[tb] = mma(a1, by23, d1[tb]);
                        }
                    }
                }
            }
        });
        if (qv) {
#pragma unroll
            for (uint32_t tb = 0; tb < 2; tb++) {
#pragma unroll
                for (uint32_t i = 0; i < 4; i++) {
                    const uint32_t m = tb * 16u + 4u * g + i;
                    if (m < nt) {
                        float* o = b.expout + (size_t)(c0 + m) * H + 32u * q;
                        gst(o + n, d0[tb][i]);
                        gst(o + 16u + n, d1[tb][i]);
                    }
                }
            }
        }
        lds_barrier();
    }
}

struct BfW {
    u32x4 w[8];
};
// Shared gate/up + SwiGLU. Unit u = (pass p, slice j): tokens [p*kMT, +kMT),
// rows [64j, 64j+64) of the shared gate and up (wave v: tile 8j + v, native
// sgu chunks: 8 bf16 per lane), K = H.
__global__ void __launch_bounds__(kThreads) bsgu_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, SI = a.SI;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, g = lane >> 4;
    const uint32_t v = uni(tid >> 6) & 7u;
    extern __shared__ __align__(16) uint8_t lds[];
    uint16_t* A = (uint16_t*)lds;
    const NativeShared NS = NativeShared::make(H, SI);
    const uint32_t S = SI / kSlice, nkt = H / 32u, P = cdiv(b.T, kMT);
    const rsrc_t rs = make_rsrc(a.sh_native + NS.sgu, (uint32_t)(NS.sdn - NS.sgu));
    for (uint32_t u = blockIdx.x; u < P * S; u += gridDim.x) {
        const uint32_t p = u / S, j = u % S;
        const uint32_t nt = min(kMT, b.T - p * kMT), t0 = p * kMT;
        const uint32_t tile = j * (kSlice / 8u) + v;
        const uint32_t voff = tile * nkt * 1024u + 16u * lane;
        const uint32_t nblk = cdiv(nt, 16u);
        f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        auto row = [&](uint32_t m) { return b.norm + (size_t)(t0 + m) * H; };
        const uint32_t nst = cdiv(H, kKC);
        auto issue = [&](uint32_t st, BfW& W) {
            const bool live = st < nst;
#pragma unroll
            for (uint32_t s8 = 0; s8 < 8; s8++)
                W.w[s8] = bld16_nt(rs, voff, live ? min(st * 8u + s8, nkt - 1u) * 1024u : kOOB);
        };
        BfW W0, W1;
        issue(0, W0);
        steps2(nst, W0, W1, [&](uint32_t st, const BfW& cur, BfW& nxt) {
            AStage as;
            a_load(as, row, nt, st * kKC, H);
            issue(st + 1u, nxt);
            lds_barrier();
            a_store(A, as);
            lds_barrier();
#pragma unroll
            for (uint32_t s8 = 0; s8 < 8; s8++) {
                const u32x4 z = {0u, 0u, 0u, 0u};
                mma_blocks(acc, A, nblk, s8 * 32u + 8u * g, as_bf16x8(st * 8u + s8 < nkt ? cur.w[s8] : z));
            }
        });
        swiglu_store(acc, nt, [&](uint32_t m, uint32_t n, float x) {
            gst(b.smid + (size_t)(t0 + m) * SI + j * kSlice + v * 8u + n, x);
        });
        lds_barrier();
    }
}

// Shared down. Unit u = (pass p, row block rb): output rows [128rb, +128)
// (wave v: rows r0 = 128rb + 16v .. +16), K = SI. Native sdn: 16 bytes (8 bf16
// columns of tile T) per row; lane (n, g) of k step s reads tile 4s + g of
// row r0 + n.
__global__ void __launch_bounds__(kThreads) bsdn_kernel(const DecodeArgs* __restrict__ pa, const BatchArgs b) {
    const DecodeArgs& a = *pa;
    const uint32_t H = a.H, SI = a.SI;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, n = lane & 15u, g = lane >> 4;
    const uint32_t v = uni(tid >> 6) & 7u;
    extern __shared__ __align__(16) uint8_t lds[];
    uint16_t* A = (uint16_t*)lds;
    const NativeShared NS = NativeShared::make(H, SI);
    const uint32_t RB = cdiv(H, 128u), P = cdiv(b.T, kMT), nks = SI / 32u;
    const rsrc_t rs = make_rsrc(a.sh_native + NS.sdn, (uint32_t)(NS.total - NS.sdn));
    for (uint32_t u = blockIdx.x; u < P * RB; u += gridDim.x) {
        const uint32_t p = u / RB, rb = u % RB;
        const uint32_t nt = min(kMT, b.T - p * kMT), t0 = p * kMT;
        const uint32_t r0 = rb * 128u + v * 16u;
        const bool rv = r0 + n < H;
        const uint32_t voff = (g * H + min(r0 + n, H - 1u)) * 16u;
        const uint32_t nblk = cdiv(nt, 16u);
        f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
        auto row = [&](uint32_t m) { return b.smid + (size_t)(t0 + m) * SI; };
        const uint32_t nst = cdiv(SI, kKC);
        auto issue = [&](uint32_t st, BfW& W) {
            const bool live = st < nst;
#pragma unroll
            for (uint32_t s8 = 0; s8 < 8; s8++)
                W.w[s8] = bld16_nt(rs, voff, live ? min(st * 8u + s8, nks - 1u) * 4u * H * 16u : kOOB);
        };
        BfW W0, W1;
        issue(0, W0);
        steps2(nst, W0, W1, [&](uint32_t st, const BfW& cur, BfW& nxt) {
            AStage as;
            a_load(as, row, nt, st * kKC, SI);
            issue(st + 1u, nxt);
            lds_barrier();
            a_store(A, as);
            lds_barrier();
#pragma unroll
            for (uint32_t s8 = 0; s8 < 8; s8++) {
                const u32x4 z = {0u, 0u, 0u, 0u};
                mma_blocks(acc, A, nblk, s8 * 32u + 8u * g, as_bf16x8(st * 8u + s8 < nks ? cur.w[s8] : z));
            }
        });
        if (rv) {
#pragma unroll
            for (uint32_t tb = 0; tb < 2; tb++) {
#pragma unroll
                for (uint32_t i = 0; i < 4; i++) {
                    const uint32_t m = tb * 16u + 4u * g + i;
                    if (m < nt) gst(b.shout + (size_t)(t0 + m) * H + r0 + n, acc[tb][i]);
                }
            }
        }
        lds_barrier();
    }
}

// out[t] = (resid[t] +) sum_k w[t][k] e_k[t] in slot order + shared[t]
// (reference pass 3, src/glm_layer_runner.cuh:904-921).
__global__ void __launch_bounds__(256) bcomb_kernel(const BatchArgs b, uint32_t H, uint32_t K) {
    const uint32_t t = blockIdx.y;
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= H) return;
    float acc = 0.f;
    for (uint32_t k = 0; k < K; k++) {
        const uint32_t c = gld(b.pos + (size_t)t * K + k);
        acc = fmaf(gld(b.wts + (size_t)t * K + k), gld(b.expout + (size_t)c * H + r), acc);
    }
    acc += gld(b.shout + (size_t)t * H + r);
    if (b.resid) acc = gld(b.resid + (size_t)t * H + r) + acc;
    gst(b.out + (size_t)t * H + r, acc);
}

int launch_batched(const DecodeArgs* d_args, const BatchArgs& b, uint32_t H, uint32_t I, uint32_t SI, uint32_t E,
                   uint32_t K, uint32_t n_cu, void* stream) {
    (void)I;
    (void)SI;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    const size_t route_lds = 0;
    const size_t topk_lds = 4u * (2u * E + 64u);
    const size_t gemm_lds = kALds + 4u * kMT + 8u * E;
    const struct { const void* fn; size_t lds; } attrs[] = {
        {(const void*)btopk_kernel, topk_lds},
        {(const void*)bgu_kernel, gemm_lds},     {(const void*)bdn_kernel, gemm_lds},
        {(const void*)bsgu_kernel, gemm_lds},    {(const void*)bsdn_kernel, gemm_lds}};
    for (const auto& at : attrs)
        if ((e = hipFuncSetAttribute(at.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)at.lds)) != hipSuccess)
            return (int)e;
    const uint32_t G = 2u * n_cu;  // two work-groups per CU fit the LDS of the GEMM kernels
    hipLaunchKernelGGL(bnorm_kernel, dim3(b.T), dim3(kThreads), 0, s, d_args, b);
    hipLaunchKernelGGL(broute_kernel, dim3(kRouteGX, (b.T + kTB - 1) / kTB), dim3(kThreads), route_lds, s, d_args, b);
    hipLaunchKernelGGL(btopk_kernel, dim3(b.T), dim3(kThreads), topk_lds, s, d_args, b);
    hipLaunchKernelGGL(bcount_kernel, dim3(E), dim3(64), 0, s, b, K);
    hipLaunchKernelGGL(bscatter_kernel, dim3(E), dim3(256), 0, s, b, E);
    hipLaunchKernelGGL(bsgu_kernel, dim3(G), dim3(kThreads), gemm_lds, s, d_args, b);
    hipLaunchKernelGGL(bsdn_kernel, dim3(G), dim3(kThreads), gemm_lds, s, d_args, b);
    hipLaunchKernelGGL(bgu_kernel, dim3(G), dim3(kThreads), gemm_lds, s, d_args, b);
    hipLaunchKernelGGL(bdn_kernel, dim3(G), dim3(kThreads), gemm_lds, s, d_args, b);
    hipLaunchKernelGGL(bcomb_kernel, dim3((H + 255) / 256, b.T), dim3(256), 0, s, b, H, K);
    return (int)hipGetLastError();
}

}  // namespace wl
