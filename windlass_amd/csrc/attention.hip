// attention.hip — the caller side of a decoder layer on gfx950: the bf16
// projections of MLA attention and of the dense MLP as one streaming GEMV
// kernel (RMSNorm / SwiGLU of its input and the residual fused in), and the
// decode attention over the KV cache: absorbed MLA (q_nope folded into the
// compressed KV space, so the cache holds only kv_c [L] and k_rot [RP] per
// position), the DSA indexer's scores and top-k selection, and a key-split
// softmax with a combine.
//
// Reference: run_attention (src/glm_layer_runner.cuh:525-661), mla_absorb_q /
// mla_decode_absorbed / mla_project_v (:198-300), launch_indexer_decode and
// the index mask (src/glm_kernels.cuh:380-560), the dense branch of run_moe
// (src/glm_layer_runner.cuh:373-384).
//
// Differences from the reference, on purpose: the indexer key cache holds
// f32 (the reference's CUDA stores bf16, its numpy and transformers f32); the
// RoPE angles are computed in double (as the reference's numpy does) on the
// device, so no host table or host copy per layer is needed.
#include <hip/hip_runtime.h>
#include <math.h>

#include "attention.h"
#include "dev_common.h"

namespace wl {
namespace attn {

namespace {

constexpr int kMaxIt = 8;  // chunk iterations per thread: K <= 8 x 8 x 256 = 16384
#ifndef WL_GEMV_PRE
#define WL_GEMV_PRE 3
#endif
constexpr int kPre = WL_GEMV_PRE;  // chunk iterations whose weight loads are issued before the input transform

WL_DEV float silu(float x) { return x / (1.0f + expf(-x)); }

// 8 bf16 (one 16-byte chunk) -> f32
WL_DEV void bf8(u32x4 v, float* o) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o[2 * i] = __uint_as_float(v[i] << 16);
        o[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
    }
}

WL_DEV u32x4 ld16_nt(const void* p) { return __builtin_nontemporal_load((const u32x4*)p); }

// Walks the flat indices i = t0, t0 + step, ... < rows x cols of a row-major
// grid as (row, col) pairs without a division per element (one at the start).
struct Walk2 {
    uint32_t r, c, dr, dc, cols;
    __device__ __forceinline__ Walk2(uint32_t t0, uint32_t step, uint32_t cols_) : cols(cols_) {
        r = t0 / cols;
        c = t0 - r * cols;
        dr = step / cols;
        dc = step - dr * cols;
    }
    __device__ __forceinline__ void next() {
        r += dr;
        c += dc;
        if (c >= cols) {
            c -= cols;
            r++;
        }
    }
};

// Sum over the `tpr` lanes of a thread group (groups aligned to tpr lanes; for
// tpr > 64 through LDS `red`, kGemvThreads / 64 entries per value, index v).
template <int NV>
WL_DEV void group_sum(float (&v)[NV], uint32_t tpr_log2, float* red) {
    const uint32_t tpr = 1u << tpr_log2;
    const uint32_t lim = tpr < 64 ? tpr : 64;
    for (uint32_t o = lim >> 1; o > 0; o >>= 1)
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] += __shfl_xor(v[i], (int)o, 64);
    if (tpr > 64) {
        const uint32_t w = threadIdx.x >> 6, nw = tpr >> 6;
        __syncthreads();
        if ((threadIdx.x & 63) == 0)
#pragma unroll
            for (int i = 0; i < NV; i++) red[i * 4 + w] = v[i];
        __syncthreads();
        const uint32_t g0 = (w / nw) * nw;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            float s = 0.f;
            for (uint32_t k = 0; k < nw; k++) s += red[i * 4 + g0 + k];
            v[i] = s;
        }
    }
}

// Work-group b of a GEMV launch.
WL_DEV void gemv_body(const GemvLaunch& L, uint32_t b) {
    __shared__ float red[(kGemvRows + 1) * 4];
    // the job of this work-group (uniform branches: kernel-argument loads at fixed offsets)
    GemvJob j = L.job[0];
    if (L.n_jobs > 3 && b >= L.job[3].wg0) j = L.job[3];
    else if (L.n_jobs > 2 && b >= L.job[2].wg0) j = L.job[2];
    else if (L.n_jobs > 1 && b >= L.job[1].wg0) j = L.job[1];
    const uint32_t tl2 = j.tpr_log2, tpr = 1u << tl2;
    const uint32_t tid = threadIdx.x, grp = tid >> tl2, lt = tid & (tpr - 1);
    const uint32_t r0 = (b - j.wg0) * j.rows_wg + grp * kGemvRows;
    const uint32_t K = j.K, nch = K >> 3;
    const uint32_t nit = (nch + tpr - 1) >> tl2;
    // the group's x and W rows (rows of one thread group share a group: G % kGemvRows == 0)
    const uint32_t rg = j.GS ? (r0 < j.N ? r0 : 0) / j.G : 0;
    const float* x = j.x + (size_t)rg * j.XS;
    const uint32_t wr0 = j.GS ? rg * j.GS + j.OFF + (r0 - rg * j.G) : r0;
    size_t roff[kGemvRows];
#pragma unroll
    for (int r = 0; r < (int)kGemvRows; r++) roff[r] = (size_t)(wr0 + r) * K;
    // the first chunks' weights are requested before the input is read and
    // normalised, so the work-group's first memory latency overlaps that work
    u32x4 pre[kPre][kGemvRows];
    if (!j.f32w) {
        const uint16_t* W = (const uint16_t*)j.W;
#pragma unroll
        for (int i = 0; i < kPre; i++) {
            const uint32_t c = lt + ((uint32_t)i << tl2);
            if (i < (int)nit && c < nch)
#pragma unroll
                for (int r = 0; r < (int)kGemvRows; r++)
                    if (r0 + r < j.N) pre[i][r] = ld16_nt(W + roff[r] + 8 * c);
        }
    }
    float xv[kMaxIt][8];
    float ss[1] = {0.f};
#pragma unroll
    for (int i = 0; i < kMaxIt; i++) {
        const uint32_t c = lt + ((uint32_t)i << tl2);
#pragma unroll
        for (int e = 0; e < 8; e++) xv[i][e] = 0.f;
        if (i < (int)nit && c < nch) {
            const f32x4 a = *(const f32x4*)(x + 8 * c), a2 = *(const f32x4*)(x + 8 * c + 4);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xv[i][e] = a[e];
                xv[i][4 + e] = a2[e];
            }
            if (j.x2) {
                const float* u = j.x2 + (x - j.x);
                const f32x4 b0 = *(const f32x4*)(u + 8 * c), b1 = *(const f32x4*)(u + 8 * c + 4);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    xv[i][e] = silu(xv[i][e]) * b0[e];
                    xv[i][4 + e] = silu(xv[i][4 + e]) * b1[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 8; e++) ss[0] += xv[i][e] * xv[i][e];
        }
    }
    if (j.norm_w) {
        group_sum<1>(ss, tl2, red);
        const float rs = 1.0f / sqrtf(ss[0] / (float)K + j.eps);
#pragma unroll
        for (int i = 0; i < kMaxIt; i++) {
            const uint32_t c = lt + ((uint32_t)i << tl2);
            if (i < (int)nit && c < nch) {
                float w[8];
                bf8(gld16(j.norm_w + 8 * c), w);
#pragma unroll
                for (int e = 0; e < 8; e++) xv[i][e] = w[e] * (xv[i][e] * rs);
            }
        }
    }
    if (j.x_out && b == j.wg0 && grp == 0) {
#pragma unroll
        for (int i = 0; i < kMaxIt; i++) {
            const uint32_t c = lt + ((uint32_t)i << tl2);
            if (i < (int)nit && c < nch) {
                *(f32x4*)(j.x_out + 8 * c) = f32x4{xv[i][0], xv[i][1], xv[i][2], xv[i][3]};
                *(f32x4*)(j.x_out + 8 * c + 4) = f32x4{xv[i][4], xv[i][5], xv[i][6], xv[i][7]};
            }
        }
    }
    float acc[kGemvRows];
#pragma unroll
    for (int r = 0; r < (int)kGemvRows; r++) acc[r] = 0.f;
    if (j.f32w) {
        const float* W = (const float*)j.W;
#pragma unroll
        for (int i = 0; i < kMaxIt; i++) {
            const uint32_t c = lt + ((uint32_t)i << tl2);
            if (i < (int)nit && c < nch) {
#pragma unroll
                for (int r = 0; r < (int)kGemvRows; r++) {
                    if (r0 + r < j.N) {
                        const u32x4 w0 = ld16_nt(W + roff[r] + 8 * c), w1 = ld16_nt(W + roff[r] + 8 * c + 4);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            acc[r] += __uint_as_float(w0[e]) * xv[i][e];
                            acc[r] += __uint_as_float(w1[e]) * xv[i][4 + e];
                        }
                    }
                }
            }
        }
    } else {
        const uint16_t* W = (const uint16_t*)j.W;
#pragma unroll
        for (int i = 0; i < kMaxIt; i++) {
            const uint32_t c = lt + ((uint32_t)i << tl2);
            if (i < (int)nit && c < nch) {
                u32x4 wv[kGemvRows];
#pragma unroll
                for (int r = 0; r < (int)kGemvRows; r++)
                    if (r0 + r < j.N) wv[r] = i < kPre ? pre[i < kPre ? i : 0][r] : ld16_nt(W + roff[r] + 8 * c);
#pragma unroll
                for (int r = 0; r < (int)kGemvRows; r++) {
                    if (r0 + r < j.N) {
                        float w[8];
                        bf8(wv[r], w);
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[r] += w[e] * xv[i][e];
                    }
                }
            }
        }
    }
    group_sum<kGemvRows>(acc, tl2, red);
    if (lt == 0) {
#pragma unroll
        for (int r = 0; r < (int)kGemvRows; r++) {
            const uint32_t row = r0 + r;
            if (row < j.N) {
                if (j.y_raw) j.y_raw[row] = acc[r];
                j.y[row] = (j.add ? j.add[row] : 0.f) + acc[r];
            }
        }
    }
}

__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvLaunch L) { gemv_body(L, blockIdx.x); }

// Sum / max over the 256 threads of a work-group (result in every thread).
WL_DEV float wg_sum(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// RoPE table of position pos: cs[i] = cos, cs[rot/2 + i] = sin of pos /
// theta^(2i / rot), computed in double and rounded to f32.
WL_DEV void rope_table(float* cs, uint32_t rot, uint32_t pos, float theta) {
    for (uint32_t i = threadIdx.x; i < rot / 2; i += blockDim.x) {
        const double inv = 1.0 / pow((double)theta, (double)(2 * i) / (double)rot);
        const double a = (double)pos * inv;
        cs[i] = (float)cos(a);
        cs[rot / 2 + i] = (float)sin(a);
    }
}

// Interleaved RoPE of in[0, rot) (pairs 2i, 2i+1) into the halves layout of
// out[0, rot): out[i] = a cos - b sin, out[rot/2 + i] = b cos + a sin, for
// `n` vectors (in + v * istride, out + v * ostride); threads stride over
// (vector, pair). in and out must not overlap.
WL_DEV void rope(const float* in, uint32_t istride, float* out, uint32_t ostride, uint32_t n, const float* cs,
                 uint32_t rot) {
    const uint32_t hp = rot / 2;
    for (uint32_t k = threadIdx.x; k < n * hp; k += blockDim.x) {
        const uint32_t v = k / hp, i = k % hp;
        const float c = cs[i], sn = cs[hp + i];
        const float a = in[(size_t)v * istride + 2 * i], b = in[(size_t)v * istride + 2 * i + 1];
        out[(size_t)v * ostride + i] = a * c - b * sn;
        out[(size_t)v * ostride + hp + i] = b * c + a * sn;
    }
}

static_assert(kGemvThreads == 256, "the prep and GEMV bodies share a launch of 256-thread work-groups");
// Work-group blk (0: the KV rows, 1: the indexer key row) of the prep stage.
// LDS: kPrepLds floats (red [4] | kbuf [1024] | cs [512]).
constexpr uint32_t kPrepLds = 4 + 1024 + 512;
WL_DEV void prep_body(const Shape& s, const AttnPtrs& p, uint32_t pos, uint32_t blk, float* lds) {
    float* red = lds;
    float* kbuf = lds + 4;
    float* cs = lds + 4 + 1024;
    const uint32_t tid = threadIdx.x;
    rope_table(cs, s.RP, pos, s.theta);
    __syncthreads();
    if (blk == 0)
        for (uint32_t i = tid; i < s.RP; i += 256) p.rope_cs[i] = cs[i];  // for the query RoPE
    if (blk == 0) {
        // kv_c row = RMSNorm(kv_raw[0, L), kv_a_ln, 1e-6); k_rot row = RoPE(kv_raw[L, L + RP))
        float ss = 0.f;
        for (uint32_t i = tid; i < s.L; i += 256) ss += p.kv_raw[i] * p.kv_raw[i];
        ss = wg_sum(ss, red);
        const float rs = 1.0f / sqrtf(ss / (float)s.L + 1e-6f);
        float* row = p.kv_c + (size_t)pos * s.L;
        for (uint32_t i = tid; i < s.L; i += 256) row[i] = bf2f(p.kv_a_ln[i]) * (p.kv_raw[i] * rs);
        rope(p.kv_raw + s.L, 0, p.k_rot + (size_t)pos * s.RP, 0, 1, cs, s.RP);
    } else {
        // indexer key row = RoPE_lead(LayerNorm(ik_raw, w, b, 1e-6)); head weights x IH^-0.5
        float sum = 0.f;
        for (uint32_t i = tid; i < s.ID; i += 256) sum += p.ik_raw[i];
        const float mu = wg_sum(sum, red) / (float)s.ID;
        float var = 0.f;
        for (uint32_t i = tid; i < s.ID; i += 256) var += (p.ik_raw[i] - mu) * (p.ik_raw[i] - mu);
        var = wg_sum(var, red) / (float)s.ID;
        const float den = sqrtf(var + 1e-6f);
        for (uint32_t i = tid; i < s.ID; i += 256)
            kbuf[i] = (p.ik_raw[i] - mu) / den * bf2f(p.idx_k_norm_w[i]) + bf2f(p.idx_k_norm_b[i]);
        __syncthreads();
        float* row = p.idx_k + (size_t)pos * s.ID;
        rope(kbuf, 0, row, 0, 1, cs, s.RP);
        for (uint32_t i = s.RP + tid; i < s.ID; i += 256) row[i] = kbuf[i];
        for (uint32_t h = tid; h < s.IH; h += 256) p.iw[h] *= p.iw_scale;
    }
}

// A GEMV launch whose last work-groups run the prep stage (the two depend on
// the same earlier stage only), so the prep needs no launch of its own.
__global__ __launch_bounds__(kGemvThreads) void gemv_prep_kernel(GemvLaunch L, uint32_t n_gemv, Shape s, AttnPtrs p,
                                                                 uint32_t pos) {
    __shared__ float lds[kPrepLds];
    if (blockIdx.x < n_gemv) gemv_body(L, blockIdx.x);
    else prep_body(s, p, pos, blockIdx.x - n_gemv, lds);
}

// ---- streaming GEMV ------------------------------------------------------------
// Work-group b of a job takes rows [rs, re) of an even split of the job's N
// rows over its nwg work-groups. It stages its input once in LDS (DMA,
// zero-padded to whole units, RMSNorm applied there), and runs its rows as one
// flat sequence of 1 KB weight units (row vr, unit c: 512 bf16 or 256 f32
// columns) split evenly over its four waves. A wave streams its units in
// batches of kSgNB non-temporal 16-byte loads per lane, two batches in flight,
// and sums a row's products in two f32 accumulators per lane; at a row change
// the wave's sum goes to LDS slot [row][wave], and the four slots of a row are
// added in wave order at the end. The weights of a work-group's first two
// batches are requested right after its input DMAs, so both arrive while the
// input is normalised. A paired job (W2) runs the rows of W, then those of W2,
// and writes silu(W x) * (W2 x).
#ifndef WL_SG_NB
#define WL_SG_NB 4
#endif
constexpr uint32_t kSgNB = WL_SG_NB;  // 1 KB units per batch

struct SgWG {
    const uint8_t *w1, *w2;  // weight bytes of row wr0 (W, W2)
    uint32_t wbytes;         // resource size: the rows [wr0, wr(re - 1)] of W
    uint32_t rs, R, K, esz, epu, nL, Kp;
    uint32_t G, GS, OFF, wr0, g0;
};
struct SgCursor {  // wave-uniform
    uint32_t u, vr, c, roff;
    uint32_t rr, gi;  // the row's index in its group, its group - g0
};

WL_DEV uint32_t sg_wrow(const SgWG& g, uint32_t r) { return g.GS ? (r / g.G) * g.GS + g.OFF + r % g.G : r; }
WL_DEV void sg_row_start(const SgWG& g, SgCursor& cu) {
    const uint32_t r = g.rs + (cu.vr < g.R ? cu.vr : cu.vr - g.R);
    cu.roff = (sg_wrow(g, r) - g.wr0) * g.K * g.esz;
    cu.rr = g.GS ? r % g.G : 0u;
    cu.gi = g.GS ? r / g.G - g.g0 : 0u;
}
WL_DEV void sg_start(const SgWG& g, SgCursor& cu, uint32_t u) {
    cu.u = u;
    cu.vr = u / g.nL;
    cu.c = u - cu.vr * g.nL;
    sg_row_start(g, cu);
}
// The next unit; the next row without a division, except where a paired
// job's W2 rows begin.
WL_DEV void sg_next(const SgWG& g, SgCursor& cu) {
    cu.u++;
    if (++cu.c == g.nL) {
        cu.c = 0;
        if (++cu.vr == g.R) {
            sg_row_start(g, cu);
        } else {
            cu.roff += g.K * g.esz;
            if (g.GS && ++cu.rr == g.G) {
                cu.rr = 0;
                cu.gi++;
                cu.roff += (g.GS - g.G) * g.K * g.esz;
            }
        }
    }
}
// The load of the cursor's unit (lanes past K, and units past u1, read zeros
// without a memory access).
WL_DEV u32x4 sg_load(const SgWG& g, const SgCursor& cu, uint32_t u1, uint32_t lane) {
    const uint32_t left = (g.K - cu.c * g.epu) * g.esz;  // bytes of the row from this unit on
    const bool ok = cu.u < u1 && 16u * lane < left;
    const rsrc_t r = make_rsrc(cu.vr < g.R ? g.w1 : g.w2, g.wbytes);
    return bld16_nt(r, ok ? 16u * lane : kOOB, cu.roff + cu.c * 1024u);
}
template <int CTRL, int ROWS>
WL_DEV float sum_step(float x) {
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWS, 0xF, false));
}
// Sum over the 64 lanes, returned uniform (DPP quad permutes, row shifts and
// row broadcasts leave it in lane 63).
WL_DEV float wave_sum(float x) {
    x = sum_step<0xB1, 0xF>(x);   // quad_perm [1,0,3,2]
    x = sum_step<0x4E, 0xF>(x);   // quad_perm [2,3,0,1]
    x = sum_step<0x114, 0xF>(x);  // row_shr:4
    x = sum_step<0x118, 0xF>(x);  // row_shr:8
    x = sum_step<0x142, 0xA>(x);  // row_bcast:15
    x = sum_step<0x143, 0xC>(x);  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

struct SgBatch {
    u32x4 w[kSgNB];
};
WL_DEV void sg_issue(const SgWG& g, SgCursor& ci, uint32_t u1, SgBatch& X) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (uint32_t i = 0; i < kSgNB; i++) {
        X.w[i] = sg_load(g, ci, u1, lane);
        sg_next(g, ci);
    }
}
// The wave's units [u0, u1) of a work-group whose weights are ESZ-byte values;
// batches A and B (the first two) are already issued, ci is two batches on.
template <uint32_t NW, uint32_t ESZ>
WL_DEV void sg_stream(const SgWG& g, uint32_t u0, uint32_t u1, SgCursor& ci, SgBatch& A, SgBatch& B,
                      const float* xs, float* part) {
    const uint32_t lane = threadIdx.x & 63u, v = uni(threadIdx.x >> 6);
    SgCursor cc;
    sg_start(g, cc, u0);
    float a0 = 0.f, a1 = 0.f;
    uint32_t cur = cc.vr, xoff = cc.gi * g.Kp;
    auto flush = [&]() {
        const float s = wave_sum(a0 + a1);
        if (lane == 0) part[cur * NW + v] = s;
        a0 = 0.f;
        a1 = 0.f;
    };
    auto consume = [&](uint32_t, const SgBatch& X) {
#pragma unroll
        for (uint32_t i = 0; i < kSgNB; i++) {
            if (cc.u < u1) {
                if (cc.vr != cur) {
                    flush();
                    cur = cc.vr;
                    xoff = cc.gi * g.Kp;
                }
                const u32x4 w = X.w[i];
                if (ESZ == 2u) {
                    const float* xp = xs + xoff + cc.c * 512u + 8u * lane;
                    const f32x4 x0 = *(const f32x4*)xp, x1 = *(const f32x4*)(xp + 4);
                    a0 += bf2f(w[0] & 0xFFFFu) * x0[0];
                    a1 += bf2f(w[0] >> 16) * x0[1];
                    a0 += bf2f(w[1] & 0xFFFFu) * x0[2];
                    a1 += bf2f(w[1] >> 16) * x0[3];
                    a0 += bf2f(w[2] & 0xFFFFu) * x1[0];
                    a1 += bf2f(w[2] >> 16) * x1[1];
                    a0 += bf2f(w[3] & 0xFFFFu) * x1[2];
                    a1 += bf2f(w[3] >> 16) * x1[3];
                } else {
                    const f32x4 x0 = *(const f32x4*)(xs + xoff + cc.c * 256u + 4u * lane);
                    a0 += __uint_as_float(w[0]) * x0[0];
                    a1 += __uint_as_float(w[1]) * x0[1];
                    a0 += __uint_as_float(w[2]) * x0[2];
                    a1 += __uint_as_float(w[3]) * x0[3];
                }
            }
            sg_next(g, cc);
        }
    };
    auto issue = [&](uint32_t, SgBatch& X) { sg_issue(g, ci, u1, X); };
    pingpong(at_least2(cdiv(u1 - u0, kSgNB)), A, B, issue, consume);
    if (u1 > u0) flush();
}

// Work-group b (< the launch's GEMV work-groups) of a streaming launch.
template <uint32_t NW>
WL_DEV void sgemv_body(const GemvLaunch& L, uint32_t b, float* lds) {
    GemvJob j = L.job[0];
    if (L.n_jobs > 3 && b >= L.job[3].wg0) j = L.job[3];
    else if (L.n_jobs > 2 && b >= L.job[2].wg0) j = L.job[2];
    else if (L.n_jobs > 1 && b >= L.job[1].wg0) j = L.job[1];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, v = uni(tid >> 6);
    const uint32_t bj = b - j.wg0;
    SgWG g;
    g.rs = (uint32_t)((uint64_t)j.N * bj / j.nwg);
    const uint32_t re = (uint32_t)((uint64_t)j.N * (bj + 1u) / j.nwg);
    g.R = re - g.rs;
    g.K = j.K;
    g.esz = j.f32w ? 4u : 2u;
    g.epu = 1024u / g.esz;
    g.nL = cdiv(g.K, g.epu);
    g.Kp = g.nL * g.epu;
    g.G = j.G;
    g.GS = j.GS;
    g.OFF = j.OFF;
    g.wr0 = sg_wrow(g, g.rs);
    g.g0 = j.GS ? g.rs / j.G : 0u;
    const uint32_t ng = j.GS ? (re - 1u) / j.G - g.g0 + 1u : 1u;
    g.wbytes = (sg_wrow(g, re - 1u) - g.wr0 + 1u) * g.K * g.esz;
    g.w1 = (const uint8_t*)j.W + (size_t)g.wr0 * g.K * g.esz;
    g.w2 = j.W2 ? (const uint8_t*)j.W2 + (size_t)g.wr0 * g.K * g.esz : g.w1;
    const uint32_t VR = j.W2 ? 2u * g.R : g.R;
    // LDS: x [ng][Kp] f32 | norm weights (bf16, whole 1 KB units) | part [VR][4] | red [4]
    float* xs = lds;
    uint16_t* nw = (uint16_t*)(xs + (size_t)ng * g.Kp);
    float* part = (float*)(nw + (j.norm_w ? cdiv(g.Kp, 512u) * 512u : 0u));
    float* red = part + VR * NW;

    // 1. input DMAs: group gi's x (f32, K columns, then zeros to Kp), the norm weights
    {
        const float* xb = j.x + (size_t)g.g0 * j.XS;
        const rsrc_t xr = make_rsrc(xb, ((ng - 1u) * j.XS + g.K) * 4u);
        const uint32_t cpg = g.Kp / 256u, nch = ng * cpg;
        for (uint32_t ci = v; ci < nch; ci += NW) {
            const uint32_t gi = ci / cpg, col = (ci - gi * cpg) * 256u + 4u * lane;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)(xs + ci * 256u), 16u,
                                                     col < g.K ? (gi * j.XS + col) * 4u : kOOB, 0, 0, 0);
        }
        if (j.norm_w) {
            const rsrc_t nr = make_rsrc(j.norm_w, g.K * 2u);
            const uint32_t nchw = cdiv(g.Kp, 512u);
            for (uint32_t ci = v; ci < nchw; ci += NW) {
                const uint32_t col = ci * 512u + 8u * lane;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(nr, (__attribute__((address_space(3))) void*)(nw + ci * 512u),
                                                         16u, col < g.K ? col * 2u : kOOB, 0, 0, 0);
            }
        }
    }
    // 2. the wave's units and its first two batches
    const uint32_t n = VR * g.nL;
    const uint32_t u0 = (uint32_t)((uint64_t)n * v / NW), u1 = (uint32_t)((uint64_t)n * (v + 1u) / NW);
    SgCursor ci;  // the issue cursor
    sg_start(g, ci, u0);
    SgBatch A, B;
    sg_issue(g, ci, u1, A);
    sg_issue(g, ci, u1, B);
    for (uint32_t i = tid; i < VR * NW; i += 64u * NW) part[i] = 0.f;
    // 3. the input in LDS (the 2 kSgNB weight loads issued after the DMAs may
    // stay in flight), then RMSNorm in place
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((2u * kSgNB & 15u) | (((2u * kSgNB) >> 4) << 14) | 0x0F70u);
    lds_barrier();
    const uint32_t nx = ng * g.Kp;
    if (j.norm_w) {  // ungrouped (ng = 1)
        float ss = 0.f;
        for (uint32_t k = 4u * tid; k < nx; k += 256u * NW) {
            const f32x4 a = *(const f32x4*)(xs + k);
            ss += a[0] * a[0] + a[1] * a[1] + a[2] * a[2] + a[3] * a[3];
        }
        ss = wave_sum(ss);
        if (lane == 0) red[v] = ss;
        lds_barrier();
        float t = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < NW; w++) t += red[w];
        const float rsn = 1.0f / sqrtf(t / (float)g.K + j.eps);
        for (uint32_t k = 4u * tid; k < nx; k += 256u * NW) {
            f32x4 a = *(const f32x4*)(xs + k);
            const uint2 wb = *(const uint2*)(nw + k);
            a[0] = bf2f(wb.x & 0xFFFFu) * (a[0] * rsn);
            a[1] = bf2f(wb.x >> 16) * (a[1] * rsn);
            a[2] = bf2f(wb.y & 0xFFFFu) * (a[2] * rsn);
            a[3] = bf2f(wb.y >> 16) * (a[3] * rsn);
            *(f32x4*)(xs + k) = a;
        }
        lds_barrier();
    }
    if (j.x_out && bj == 0u)
        for (uint32_t k = 4u * tid; k < g.K; k += 256u * NW) *(f32x4*)(j.x_out + k) = *(const f32x4*)(xs + k);
    // 4. the stream
    if (g.esz == 2u) sg_stream<NW, 2>(g, u0, u1, ci, A, B, xs, part);
    else sg_stream<NW, 4>(g, u0, u1, ci, A, B, xs, part);
    lds_barrier();
    // 5. each row: its four wave slots in order (+ add)
    for (uint32_t t = tid; t < g.R; t += 64u * NW) {
        float y = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < NW; w++) y += part[t * NW + w];
        if (j.W2) {
            float y2 = 0.f;
#pragma unroll
            for (uint32_t w = 0; w < NW; w++) y2 += part[(g.R + t) * NW + w];
            y = silu(y) * y2;
        }
        const uint32_t row = g.rs + t;
        if (j.y_raw) j.y_raw[row] = y;
        j.y[row] = (j.add ? j.add[row] : 0.f) + y;
    }
}

// Four waves per work-group, two work-groups per CU at the GLM shapes (one
// eight-wave work-group per CU, staging the input once per CU, measured within
// 1 % of it on every attention and MLP shape). Work-groups past n_gemv run
// the prep stage.
__global__ __launch_bounds__(256) void sgemv_kernel(GemvLaunch L, uint32_t n_gemv, Shape s, AttnPtrs p, uint32_t pos) {
    extern __shared__ __align__(16) float sg_lds[];
    if (blockIdx.x < n_gemv) sgemv_body<4>(L, blockIdx.x, sg_lds);
    else prep_body(s, p, pos, blockIdx.x - n_gemv, sg_lds);
}

// q_abs[h][c] = sum_{d < NP} q[h][d] * kv_b[h (NP + VD) + d][c]: work-group
// (h, column block of up to 128 columns); 8 columns per thread, the rows
// split over the remaining thread dimension and summed through LDS. The last
// work-group applies RoPE to the queries.
WL_DEV void index_score_body(const Shape& s, const AttnPtrs& p, uint32_t T, uint32_t blk, float* lq);

// Work-groups [0, HN nb): the absorption; HN nb: the RoPE of the queries;
// after it, on owner layers, the index scores over T keys (kIdxKeys per
// work-group), which depend on the same earlier stages only.
__global__ __launch_bounds__(256) void attn_absorb_kernel(Shape s, AttnPtrs p, uint32_t owner, uint32_t T) {
    __shared__ float red[2048];
    extern __shared__ float dyn[];
    const uint32_t tid = threadIdx.x;
    const uint32_t nb = (s.L + 127) / 128;
    const uint32_t DH = s.NP + s.RP;
    if (blockIdx.x > s.HN * nb) {
        index_score_body(s, p, T, blockIdx.x - s.HN * nb - 1u, dyn);
        return;
    }
    if (blockIdx.x == s.HN * nb) {
        float* cs = red;
        for (uint32_t i = tid; i < s.RP; i += 256) cs[i] = p.rope_cs[i];
        __syncthreads();
        rope(p.q + s.NP, DH, p.q_rope, s.RP, s.HN, cs, s.RP);
        if (owner) {
            rope(p.iq, s.ID, p.iqr, s.ID, s.IH, cs, s.RP);
            for (uint32_t k = tid; k < s.IH * (s.ID - s.RP); k += 256) {
                const uint32_t h = k / (s.ID - s.RP), i = s.RP + k % (s.ID - s.RP);
                p.iqr[(size_t)h * s.ID + i] = p.iq[(size_t)h * s.ID + i];
            }
        }
        return;
    }
    const uint32_t h = blockIdx.x / nb, cb = blockIdx.x % nb;
    const uint32_t c0 = cb * 128, ncol = (s.L - c0) < 128 ? (s.L - c0) : 128;
    const uint32_t ct = ncol / 8, rl = 256 / ct;
    const uint32_t cl = tid % ct, rlane = tid / ct;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (rlane < rl) {
        const float* qh = p.q + (size_t)h * DH;
        const uint16_t* wb = p.kv_b + (size_t)h * (s.NP + s.VD) * s.L + c0 + 8 * cl;
        uint32_t d = rlane;
        for (; d + 3 * rl < s.NP; d += 4 * rl) {  // four rows' loads in flight
            u32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = ld16_nt(wb + (size_t)(d + u * rl) * s.L);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float w[8];
                bf8(v[u], w);
                const float qv = qh[d + u * rl];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] += qv * w[e];
            }
        }
        for (; d < s.NP; d += rl) {
            float w[8];
            bf8(ld16_nt(wb + (size_t)d * s.L), w);
            const float qv = qh[d];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] += qv * w[e];
        }
#pragma unroll
        for (int e = 0; e < 8; e++) red[rlane * ncol + 8 * cl + e] = acc[e];
    }
    __syncthreads();
    for (uint32_t c = tid; c < ncol; c += 256) {
        float t = 0.f;
        for (uint32_t r = 0; r < rl; r++) t += red[r * ncol + c];
        p.q_abs[(size_t)h * s.L + c0 + c] = t;
    }
}

// isc[t] = sum_h w[h] * relu(q[h] . k[t] * ID^-0.5): 16 keys per
// work-group; thread (key, head part): 2 consecutive heads of one key over
// all ID dims from LDS, then the head parts summed by shuffles in head order.
constexpr uint32_t kIdxKeys = 16;

// Work-group blk of the index scores. lq: q [IH][ID + 4] | w [IH] |
// k [kIdxKeys][ID + 4] | RoPE table [RP]. The query is the wq_b output with
// RoPE on its leading RP dims, applied here as the absorb stage's RoPE
// work-group applies it, so the scores need not wait for that work-group.
WL_DEV void index_score_body(const Shape& s, const AttnPtrs& p, uint32_t T, uint32_t blk, float* lq) {
    const uint32_t tid = threadIdx.x, QS = s.ID + 4;
    float* lw = lq + s.IH * QS;
    float* lk = lw + s.IH;
    float* cs = lk + kIdxKeys * QS;
    const uint32_t k0 = blk * kIdxKeys;
    const uint32_t nk = (T - k0) < kIdxKeys ? (T - k0) : kIdxKeys;
    for (uint32_t i = tid; i < s.RP; i += 256) cs[i] = p.rope_cs[i];
    __syncthreads();
    rope(p.iq, s.ID, lq, QS, s.IH, cs, s.RP);
    for (Walk2 w(tid, 256, (s.ID - s.RP) / 4); w.r < s.IH; w.next())
        *(f32x4*)(lq + w.r * QS + s.RP + 4 * w.c) = *(const f32x4*)(p.iq + (size_t)w.r * s.ID + s.RP + 4 * w.c);
    for (uint32_t i = tid; i < s.IH; i += 256) lw[i] = p.iw[i];
    for (Walk2 w(tid, 256, s.ID / 4); w.r < nk; w.next())
        *(f32x4*)(lk + w.r * QS + 4 * w.c) = *(const f32x4*)(p.idx_k + (size_t)(k0 + w.r) * s.ID + 4 * w.c);
    __syncthreads();
    const uint32_t key = tid >> 4, hp = tid & 15;
    const uint32_t hpt = (s.IH + 15) / 16;  // heads per thread (2 at IH = 32)
    float sc = 0.f;
    if (key < nk) {
        for (uint32_t j = 0; j < hpt; j++) {
            const uint32_t h = hp * hpt + j;
            if (h >= s.IH) break;
            const float* q = lq + h * QS;
            const float* k = lk + key * QS;
            float d = 0.f;
            for (uint32_t c = 0; c < s.ID; c += 4) {
                const f32x4 x = *(const f32x4*)(q + c), y = *(const f32x4*)(k + c);
                d += x[0] * y[0];
                d += x[1] * y[1];
                d += x[2] * y[2];
                d += x[3] * y[3];
            }
            sc += lw[h] * fmaxf(d * p.ix_scale, 0.f);
        }
    }
    sc += __shfl_xor(sc, 1, 64);
    sc += __shfl_xor(sc, 2, 64);
    sc += __shfl_xor(sc, 4, 64);
    sc += __shfl_xor(sc, 8, 64);
    if (key < nk && hp == 0) p.isc[k0 + key] = sc;
}


// Order-preserving key of an f32 (larger float -> larger key).
WL_DEV uint32_t okey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// keep[t] = 1 for the TOPK largest scores of [0, T) (ties to the lowest
// index), every key when T <= TOPK; klist[0, count) the kept keys in
// ascending order and klist[max_seq] = count (the list the attention core
// walks). One work-group; thread tid owns keys [tid per, tid per + per): a
// radix select of the TOPK-th largest key (4 passes of 8 bits), then the
// marking, then the list (each thread's kept keys at the exclusive prefix of
// the threads' counts). CACHED (per <= kTopkCache): each thread's keys stay
// in registers across the passes instead of being read again from memory.
constexpr uint32_t kTopkCache = 8;

template <bool CACHED>
WL_DEV void index_topk_body(const float* isc, uint8_t* keep, uint32_t* klist, uint32_t max_seq, uint32_t T,
                            uint32_t K) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t cnt[16];
    __shared__ uint32_t sh_prefix, sh_kk;
    const uint32_t tid = threadIdx.x;
    const uint32_t per = (T + 1023) / 1024, t0 = tid * per, t1 = (t0 + per < T) ? t0 + per : T;
    const uint32_t n = t1 > t0 ? t1 - t0 : 0u;
    uint32_t kc[CACHED ? kTopkCache : 1];
    if (CACHED) {
#pragma unroll
        for (uint32_t i = 0; i < kTopkCache; i++) kc[i] = i < n ? okey(isc[t0 + i]) : 0u;
    }
    // the key of this thread's i-th score
    auto key = [&](uint32_t i) { return CACHED ? kc[i] : okey(isc[t0 + i]); };
    constexpr uint32_t kLoop = CACHED ? kTopkCache : 0xFFFFFFFFu;
    uint32_t prefix = 0, mask = 0, kk = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t i = tid; i < 256; i += 1024) hist[i] = 0;
        __syncthreads();
        if (CACHED) {
#pragma unroll
            for (uint32_t i = 0; i < kTopkCache; i++) {
                const uint32_t u = kc[i];
                if (i < n && (u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
            }
        } else {
            for (uint32_t t = tid; t < T; t += 1024) {  // coalesced
                const uint32_t u = okey(isc[t]);
                if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
            }
        }
        __syncthreads();
        if (tid < 64) {
            // the digit d with (count above d) < kk <= (count above d) + hist[d]:
            // lane l holds bins 4l .. 4l + 3; counts above a lane by a suffix scan
            const uint32_t b0 = hist[4 * tid], b1 = hist[4 * tid + 1], b2 = hist[4 * tid + 2], b3 = hist[4 * tid + 3];
            const uint32_t own = b0 + b1 + b2 + b3;
            uint32_t inc = own;  // sum over lanes >= tid
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t v = __shfl_down(inc, o, 64);
                if (tid + o < 64) inc += v;
            }
            uint32_t above = inc - own;
            const uint32_t bins[4] = {b0, b1, b2, b3};
            for (int b = 3; b >= 0; b--) {
                if (above < kk && kk <= above + bins[b]) {
                    sh_prefix = prefix | ((4 * tid + b) << shift);
                    sh_kk = kk - above;
                }
                above += bins[b];
            }
        }
        __syncthreads();
        prefix = sh_prefix;
        kk = sh_kk;
        mask |= 255u << shift;
        __syncthreads();
    }
    // prefix: the key of the K-th largest score; kk (>= 1) of the keys equal
    // to it are kept, the lowest indices first
    uint32_t eq = 0;
#pragma unroll
    for (uint32_t i = 0; i < kLoop && i < n; i++) eq += key(i) == prefix;
    // exclusive prefix of eq over the threads: a scan in each wave, then the wave totals
    uint32_t inc = eq;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if ((tid & 63) >= (uint32_t)o) inc += v;
    }
    if ((tid & 63) == 63) cnt[tid >> 6] = inc;
    __syncthreads();
    uint32_t before = inc - eq;
    for (uint32_t w = 0; w < (tid >> 6); w++) before += cnt[w];
    uint32_t mine = 0, kept = 0;  // kept: bit i = key i kept (cached path)
#pragma unroll
    for (uint32_t i = 0; i < kLoop && i < n; i++) {
        const uint32_t u = key(i);
        uint8_t k = u > prefix;
        if (u == prefix) {
            k = before < kk;
            before++;
        }
        keep[t0 + i] = k;
        mine += k;
        if (CACHED) kept |= (uint32_t)k << i;
    }
    // the list: exclusive prefix of the kept counts, as above
    __syncthreads();  // cnt is free again
    inc = mine;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if ((tid & 63) >= (uint32_t)o) inc += v;
    }
    if ((tid & 63) == 63) cnt[tid >> 6] = inc;
    __syncthreads();
    uint32_t at = inc - mine;
    for (uint32_t w = 0; w < (tid >> 6); w++) at += cnt[w];
#pragma unroll
    for (uint32_t i = 0; i < kLoop && i < n; i++)
        if (CACHED ? ((kept >> i) & 1u) : keep[t0 + i]) klist[at++] = t0 + i;
    if (tid == 0) klist[max_seq] = K;
}

__global__ __launch_bounds__(1024) void index_topk_kernel(const float* isc, uint8_t* keep, uint32_t* klist,
                                                          uint32_t max_seq, uint32_t T, uint32_t K) {
    const uint32_t tid = threadIdx.x;
    if (T <= K) {
        for (uint32_t t = tid; t < T; t += 1024) {
            keep[t] = 1;
            klist[t] = t;
        }
        if (tid == 0) klist[max_seq] = T;
        return;
    }
    if ((T + 1023) / 1024 <= kTopkCache) index_topk_body<true>(isc, keep, klist, max_seq, T, K);
    else index_topk_body<false>(isc, keep, klist, max_seq, T, K);
}

// Attention over the kept keys klist[sp kps, min(count, (sp + 1) kps)) (the
// selection in ascending key order, count = klist[max_seq]) for heads
// [hg 16, hg 16 + 16) (all heads when fewer), 32 keys at a time, on the
// matrix cores (v_mfma_f32_16x16x4_f32: f32 products and sums). LDS rows of
// W16 = W rounded up to 16 floats (zero past W) at a stride of W16 + 4 floats
// (an odd number of 16-byte groups, so the 16 rows an MFMA operand reads sit
// in different banks): the queries qa [16][.] and the chunk's rows kv [32][.]
// (kv_c | k_rot of each key, zero rows past the chunk).
//   scores  S[16 heads][32 keys]: wave w takes key tile w & 1 and the 16-float
//           column blocks b = (w >> 1) + 4i; lane (n, g) reads floats
//           [16 b + 4 g, +4) of query row n and of key row n of the tile (one
//           16-byte read each) and feeds them to 4 MFMAs (k index g), so the
//           4 partial tiles of a key tile sum to the full dot products;
//   softmax online per head (running max, sum and rescale of the context);
//   context C[16 heads][L] += P[16][32] V[32][L]: wave w owns column tiles
//           w + 8 i, 8 MFMAs (4 keys each) per tile per chunk.
// The split's max, sum and unnormalised context go to its slots.
constexpr uint32_t kHG = 16;
constexpr uint32_t kKeys = 32;
constexpr uint32_t kSplitThreads = 512;
constexpr uint32_t kCT = 4;  // context column tiles per wave: L <= 512 = 8 waves x 4 x 16
// float4 elements per thread of the query block (16 x W16/4) and of a chunk
// (32 x W16/4), W <= 768
constexpr uint32_t kQE = 6, kKE = 12;

WL_DEV f32x4 mma_f32(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
// Max / sum over each 32-lane half of the wave, in every lane of the half:
// DPP within the 16-lane rows (pairs at xor 1 and 2, then the mirrored
// 8-lane halves and rows), one permute across the two rows of the half.
template <int CTRL>
WL_DEV float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, 0xF, 0xF, false));
}
WL_DEV float half_max(float x) {
    x = fmaxf(x, dpp<0xB1>(x));   // quad_perm [1,0,3,2]
    x = fmaxf(x, dpp<0x4E>(x));   // quad_perm [2,3,0,1]
    x = fmaxf(x, dpp<0x141>(x));  // row_half_mirror
    x = fmaxf(x, dpp<0x140>(x));  // row_mirror
    return fmaxf(x, __shfl_xor(x, 16, 32));
}
WL_DEV float half_sum(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return x + __shfl_xor(x, 16, 32);
}

__global__ __launch_bounds__(kSplitThreads) void attn_split_kernel(Shape s, AttnPtrs p) {
    extern __shared__ __align__(16) float lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t HG = s.HN < kHG ? s.HN : kHG;
    const uint32_t NHG = s.HN / HG;
    // work-group b runs on XCD b % 8: the head groups of split sp all run on
    // XCD sp % 8, so the chunk rows one of them fetches serve the others from
    // that XCD's L2 (the grid is NHG x the splits rounded up to 8)
    const uint32_t xcd = blockIdx.x % 8u, slot = blockIdx.x / 8u;
    const uint32_t hg = slot % NHG, sp = xcd + 8u * (slot / NHG);
    if (sp >= p.nsplit) return;  // the grid's rounding: no split, no slots (the whole work-group)
    const uint32_t L = s.L, RP = s.RP, W = L + RP, W16 = (W + 15u) & ~15u, KS = W16 + 4u;
    const uint32_t NCT = (L + 15u) / 16u;
    float* qa = lds;                // [kHG][KS]
    float* kv = qa + kHG * KS;      // [kKeys][KS]
    float* st = kv + kKeys * KS;    // [8 waves][16 x 16] partial score tiles
    float* ps = st + 8u * 256u;     // [kKeys][kHG] scores, then probabilities
    float* al = ps + kKeys * kHG;   // [kHG] rescale of this chunk
    float* mx = al + kHG;           // [kHG] running max
    float* sm = mx + kHG;           // [kHG] running sum
    // every load of the queries and of a chunk is issued before any is
    // stored, branch-free (an element outside the data loads from a valid
    // address and is zeroed after), so they are all in flight together
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 qv[kQE];
    uint32_t qok = 0;  // bit i: element i is inside the queries (the zeroing waits for the store)
    {
        Walk2 w(tid, kSplitThreads, W16 / 4);
#pragma unroll
        for (uint32_t i = 0; i < kQE; i++) {
            const uint32_t h = w.r, c = 4 * w.c;
            const bool ok = h < HG && c < W;
            const float* src = c < L ? p.q_abs + (size_t)(hg * HG + h) * L + c
                                     : p.q_rope + (size_t)(hg * HG + h) * RP + (c - L);
            qv[i] = *(const f32x4*)(ok ? src : p.q_abs);
            qok |= (ok ? 1u : 0u) << i;
            w.next();
        }
    }
    if (tid < kHG) {
        mx[tid] = -INFINITY;
        sm[tid] = 0.f;
    }
    f32x4 acc[kCT];
#pragma unroll
    for (uint32_t i = 0; i < kCT; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t k0 = sp * p.kps, k1 = (k0 + p.kps < p.count) ? k0 + p.kps : p.count;
    const uint32_t tile = wv & 1u, kq = wv >> 1;
    const Walk2 w0(tid, kSplitThreads, W16 / 4);
    // the key of each element of chunk kb (the list, or the position itself
    // when every key is kept; past the chunk's keys: 0)
    uint32_t key[kKE];
    auto load_keys = [&](uint32_t kb, uint32_t nk) {
        const rsrc_t kl = make_rsrc(p.klist + kb, 4u * nk);
        Walk2 w = w0;
#pragma unroll
        for (uint32_t i = 0; i < kKE; i++) {
            key[i] = p.ident ? kb + w.r : __builtin_amdgcn_raw_buffer_load_b32(kl, (int)(4u * w.r), 0, 0);
            w.next();
        }
    };
    // the first chunk's keys are in flight with the queries; the queries go
    // to LDS while they arrive (qa is not read before the first barrier)
    if (k0 < k1) load_keys(k0, (k1 - k0) < kKeys ? (k1 - k0) : kKeys);
    {
        Walk2 wq(tid, kSplitThreads, W16 / 4);
#pragma unroll
        for (uint32_t i = 0; i < kQE; i++) {
            if (wq.r < kHG) *(f32x4*)(qa + wq.r * KS + 4 * wq.c) = ((qok >> i) & 1u) ? qv[i] : z4;
            wq.next();
        }
    }
    for (uint32_t kb = k0; kb < k1; kb += kKeys) {
        const uint32_t nk = (k1 - kb) < kKeys ? (k1 - kb) : kKeys;
        {
            f32x4 v[kKE];
            if (kb != k0) load_keys(kb, nk);
            Walk2 w = w0;
#pragma unroll
            for (uint32_t i = 0; i < kKE; i++) {
                const uint32_t r = w.r, c = 4 * w.c;
                const bool ok = r < nk && c < W;
                const uint32_t k = ok ? key[i] : 0u;
                const float* src = c < L ? p.kv_c + (size_t)k * L + c : p.k_rot + (size_t)k * RP + (c - L);
                const f32x4 x = *(const f32x4*)(ok ? src : p.kv_c);
                v[i] = ok ? x : z4;
                w.next();
            }
            __syncthreads();  // the previous chunk's rows and probabilities are read
            w = w0;
#pragma unroll
            for (uint32_t i = 0; i < kKE; i++) {
                if (w.r < kKeys) *(f32x4*)(kv + w.r * KS + 4 * w.c) = v[i];
                w.next();
            }
        }
        __syncthreads();
        {
            // two accumulators (even / odd column blocks), so consecutive
            // MFMAs do not wait on each other
            f32x4 t0 = {0.f, 0.f, 0.f, 0.f}, t1 = t0;
            const float* qrow = qa + n * KS + 4u * g;
            const float* krow = kv + (16u * tile + n) * KS + 4u * g;
            const uint32_t NB = W16 / 16u;
            uint32_t b = kq;
            for (; b + 4u < NB; b += 8u) {
                const f32x4 x0 = *(const f32x4*)(qrow + 16u * b), y0 = *(const f32x4*)(krow + 16u * b);
                const f32x4 x1 = *(const f32x4*)(qrow + 16u * (b + 4u)), y1 = *(const f32x4*)(krow + 16u * (b + 4u));
#pragma unroll
                for (uint32_t i = 0; i < 4; i++) {
                    t0 = mma_f32(x0[i], y0[i], t0);
                    t1 = mma_f32(x1[i], y1[i], t1);
                }
            }
            if (b < NB) {
                const f32x4 x0 = *(const f32x4*)(qrow + 16u * b), y0 = *(const f32x4*)(krow + 16u * b);
#pragma unroll
                for (uint32_t i = 0; i < 4; i++) t0 = mma_f32(x0[i], y0[i], t0);
            }
            // lane (n, g) holds S[head 4 g + j][key 16 tile + n]
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) st[wv * 256u + (4u * g + j) * 16u + n] = t0[j] + t1[j];
        }
        __syncthreads();
        // the four column-block partials (in block order), then the online
        // softmax: two heads per wave, one per 32-lane half, lanes over the keys
        {
            const uint32_t h = wv + 8u * (lane >> 5), key = lane & 31u, t = key >> 4;
            const uint32_t idx = h * 16u + (key & 15u);
            float v = ((st[t * 256u + idx] + st[(2u + t) * 256u + idx]) + st[(4u + t) * 256u + idx]) +
                      st[(6u + t) * 256u + idx];
            v = key < nk ? v * p.qk_scale : -INFINITY;
            const float m = half_max(v);
            const float mo = mx[h];
            const float mn = fmaxf(mo, m);
            const float e = v != -INFINITY ? expf(v - mn) : 0.f;
            const float z = half_sum(e);
            ps[key * kHG + h] = e;
            // head h is this half-wave's alone; its LDS reads of mx[h] above
            // precede the write below in the wave's program order
            if (key == 0 && h < HG) {
                const float a = (mo == -INFINITY) ? 0.f : expf(mo - mn);
                const float r = (mn == -INFINITY) ? 1.f : a;
                al[h] = r;
                mx[h] = mn;
                sm[h] = sm[h] * r + z;
            }
        }
        __syncthreads();
        float r[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) r[j] = (4u * g + j < HG) ? al[4u * g + j] : 0.f;
#pragma unroll
        for (uint32_t i = 0; i < kCT; i++) {
            const uint32_t ct = wv + 8u * i;
            if (ct < NCT) {
#pragma unroll
                for (uint32_t j = 0; j < 4; j++) acc[i][j] *= r[j];
#pragma unroll
                for (uint32_t kk = 0; kk < kKeys / 4u; kk++)
                    acc[i] = mma_f32(ps[(4u * kk + g) * kHG + n], kv[(4u * kk + g) * KS + 16u * ct + n], acc[i]);
            }
        }
    }
    __syncthreads();
    const uint32_t hb = hg * HG;
    if (tid < HG) {
        p.part_m[(size_t)sp * s.HN + hb + tid] = mx[tid];
        p.part_l[(size_t)sp * s.HN + hb + tid] = sm[tid];
    }
#pragma unroll
    for (uint32_t i = 0; i < kCT; i++) {
        const uint32_t ct = wv + 8u * i, col = 16u * ct + n;
        if (ct < NCT && col < L) {
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t h = 4u * g + j;
                if (h < HG) p.part_ctx[((size_t)sp * s.HN + hb + h) * L + col] = acc[i][j];
            }
        }
    }
}

// ctx[h] = sum_s e^(m_s - M) ctx_s[h] / sum_s e^(m_s - M) l_s, M = max_s m_s:
// work-group (head, 64 columns); thread (column c, quarter q) sums the splits
// q, q + 4, ... (all of its loads issued together, beside the split weights'
// loads; S <= 64), and the four quarter sums of a column are added in order.
constexpr uint32_t kCombCols = 64;
__global__ __launch_bounds__(256) void attn_combine_kernel(Shape s, AttnPtrs p, uint32_t S) {
    __shared__ float w[64];
    __shared__ float red[4][kCombCols];
    __shared__ float zz;
    const uint32_t nb = (s.L + kCombCols - 1) / kCombCols;
    const uint32_t h = blockIdx.x / nb, tid = threadIdx.x, cq = tid % kCombCols, q = tid / kCombCols;
    const uint32_t c = (blockIdx.x % nb) * kCombCols + cq;
    const bool col_ok = c < s.L;
    float v[16];
    const float* src = p.part_ctx + (size_t)h * s.L + (col_ok ? c : 0u);
#pragma unroll
    for (uint32_t i = 0; i < 16; i++) {
        const uint32_t sp = q + 4u * i;
        v[i] = sp < S ? src[(size_t)sp * s.HN * s.L] : 0.f;
    }
    if (tid < 64) {
        const float m = tid < S ? p.part_m[(size_t)tid * s.HN + h] : -INFINITY;
        float M = m;
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        const float e = (m == -INFINITY) ? 0.f : expf(m - M);
        w[tid] = e;
        float z = tid < S ? e * p.part_l[(size_t)tid * s.HN + h] : 0.f;
        for (int o = 32; o > 0; o >>= 1) z += __shfl_xor(z, o, 64);
        if (tid == 0) zz = z;
    }
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < 16; i++) t += w[(q + 4u * i) & 63u] * v[i];
    red[q][cq] = t;
    __syncthreads();
    if (q == 0 && col_ok) p.ctx[(size_t)h * s.L + c] = (((red[0][cq] + red[1][cq]) + red[2][cq]) + red[3][cq]) / zz;
}

}  // namespace

#ifndef WL_GEMV_TPR_MIN
#define WL_GEMV_TPR_MIN 32
#endif
// Threads per row: the fewest (from WL_GEMV_TPR_MIN; at most one wave, so the
// sums need no barrier) whose chunk iterations fit the kMaxIt input
// registers, then doubled while the launch would have fewer than 512
// work-groups (small matrices: more, shorter work-groups spread the rows over
// the chip); never more than the row has chunks. Measured on MI355X (µs,
// wl_matvec_bf16): 16384 x 512 7.2 at 32 threads per row (9.2 at 64),
// 16384 x 2048 17.0 at 32 (18.4 at 64, 2.4 TB/s at 256), 2048 x 6144 2.7 TB/s
// at 128 (2.4 at 64); a minimum of 8 or 16 ends at the same 32 for these.
uint32_t gemv_plan(GemvJob& j) {
    const uint32_t nch = j.K / 8;
    uint32_t l2 = 0;
    while ((1u << (l2 + 1)) <= nch && (1u << (l2 + 1)) <= WL_GEMV_TPR_MIN) l2++;
    while ((nch + (1u << l2) - 1) >> l2 > (uint32_t)kMaxIt && (1u << l2) < kGemvThreads) l2++;
    auto wgs = [&](uint32_t t2) {
        const uint32_t rows = kGemvRows * (kGemvThreads >> t2);
        return (j.N + rows - 1) / rows;
    };
    while (wgs(l2) < 512 && (1u << (l2 + 1)) <= nch && (1u << l2) < kGemvThreads) l2++;
    j.tpr_log2 = l2;
    j.rows_wg = kGemvRows * (kGemvThreads >> l2);
    return (j.N + j.rows_wg - 1) / j.rows_wg;
}

#ifndef WL_SG_WGS
#define WL_SG_WGS 512
#endif
constexpr uint32_t kSgTarget = WL_SG_WGS;  // work-groups of a streaming launch (two per CU at the GLM shapes)
constexpr size_t kSgMaxLds = 160u * 1024u;  // dynamic LDS

// Rows shorter than this run on the row-group kernel (measured on MI355X,
// 16384 x 512: 7.2 us there against 7.6 for the streaming kernel, whose
// staging of the input is one more round trip before the first product).
constexpr uint32_t kSgMinK = 1024;
// Streaming plan of l: every job's work-groups (in proportion to its weight
// bytes, at least one, at most one per row) and the launch's dynamic LDS.
// Returns the work-group count, 0 when a job does not fit the kernel (an x2
// input, an LDS or resource size past its limits).
uint32_t sgemv_plan(GemvLaunch& l, size_t& lds, uint32_t target, uint32_t nw) {
    double total = 0;
    for (uint32_t i = 0; i < l.n_jobs; i++) {
        const GemvJob& j = l.job[i];
        const uint32_t epu = j.f32w ? 256u : 512u;
        total += (double)j.N * (j.W2 ? 2 : 1) * ((j.K + epu - 1) / epu);
    }
    uint32_t wg = 0;
    lds = 0;
    for (uint32_t i = 0; i < l.n_jobs; i++) {
        GemvJob& j = l.job[i];
        if (j.x2 || (j.W2 && (j.f32w || j.GS))) return 0;
        if (!j.W2 && j.K < kSgMinK) return 0;
        const uint32_t esz = j.f32w ? 4u : 2u, epu = 1024u / esz, nL = (j.K + epu - 1) / epu, Kp = nL * epu;
        const double units = (double)j.N * (j.W2 ? 2 : 1) * nL;
        uint32_t nwg = (uint32_t)(target * units / total + 0.5);
        nwg = nwg < 1u ? 1u : nwg > j.N ? j.N : nwg;
        const uint32_t R = (j.N + nwg - 1) / nwg;
        const uint32_t ng = j.GS ? std::min((j.N + j.G - 1) / j.G, (R + j.G - 1) / j.G + 1u) : 1u;
        if (j.norm_w && j.GS) return 0;
        const size_t need = (size_t)ng * Kp * 4 + (j.norm_w ? (size_t)(Kp + 511) / 512 * 1024 : 0) +
                            (size_t)(j.W2 ? 2 : 1) * R * nw * 4 + nw * 4;
        const uint64_t span = (uint64_t)(j.GS ? ng * j.GS : R) * j.K * esz;
        if (need > kSgMaxLds || span >= (1ull << 31) || (uint64_t)((ng - 1) * j.XS + j.K) * 4 >= (1ull << 31)) return 0;
        lds = std::max(lds, need);
        j.wg0 = wg;
        j.nwg = nwg;
        wg += nwg;
    }
    return wg;
}

int launch_sgemv(const GemvLaunch& l0, uint32_t n_wg, const Shape* s, const AttnPtrs* p, uint32_t pos,
                 uint32_t n_prep, void* stream) {
    GemvLaunch l = l0;
    size_t lds = 0;
    const uint32_t ns = sgemv_plan(l, lds, kSgTarget, 4);
    if (ns == 0) {
        if (n_prep) {
            hipLaunchKernelGGL(gemv_prep_kernel, dim3(n_wg + n_prep), dim3(kGemvThreads), 0, (hipStream_t)stream, l0,
                               n_wg, *s, *p, pos);
        } else {
            hipLaunchKernelGGL(gemv_kernel, dim3(n_wg), dim3(kGemvThreads), 0, (hipStream_t)stream, l0);
        }
        return (int)hipGetLastError();
    }
    hipError_t ae = hipFuncSetAttribute((const void*)sgemv_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)kSgMaxLds);
    if (ae != hipSuccess) return (int)ae;
    const Shape s0{};
    const AttnPtrs p0{};
    if (n_prep) lds = std::max(lds, (size_t)kPrepLds * 4);
    hipLaunchKernelGGL(sgemv_kernel, dim3(ns + n_prep), dim3(256), lds, (hipStream_t)stream, l, ns, s ? *s : s0,
                       p ? *p : p0, pos);
    return (int)hipGetLastError();
}

int launch_gemv(const GemvLaunch& l, uint32_t n_wg, void* stream) {
    return launch_sgemv(l, n_wg, nullptr, nullptr, 0u, 0u, stream);
}

bool sgemv_fits(const GemvLaunch& l0) {
    GemvLaunch l = l0;
    size_t lds = 0;
    return sgemv_plan(l, lds, kSgTarget, 4) != 0;
}

// Dynamic LDS of the index scores: q [IH][ID + 4], w [IH], k [kIdxKeys][ID + 4], RoPE table [RP].
size_t index_score_lds(const Shape& s) {
    return ((size_t)s.IH * (s.ID + 4) + s.IH + (size_t)kIdxKeys * (s.ID + 4) + s.RP) * 4;
}

int launch_gemv_prep(const GemvLaunch& l, uint32_t n_wg, const Shape& s, const AttnPtrs& p, uint32_t pos, bool owner,
                     void* stream) {
    return launch_sgemv(l, n_wg, &s, &p, pos, owner ? 2u : 1u, stream);
}

int launch_attn_absorb(const Shape& s, const AttnPtrs& p, bool owner, uint32_t T, void* stream) {
    const uint32_t nb = (s.L + 127) / 128;
    const uint32_t nsc = owner ? (T + kIdxKeys - 1) / kIdxKeys : 0u;
    const size_t lds = owner ? index_score_lds(s) : 0;
    hipError_t ae = hipFuncSetAttribute((const void*)attn_absorb_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)lds);
    if (ae != hipSuccess) return (int)ae;
    hipLaunchKernelGGL(attn_absorb_kernel, dim3(s.HN * nb + 1 + nsc), dim3(256), lds, (hipStream_t)stream, s, p,
                       owner ? 1u : 0u, T);
    return (int)hipGetLastError();
}

int launch_index_topk(const Shape& s, const AttnPtrs& p, uint32_t T, void* stream) {
    hipLaunchKernelGGL(index_topk_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, (const float*)p.isc, p.keep,
                       p.klist, p.max_seq, T, s.TOPK);
    return (int)hipGetLastError();
}

// Splits of the kept keys (at most min(T, TOPK) of them): about 512
// work-groups, each split a multiple of 32 keys.
uint32_t attn_splits(const Shape& s, uint32_t T, uint32_t max_splits) {
    const uint32_t HG = s.HN < kHG ? s.HN : kHG;
    const uint32_t NHG = s.HN / HG;
    const uint32_t nk = T < s.TOPK ? T : s.TOPK;
    uint32_t S = (nk + kKeys - 1) / kKeys;
    const uint32_t want = (512 + NHG - 1) / NHG;
    if (S > want) S = want;
    if (S > max_splits) S = max_splits;
    if (S == 0) S = 1;
    return S;
}

size_t attn_split_lds(const Shape& s) {
    const size_t KS = ((s.L + s.RP + 15) & ~15u) + 4;
    return 4 * ((size_t)(kHG + kKeys) * KS + 8 * 256 + (size_t)kKeys * kHG + 3 * kHG);
}

int launch_attn_core(const Shape& s, const AttnPtrs& p0, uint32_t T, uint32_t splits, void* stream) {
    AttnPtrs p = p0;
    const uint32_t HG = s.HN < kHG ? s.HN : kHG;
    const uint32_t NHG = s.HN / HG;
    const uint32_t nk = T < s.TOPK ? T : s.TOPK;  // the selection's size
    uint32_t kps = (nk + splits - 1) / splits;
    kps = (kps + kKeys - 1) / kKeys * kKeys;
    const uint32_t S = (nk + kps - 1) / kps;  // every split holds at least one key
    p.kps = kps;
    p.count = nk;
    p.ident = T <= s.TOPK ? 1u : 0u;
    hipError_t ae = hipFuncSetAttribute((const void*)attn_split_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)attn_split_lds(s));
    if (ae != hipSuccess) return (int)ae;
    p.nsplit = S;
    hipLaunchKernelGGL(attn_split_kernel, dim3(NHG * ((S + 7u) / 8u) * 8u), dim3(kSplitThreads), attn_split_lds(s),
                       (hipStream_t)stream, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(s.HN * ((s.L + kCombCols - 1) / kCombCols)), dim3(256), 0,
                       (hipStream_t)stream, s, p, S);
    return (int)hipGetLastError();
}

}  // namespace attn
}  // namespace wl
