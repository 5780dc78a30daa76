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

__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvLaunch L) {
    __shared__ float red[(kGemvRows + 1) * 4];
    const uint32_t b = blockIdx.x;
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
    // the group's x (rows of one group share it: G % kGemvRows == 0)
    const float* x = j.x + (size_t)((r0 < j.N ? r0 : 0) / j.G) * j.XS;
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
    size_t roff[kGemvRows];
#pragma unroll
    for (int r = 0; r < (int)kGemvRows; r++) {
        acc[r] = 0.f;
        const uint32_t row = r0 + r;
        const uint32_t wr = (row / j.G) * j.GS + j.OFF + row % j.G;
        roff[r] = (size_t)wr * K;
    }
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
                    if (r0 + r < j.N) wv[r] = ld16_nt(W + roff[r] + 8 * c);
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

__global__ __launch_bounds__(256) void attn_prep_kernel(Shape s, AttnPtrs p, uint32_t pos) {
    __shared__ float red[4];
    __shared__ float kbuf[1024];
    __shared__ float cs[512];
    const uint32_t tid = threadIdx.x;
    rope_table(cs, s.RP, pos, s.theta);
    __syncthreads();
    if (blockIdx.x == 0)
        for (uint32_t i = tid; i < s.RP; i += 256) p.rope_cs[i] = cs[i];  // for the query RoPE
    if (blockIdx.x == 0) {
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

// q_abs[h][c] = sum_{d < NP} q[h][d] * kv_b[h (NP + VD) + d][c]: work-group
// (h, column block of up to 128 columns); 8 columns per thread, the rows
// split over the remaining thread dimension and summed through LDS. The last
// work-group applies RoPE to the queries.
__global__ __launch_bounds__(256) void attn_absorb_kernel(Shape s, AttnPtrs p, uint32_t owner) {
    __shared__ float red[2048];
    const uint32_t tid = threadIdx.x;
    const uint32_t nb = (s.L + 127) / 128;
    const uint32_t DH = s.NP + s.RP;
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
        for (uint32_t d = rlane; d < s.NP; d += rl) {
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

// isc[t] = sum_h w[h] * relu(q[h] . k[t] * ID^-0.5): 32 keys per work-group,
// 8 threads per key (each ID/8 dims, summed by shuffles), heads in order.
__global__ __launch_bounds__(256) void index_score_kernel(Shape s, AttnPtrs p, uint32_t T) {
    extern __shared__ float lq[];  // [IH][ID] then [IH]
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < s.IH * s.ID; i += 256) lq[i] = p.iqr[i];
    for (uint32_t i = tid; i < s.IH; i += 256) lq[s.IH * s.ID + i] = p.iw[i];
    __syncthreads();
    const uint32_t key = blockIdx.x * 32 + (tid >> 3), part = tid & 7, dp = s.ID / 8;
    const bool live = key < T;
    float k[32];
#pragma unroll
    for (uint32_t e = 0; e < 32; e++) k[e] = (live && e < dp) ? p.idx_k[(size_t)key * s.ID + part * dp + e] : 0.f;
    float sc = 0.f;
    for (uint32_t h = 0; h < s.IH; h++) {
        const float* qh = lq + (size_t)h * s.ID + part * dp;
        float d = 0.f;
#pragma unroll
        for (uint32_t e = 0; e < 32; e++)
            if (e < dp) d += qh[e] * k[e];
        d += __shfl_xor(d, 1, 64);
        d += __shfl_xor(d, 2, 64);
        d += __shfl_xor(d, 4, 64);
        sc += lq[s.IH * s.ID + h] * fmaxf(d * p.ix_scale, 0.f);
    }
    if (live && part == 0) p.isc[key] = sc;
}

// Order-preserving key of an f32 (larger float -> larger key).
WL_DEV uint32_t okey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// keep[t] = 1 for the TOPK largest scores of [0, T) (ties to the lowest
// index), every key when T <= TOPK. One work-group: a radix select of the
// TOPK-th largest key (4 passes of 8 bits), then the marking.
__global__ __launch_bounds__(1024) void index_topk_kernel(const float* isc, uint8_t* keep, uint32_t T, uint32_t K) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t cnt[1024];
    __shared__ uint32_t sh_prefix, sh_kk;
    const uint32_t tid = threadIdx.x;
    if (T <= K) {
        for (uint32_t t = tid; t < T; t += 1024) keep[t] = 1;
        return;
    }
    uint32_t prefix = 0, mask = 0, kk = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t i = tid; i < 256; i += 1024) hist[i] = 0;
        __syncthreads();
        for (uint32_t t = tid; t < T; t += 1024) {
            const uint32_t u = okey(isc[t]);
            if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t cum = 0;
            int d = 255;
            for (; d > 0; d--) {
                if (cum + hist[d] >= kk) break;
                cum += hist[d];
            }
            sh_prefix = prefix | ((uint32_t)d << shift);
            sh_kk = kk - cum;
        }
        __syncthreads();
        prefix = sh_prefix;
        kk = sh_kk;
        mask |= 255u << shift;
        __syncthreads();
    }
    // prefix: the key of the K-th largest score; kk (>= 1) of the keys equal
    // to it are kept, the lowest indices first
    const uint32_t per = (T + 1023) / 1024, t0 = tid * per, t1 = (t0 + per < T) ? t0 + per : T;
    uint32_t eq = 0;
    for (uint32_t t = t0; t < t1; t++) eq += okey(isc[t]) == prefix;
    cnt[tid] = eq;
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t i = 0; i < tid; i++) before += cnt[i];
    for (uint32_t t = t0; t < t1; t++) {
        const uint32_t u = okey(isc[t]);
        uint8_t k = u > prefix;
        if (u == prefix) {
            k = before < kk;
            before++;
        }
        keep[t] = k;
    }
}

// Attention over keys [s kps, min(T, (s + 1) kps)) for heads [hg HG, hg HG +
// HG): 32 keys at a time staged in LDS (kv_c | k_rot per row), scores for all
// heads, an online softmax, and the unnormalised context; partial max, sum
// and context go to the split's slots.
constexpr uint32_t kHG = 16;
constexpr uint32_t kKeys = 32;

__global__ __launch_bounds__(256) void attn_split_kernel(Shape s, AttnPtrs p, uint32_t T) {
    extern __shared__ float lds[];
    const uint32_t tid = threadIdx.x;
    const uint32_t HG = s.HN < kHG ? s.HN : kHG;
    const uint32_t NHG = s.HN / HG;
    const uint32_t hg = blockIdx.x % NHG, sp = blockIdx.x / NHG;
    const uint32_t L = s.L, RP = s.RP, KS = L + RP + 4;
    float* qa = lds;                      // [HG][L + RP]: q_abs | q_rope
    float* kv = qa + HG * (L + RP);       // [kKeys][KS]
    float* ps = kv + kKeys * KS;          // [HG][kKeys]
    float* al = ps + HG * kKeys;          // [HG] rescale of this step
    float* mx = al + HG;                  // [HG] running max
    float* sm = mx + HG;                  // [HG] running sum
    for (uint32_t i = tid; i < HG * L; i += 256) qa[(i / L) * (L + RP) + i % L] = p.q_abs[(size_t)(hg * HG) * L + i];
    for (uint32_t i = tid; i < HG * RP; i += 256) qa[(i / RP) * (L + RP) + L + i % RP] = p.q_rope[(size_t)(hg * HG) * RP + i];
    if (tid < HG) {
        mx[tid] = -INFINITY;
        sm[tid] = 0.f;
    }
    // context accumulators: thread -> 8 columns x up to 4 heads
    const uint32_t tph = L / 8, rp = 256 / tph;  // threads per head row, head rows per pass
    const uint32_t cc = (tid % tph) * 8, hr = tid / tph;
    float acc[4][8];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[a][e] = 0.f;
    const uint32_t k0 = sp * p.kps, k1 = (k0 + p.kps < T) ? k0 + p.kps : T;
    for (uint32_t kb = k0; kb < k1; kb += kKeys) {
        const uint32_t nk = (k1 - kb) < kKeys ? (k1 - kb) : kKeys;
        __syncthreads();
        for (uint32_t i = tid; i < nk * (L / 4); i += 256) {
            const uint32_t r = i / (L / 4), c = i % (L / 4);
            *(f32x4*)(kv + r * KS + 4 * c) = *(const f32x4*)(p.kv_c + (size_t)(kb + r) * L + 4 * c);
        }
        for (uint32_t i = tid; i < nk * RP; i += 256) {
            const uint32_t r = i / RP, c = i % RP;
            kv[r * KS + L + c] = p.k_rot[(size_t)(kb + r) * RP + c];
        }
        __syncthreads();
        // scores: dot (h, key) for HG x kKeys pairs, two per thread
        for (uint32_t d = tid; d < HG * kKeys; d += 256) {
            const uint32_t h = d / kKeys, key = d % kKeys;
            float v = -INFINITY;
            if (key < nk && (!p.keep || p.keep[kb + key])) {
                const float* a = qa + h * (L + RP);
                const float* b = kv + key * KS;
                float t = 0.f;
                for (uint32_t c = 0; c < L + RP; c += 4) {
                    const f32x4 x = *(const f32x4*)(a + c), y = *(const f32x4*)(b + c);
                    t += x[0] * y[0];
                    t += x[1] * y[1];
                    t += x[2] * y[2];
                    t += x[3] * y[3];
                }
                v = t * p.qk_scale;
            }
            ps[h * kKeys + key] = v;
        }
        __syncthreads();
        // online softmax: one wave per head at a time
        for (uint32_t h = tid >> 6; h < HG; h += 4) {
            const uint32_t ln = tid & 63;
            const float v = ln < kKeys ? ps[h * kKeys + ln] : -INFINITY;
            float m = v;
            for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
            const float mo = mx[h];
            const float mn = fmaxf(mo, m);
            const float e = (ln < kKeys && v != -INFINITY) ? expf(v - mn) : 0.f;
            float z = e;
            for (int o = 32; o > 0; o >>= 1) z += __shfl_xor(z, o, 64);
            const float a = (mo == -INFINITY) ? 0.f : expf(mo - mn);
            if (ln < kKeys) ps[h * kKeys + ln] = e;
            if (ln == 0) {
                al[h] = (mn == -INFINITY) ? 1.f : a;
                mx[h] = mn;
                sm[h] = sm[h] * ((mn == -INFINITY) ? 1.f : a) + z;
            }
        }
        __syncthreads();
        // context: acc[h][c] = acc * alpha[h] + sum_key p[h][key] kv_c[key][c]
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint32_t h = hr + a * rp;
            if (h < HG) {
                const float sc = al[h];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[a][e] *= sc;
                for (uint32_t key = 0; key < nk; key++) {
                    const float w = ps[h * kKeys + key];
                    const f32x4 x = *(const f32x4*)(kv + key * KS + cc), y = *(const f32x4*)(kv + key * KS + cc + 4);
                    acc[a][0] += w * x[0];
                    acc[a][1] += w * x[1];
                    acc[a][2] += w * x[2];
                    acc[a][3] += w * x[3];
                    acc[a][4] += w * y[0];
                    acc[a][5] += w * y[1];
                    acc[a][6] += w * y[2];
                    acc[a][7] += w * y[3];
                }
            }
        }
    }
    __syncthreads();
    const uint32_t h0 = hg * HG;
    if (tid < HG) {
        p.part_m[(size_t)sp * s.HN + h0 + tid] = mx[tid];
        p.part_l[(size_t)sp * s.HN + h0 + tid] = sm[tid];
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint32_t h = hr + a * rp;
        if (h < HG) {
            float* o = p.part_ctx + ((size_t)sp * s.HN + h0 + h) * L + cc;
            *(f32x4*)o = f32x4{acc[a][0], acc[a][1], acc[a][2], acc[a][3]};
            *(f32x4*)(o + 4) = f32x4{acc[a][4], acc[a][5], acc[a][6], acc[a][7]};
        }
    }
}

// ctx[h] = sum_s e^(m_s - M) ctx_s[h] / sum_s e^(m_s - M) l_s, M = max_s m_s.
__global__ __launch_bounds__(256) void attn_combine_kernel(Shape s, AttnPtrs p, uint32_t S) {
    const uint32_t h = blockIdx.x;
    float M = -INFINITY;
    for (uint32_t i = 0; i < S; i++) M = fmaxf(M, p.part_m[(size_t)i * s.HN + h]);
    float z = 0.f;
    for (uint32_t i = 0; i < S; i++) {
        const float m = p.part_m[(size_t)i * s.HN + h];
        if (m != -INFINITY) z += expf(m - M) * p.part_l[(size_t)i * s.HN + h];
    }
    const float inv = 1.0f / z;
    for (uint32_t c = threadIdx.x; c < s.L; c += 256) {
        float t = 0.f;
        for (uint32_t i = 0; i < S; i++) {
            const float m = p.part_m[(size_t)i * s.HN + h];
            if (m != -INFINITY) t += expf(m - M) * p.part_ctx[((size_t)i * s.HN + h) * s.L + c];
        }
        p.ctx[(size_t)h * s.L + c] = t * inv;
    }
}

}  // namespace

uint32_t gemv_plan(GemvJob& j) {
    const uint32_t nch = j.K / 8;
    uint32_t l2 = 0;
    while ((1u << (l2 + 1)) <= nch && (1u << (l2 + 1)) <= kGemvThreads) l2++;
    j.tpr_log2 = l2;
    j.rows_wg = kGemvRows * (kGemvThreads >> l2);
    return (j.N + j.rows_wg - 1) / j.rows_wg;
}

int launch_gemv(const GemvLaunch& l, uint32_t n_wg, void* stream) {
    hipLaunchKernelGGL(gemv_kernel, dim3(n_wg), dim3(kGemvThreads), 0, (hipStream_t)stream, l);
    return (int)hipGetLastError();
}

int launch_attn_prep(const Shape& s, const AttnPtrs& p, uint32_t pos, bool owner, void* stream) {
    hipLaunchKernelGGL(attn_prep_kernel, dim3(owner ? 2 : 1), dim3(256), 0, (hipStream_t)stream, s, p, pos);
    return (int)hipGetLastError();
}

int launch_attn_absorb(const Shape& s, const AttnPtrs& p, uint32_t pos, bool owner, void* stream) {
    const uint32_t nb = (s.L + 127) / 128;
    (void)pos;
    hipLaunchKernelGGL(attn_absorb_kernel, dim3(s.HN * nb + 1), dim3(256), 0, (hipStream_t)stream, s, p,
                       owner ? 1u : 0u);
    return (int)hipGetLastError();
}

int launch_index_select(const Shape& s, const AttnPtrs& p, uint32_t T, void* stream) {
    const size_t lds = ((size_t)s.IH * s.ID + s.IH) * 4;
    hipError_t ae = hipFuncSetAttribute((const void*)index_score_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)lds);
    if (ae != hipSuccess) return (int)ae;
    hipLaunchKernelGGL(index_score_kernel, dim3((T + 31) / 32), dim3(256), lds, (hipStream_t)stream, s, p, T);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(index_topk_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, (const float*)p.isc, p.keep, T,
                       s.TOPK);
    return (int)hipGetLastError();
}

uint32_t attn_splits(const Shape& s, uint32_t T, uint32_t max_splits) {
    const uint32_t HG = s.HN < kHG ? s.HN : kHG;
    const uint32_t NHG = s.HN / HG;
    uint32_t S = (T + kKeys - 1) / kKeys;
    const uint32_t want = (512 + NHG - 1) / NHG;
    if (S > want) S = want;
    if (S > max_splits) S = max_splits;
    if (S == 0) S = 1;
    return S;
}

size_t attn_split_lds(const Shape& s) {
    const uint32_t HG = s.HN < kHG ? s.HN : kHG;
    return 4 * ((size_t)HG * (s.L + s.RP) + (size_t)kKeys * (s.L + s.RP + 4) + (size_t)HG * kKeys + 3 * HG);
}

int launch_attn_core(const Shape& s, const AttnPtrs& p0, uint32_t T, uint32_t splits, void* stream) {
    AttnPtrs p = p0;
    const uint32_t HG = s.HN < kHG ? s.HN : kHG;
    const uint32_t NHG = s.HN / HG;
    uint32_t kps = (T + splits - 1) / splits;
    kps = (kps + kKeys - 1) / kKeys * kKeys;
    const uint32_t S = (T + kps - 1) / kps;  // every split holds at least one key
    p.kps = kps;
    hipError_t ae = hipFuncSetAttribute((const void*)attn_split_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)attn_split_lds(s));
    if (ae != hipSuccess) return (int)ae;
    hipLaunchKernelGGL(attn_split_kernel, dim3(NHG * S), dim3(256), attn_split_lds(s), (hipStream_t)stream, s, p, T);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(s.HN), dim3(256), 0, (hipStream_t)stream, s, p, S);
    return (int)hipGetLastError();
}

}  // namespace attn
}  // namespace wl
