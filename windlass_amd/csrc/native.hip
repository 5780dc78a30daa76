// native.hip — conversion of expert blocks and shared experts into the decode
// kernel's HBM layout (NativeLayout / NativeShared in internal.h).
//
// Expert blocks: a work-group stages whole reference rows in LDS with
// coalesced 16-byte loads and writes whole 1 KB native chunks, in three roles
// (gate/up tile x 16 k tiles, down row group x 32 slices, down scales). With
// a null source the bytes come from the synthetic-weight generator (synth.hip)
// at the reference position they would have been copied from, so a synthetic
// block can be written in the native layout directly. One launch converts up
// to kConvMax blocks (blockIdx.y).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"

namespace wl {

// The six regions of a reference-layout expert (gate_w, gate_s, up_w, up_s,
// down_w, down_s): one pointer each (a packed block's regions, or six
// separate tensors), or all null: synthesise from `key`.
struct RefBlock {
    const uint8_t* src[6];
    uint32_t salt[6];
    uint32_t key;
};
constexpr uint32_t kConvMax = 16;
struct ConvBatch {
    RefBlock b[kConvMax];
    uint8_t* dst[kConvMax];
};

// 16 weight bytes at byte j (a multiple of 16) of region r.
__device__ static inline uint4 ref16(const RefBlock& b, int r, uint64_t j) {
    if (b.src[r]) return *(const uint4*)(b.src[r] + j);
    const uint32_t w0 = (uint32_t)(j / 4);
    uint4 v;
    v.x = mix32(mix32((w0 + 0) ^ b.salt[r]) ^ b.key);
    v.y = mix32(mix32((w0 + 1) ^ b.salt[r]) ^ b.key);
    v.z = mix32(mix32((w0 + 2) ^ b.salt[r]) ^ b.key);
    v.w = mix32(mix32((w0 + 3) ^ b.salt[r]) ^ b.key);
    return v;
}
// 4 weight bytes at byte j (a multiple of 4) of region r.
__device__ static inline uint32_t ref4(const RefBlock& b, int r, uint64_t j) {
    if (b.src[r]) return *(const uint32_t*)(b.src[r] + j);
    return mix32(mix32((uint32_t)(j / 4) ^ b.salt[r]) ^ b.key);
}
// Scale byte j of region r.
__device__ static inline uint32_t ref1(const RefBlock& b, int r, uint64_t j) {
    if (b.src[r]) return b.src[r][j];
    return 118u + mix32(mix32((uint32_t)j ^ b.salt[r]) ^ b.key) % 9u;
}
// Scale bytes j .. j + 3 (j a multiple of 4) of region r.
__device__ static inline uint32_t ref4s(const RefBlock& b, int r, uint64_t j) {
    if (b.src[r]) return *(const uint32_t*)(b.src[r] + j);
    return ref1(b, r, j) | ref1(b, r, j + 1) << 8 | ref1(b, r, j + 2) << 16 | ref1(b, r, j + 3) << 24;
}

constexpr uint32_t kConvThreads = 256;
constexpr uint32_t kRowPad = 1040;  // LDS stride of a staged 1 KB row (16 B of padding: no bank conflicts)
constexpr uint32_t kScPad = 68;     // LDS stride of a staged row of 64 scale bytes
constexpr uint32_t kConvLds = 512 * kScPad;  // the largest role (down scales, 512 rows)
static_assert(kConvLds >= 32 * kRowPad && kConvLds >= 16 * kRowPad + 16 * kScPad && kConvLds >= 64 * 260,
              "conversion LDS");

// Work items per block: role A = gate/up tile T x 16 k tiles (cc), role B =
// 32 down rows (q) x 32 slices (jb), role C = 512 down rows (cc) x 32 slices,
// role D = bgus (slice group, wave) x 32 steps, role E = bdns (row block,
// wave) x 32 steps.
struct ConvGrid {
    uint32_t nkt, ncca, nq, nccc, nj, njb, nsg, nstu, nrb, nstd, nA, nB, nC, nD, nE;
    __host__ __device__ static ConvGrid make(uint32_t H, uint32_t I) {
        ConvGrid g;
        g.nkt = H / 128;
        g.ncca = (g.nkt + 15) / 16;
        g.nq = H / 32;
        g.nccc = (g.nq + 15) / 16;
        g.nj = I / 64;
        g.njb = (g.nj + 31) / 32;
        g.nsg = (I + 255) / 256;
        g.nstu = (H + 255) / 256;
        g.nrb = (H + 511) / 512;
        g.nstd = (I + 255) / 256;
        g.nA = (I / 8) * g.ncca;
        g.nB = g.nq * g.njb;
        g.nC = g.nccc * g.njb;
        g.nD = g.nsg * 8 * ((g.nstu + 31) / 32);
        g.nE = g.nrb * 8 * ((g.nstd + 31) / 32);
        return g;
    }
};
constexpr uint32_t kBPad = 260;  // LDS stride of a staged row of 256 scale bytes

__global__ void __launch_bounds__(kConvThreads) to_native_kernel(const ConvBatch cb, uint32_t H, uint32_t I) {
    const RefBlock& b = cb.b[blockIdx.y];
    uint8_t* __restrict__ dst = cb.dst[blockIdx.y];
    const NativeLayout L = NativeLayout::make(H, I);
    const ConvGrid G = ConvGrid::make(H, I);
    __shared__ __align__(16) uint8_t lds[kConvLds];
    const uint32_t tid = threadIdx.x;
    uint32_t w = blockIdx.x;
    if (w < G.nA) {
        // gu chunks (T, kt) for 16 k tiles, and their gus chunk (T, cc):
        // LDS row n = gate row 8T + n (n < 8) or up row 8T + n - 8
        const uint32_t T = w / G.ncca, cc = w % G.ncca, nk = min(16u, G.nkt - 16u * cc);
        uint8_t* sc = lds + 16 * kRowPad;
        for (uint32_t u = tid; u < 16u * 4u * nk; u += kConvThreads) {
            const uint32_t r = u / (4u * nk), c = u % (4u * nk), row = 8u * T + (r & 7u);
            *(uint4*)(lds + r * kRowPad + 16u * c) =
                ref16(b, r < 8 ? 0 : 2, (uint64_t)row * (H / 2) + 1024u * cc + 16u * c);
        }
        for (uint32_t u = tid; u < 16u * nk; u += kConvThreads) {
            const uint32_t r = u / nk, c = u % nk, row = 8u * T + (r & 7u);
            *(uint32_t*)(sc + r * kScPad + 4u * c) = ref4s(b, r < 8 ? 1 : 3, (uint64_t)row * (H / 32) + 64u * cc + 4u * c);
        }
        __syncthreads();
        for (uint32_t u = tid; u < 64u * nk; u += kConvThreads) {
            const uint32_t kk = u / 64u, lane = u % 64u, n = lane % 16u, g = lane / 16u;
            *(uint4*)(dst + L.gu + (uint64_t)(T * G.nkt + 16u * cc + kk) * 1024 + 16u * lane) =
                *(const uint4*)(lds + n * kRowPad + 64u * kk + 16u * g);
        }
        if (tid < 64) {
            const uint32_t n = tid % 16u, g = tid / 16u;
            uint32_t v[4] = {0u, 0u, 0u, 0u};
            for (uint32_t i = 0; i < nk; i++) v[i / 4] |= (uint32_t)sc[n * kScPad + 4u * i + g] << (8 * (i % 4));
            *(uint4*)(dst + L.gus + (uint64_t)(T * G.ncca + cc) * 1024 + 16u * tid) = uint4{v[0], v[1], v[2], v[3]};
        }
        return;
    }
    w -= G.nA;
    if (w < G.nB) {
        // dn chunks (j, q) for 32 slices: LDS row r = down row 32q + r
        const uint32_t q = w / G.njb, jb = w % G.njb, nsl = min(32u, G.nj - 32u * jb);
        for (uint32_t u = tid; u < 32u * 2u * nsl; u += kConvThreads) {
            const uint32_t r = u / (2u * nsl), c = u % (2u * nsl);
            *(uint4*)(lds + r * kRowPad + 16u * c) = ref16(b, 4, (uint64_t)(32u * q + r) * (I / 2) + 1024u * jb + 16u * c);
        }
        __syncthreads();
        for (uint32_t u = tid; u < 64u * nsl; u += kConvThreads) {
            const uint32_t jj = u / 64u, lane = u % 64u, n = lane % 16u, g = lane / 16u;
            *(uint4*)(dst + L.dn + ((uint64_t)(32u * jb + jj) * G.nq + q) * 1024 + 16u * lane) =
                *(const uint4*)(lds + (n + 16u * (g >> 1)) * kRowPad + 32u * jj + 16u * (g & 1u));
        }
        return;
    }
    w -= G.nB;
    if (w >= G.nC) {
        w -= G.nC;
        if (w < G.nD) {
            // bgus words (sg, v, s) for 32 steps: LDS row 16i + n = the scale
            // row of tile 8(4sg + i) + v, row n, bytes [256c, +256) (64 k tiles)
            const uint32_t nc = (G.nstu + 31) / 32, sg = w / (8 * nc), v = (w / nc) % 8, c = w % nc;
            const uint32_t S = G.nj, nb = min(256u, H / 32 - 256u * c);  // scale bytes per row in this item
            for (uint32_t u = tid; u < 64u * (nb / 4u); u += kConvThreads) {
                const uint32_t r = u / (nb / 4u), cw = u % (nb / 4u), i = r / 16u, n = r % 16u, sl = 4u * sg + i;
                const uint32_t row = 8u * (8u * sl + v) + (n & 7u);
                *(uint32_t*)(lds + r * kBPad + 4u * cw) =
                    sl < S ? ref4s(b, n < 8 ? 1 : 3, (uint64_t)row * (H / 32) + 256u * c + 4u * cw) : 0u;
            }
            __syncthreads();
            const uint32_t ns = min(32u, G.nstu - 32u * c);
            for (uint32_t u = tid; u < 64u * ns; u += kConvThreads) {
                const uint32_t sl = u / 64u, lane = u % 64u, n = lane % 16u, g = lane / 16u;
                uint32_t v2[2] = {0u, 0u};
#pragma unroll
                for (uint32_t bb = 0; bb < 8; bb++) {
                    const uint32_t i = bb / 2u, q = bb % 2u, kt = 2u * (32u * c + sl) + q;
                    if (kt < G.nkt)  // tiles past I were staged as zeros
                        v2[bb / 4] |= (uint32_t)lds[(16u * i + n) * kBPad + 4u * (kt - 64u * c) + g] << (8 * (bb % 4));
                }
                *(uint2*)(dst + L.bgus + ((uint64_t)(sg * 8u + v) * G.nstu + 32u * c + sl) * 512 + 8u * lane) =
                    uint2{v2[0], v2[1]};
            }
            return;
        }
        w -= G.nD;
        // bdns words (rb, v, st) for 32 steps: LDS row 32h + r = the scale row
        // of down row 32q + r, q = 16rb + 2v + h, bytes [256c, +256) (128 slices)
        const uint32_t nc = (G.nstd + 31) / 32, rb = w / (8 * nc), v = (w / nc) % 8, c = w % nc;
        const uint32_t nb = min(256u, I / 32 - 256u * c);
        for (uint32_t u = tid; u < 64u * (nb / 4u); u += kConvThreads) {
            const uint32_t r = u / (nb / 4u), cw = u % (nb / 4u), q = 16u * rb + 2u * v + r / 32u;
            *(uint32_t*)(lds + r * kBPad + 4u * cw) =
                q < G.nq ? ref4s(b, 5, (uint64_t)(32u * q + r % 32u) * (I / 32) + 256u * c + 4u * cw) : 0u;
        }
        __syncthreads();
        const uint32_t ns = min(32u, G.nstd - 32u * c);
        for (uint32_t u = tid; u < 64u * ns; u += kConvThreads) {
            const uint32_t sl = u / 64u, lane = u % 64u, n = lane % 16u, g = lane / 16u;
            uint32_t v2[2] = {0u, 0u};
#pragma unroll
            for (uint32_t bb = 0; bb < 8; bb++) {
                const uint32_t i = bb / 2u, h = bb % 2u, sj = 4u * (32u * c + sl) + i;
                if (sj < G.nj)  // row pairs past H were staged as zeros
                    v2[bb / 4] |= (uint32_t)lds[(32u * h + n + 16u * (g >> 1)) * kBPad + 2u * (sj - 128u * c) + (g & 1u)]
                                  << (8 * (bb % 4));
            }
            *(uint2*)(dst + L.bdns + ((uint64_t)(rb * 8u + v) * G.nstd + 32u * c + sl) * 512 + 8u * lane) =
                uint2{v2[0], v2[1]};
        }
        return;
    }
    {
        // dns chunks (j, cc) for 32 slices: LDS row r = down row 512cc + r,
        // its scale bytes [64jb, +2 nsl)
        const uint32_t cc = w / G.njb, jb = w % G.njb, nsl = min(32u, G.nj - 32u * jb), nw = nsl / 2u;
        for (uint32_t u = tid; u < 512u * nw; u += kConvThreads) {
            const uint32_t r = u / nw, c = u % nw, row = 512u * cc + r;
            *(uint32_t*)(lds + r * kScPad + 4u * c) = row < H ? ref4s(b, 5, (uint64_t)row * (I / 32) + 64u * jb + 4u * c) : 0u;
        }
        __syncthreads();
        for (uint32_t u = tid; u < 64u * nsl; u += kConvThreads) {
            const uint32_t jj = u / 64u, lane = u % 64u, n = lane % 16u, g = lane / 16u;
            uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (uint32_t i = 0; i < 16; i++)
                if (16u * cc + i < G.nq)
                    v[i / 4] |= (uint32_t)lds[(32u * i + n + 16u * (g >> 1)) * kScPad + 2u * jj + (g & 1u)] << (8 * (i % 4));
            *(uint4*)(dst + L.dns + ((uint64_t)(32u * jb + jj) * G.nccc + cc) * 1024 + 16u * lane) =
                uint4{v[0], v[1], v[2], v[3]};
        }
    }
}

__global__ void shared_to_native_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, uint32_t H,
                                        uint32_t SI) {
    const NativeShared L = NativeShared::make(H, SI);
    const uint64_t nchunks = L.total / 16;
    const uint16_t* gate = src;
    const uint16_t* up = src + (uint64_t)SI * H;
    const uint16_t* down = src + (uint64_t)2 * SI * H;
    const uint32_t nkt = H / 32;
    for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < nchunks;
         c += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t off = c * 16;
        const uint16_t* from;
        if (off < L.sdn) {
            const uint32_t lane = (uint32_t)((off % 1024) / 16), n = lane % 16, g = lane / 16;
            const uint64_t k1 = off / 1024;
            const uint32_t T = (uint32_t)(k1 / nkt), kt = (uint32_t)(k1 % nkt);
            const uint32_t row = 8 * T + (n & 7);
            from = (n < 8 ? gate : up) + (uint64_t)row * H + kt * 32 + 8 * g;
        } else {
            const uint64_t idx = (off - L.sdn) / 16;
            const uint32_t T = (uint32_t)(idx / H), r = (uint32_t)(idx % H);
            from = down + (uint64_t)r * SI + 8 * T;
        }
        *(uint4*)((uint8_t*)dst + off) = *(const uint4*)from;
    }
}

// The down projection of an MXFP4 shared expert in the decode kernel's
// per-tile order (NativeShared4): dn8[T][r] = the 4 bytes of columns
// [8T, 8T + 8) of down row r, dns8[q][r] = the scale of columns [32q, +32).
__global__ void shared4_down_kernel(const RefBlock b, uint8_t* __restrict__ dst, uint32_t H, uint32_t SI) {
    const NativeShared4 L = NativeShared4::make(H, SI);
    const uint64_t nw = (uint64_t)(SI / 8) * H, nb = (uint64_t)(SI / 32) * H;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nw + nb;
         i += (uint64_t)gridDim.x * blockDim.x) {
        if (i < nw) {
            const uint32_t T = (uint32_t)(i / H), r = (uint32_t)(i % H);
            *(uint32_t*)(dst + L.dn8 + 4 * i) = ref4(b, 4, (uint64_t)r * (SI / 2) + 4 * T);
        } else {
            const uint64_t k = i - nw;
            const uint32_t q = (uint32_t)(k / H), r = (uint32_t)(k % H);
            dst[L.dns8 + k] = (uint8_t)ref1(b, 5, (uint64_t)r * (SI / 32) + q);
        }
    }
}

static RefBlock ref_block(const uint8_t* const* parts, uint32_t key) {
    RefBlock b;
    for (int r = 0; r < 6; r++) {
        b.src[r] = parts ? parts[r] : nullptr;
        b.salt[r] = mix32(0x632BE5ABu * (uint32_t)(r + 1));
    }
    b.key = key;
    return b;
}

static void ref_parts(const uint8_t* src, uint32_t H, uint32_t I, const uint8_t** parts) {
    uint64_t o = 0;
    const uint64_t len[6] = {(uint64_t)I * H / 2, (uint64_t)I * H / 32, (uint64_t)I * H / 2,
                             (uint64_t)I * H / 32, (uint64_t)H * I / 2, (uint64_t)H * I / 32};
    for (int r = 0; r < 6; r++) {
        parts[r] = src + o;
        o += len[r];
    }
}

static int launch_conv(const ConvBatch& cb, uint32_t n, uint32_t H, uint32_t I, void* stream) {
    const ConvGrid G = ConvGrid::make(H, I);
    hipLaunchKernelGGL(to_native_kernel, dim3(G.nA + G.nB + G.nC + G.nD + G.nE, n), dim3(kConvThreads), 0,
                       (hipStream_t)stream, cb,
                       H, I);
    return (int)hipGetLastError();
}

int launch_shared4_to_native(const uint8_t* const* parts, uint8_t* dst, uint32_t H, uint32_t SI, void* stream) {
    ConvBatch cb{};
    cb.b[0] = ref_block(parts, 0u);
    cb.dst[0] = dst + NativeShared4::make(H, SI).blk;
    int e = launch_conv(cb, 1, H, SI, stream);
    if (e != 0) return e;
    const RefBlock b = cb.b[0];
    const uint64_t n = (uint64_t)(SI / 8) * H + (uint64_t)(SI / 32) * H;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(shared4_down_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, b, dst, H, SI);
    return (int)hipGetLastError();
}

int launch_expert_to_native(const uint8_t* src, uint8_t* dst, uint32_t H, uint32_t I, uint32_t key, void* stream) {
    const uint8_t* parts[6];
    if (src) ref_parts(src, H, I, parts);
    ConvBatch cb{};
    cb.b[0] = ref_block(src ? parts : nullptr, key);
    cb.dst[0] = dst;
    return launch_conv(cb, 1, H, I, stream);
}

int launch_experts_to_native(const uint8_t* const* src, uint8_t* const* dst, uint32_t n, uint32_t H, uint32_t I,
                             void* stream) {
    for (uint32_t i0 = 0; i0 < n; i0 += kConvMax) {
        const uint32_t m = std::min(kConvMax, n - i0);
        ConvBatch cb{};
        for (uint32_t i = 0; i < m; i++) {
            const uint8_t* parts[6];
            ref_parts(src[i0 + i], H, I, parts);
            cb.b[i] = ref_block(parts, 0u);
            cb.dst[i] = dst[i0 + i];
        }
        const int e = launch_conv(cb, m, H, I, stream);
        if (e != 0) return e;
    }
    return 0;
}

int launch_shared_to_native(const uint16_t* src, uint16_t* dst, uint32_t H, uint32_t SI, void* stream) {
    const uint64_t chunks = NativeShared::make(H, SI).total / 16;
    uint64_t blocks = (chunks + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(shared_to_native_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, src, dst,
                       H, SI);
    return (int)hipGetLastError();
}

}  // namespace wl
