// native.hip — conversion of expert blocks and shared experts into the decode
// kernel's HBM layout (NativeLayout / NativeShared in internal.h).
//
// One thread per 16-byte chunk of the destination: a weight chunk is one
// contiguous 16-byte run of a reference row (a copy), a scale chunk gathers 16
// scale bytes of one row (16 consecutive k tiles or row pairs). With a null
// source the bytes come from the synthetic-weight generator (synth.hip) at the
// reference position they would have been copied from, so a synthetic block
// can be written in the native layout directly.
#include <hip/hip_runtime.h>
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

__global__ void expert_to_native_kernel(const RefBlock b, uint8_t* __restrict__ dst, uint32_t H, uint32_t I) {
    const NativeLayout L = NativeLayout::make(H, I);
    const uint64_t nchunks = L.total / 16;
    const uint32_t nkt = H / 128, nsc = (nkt + 15) / 16, nq = H / 32, ndc = (nq + 15) / 16;
    for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < nchunks;
         c += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t off = c * 16;
        const uint32_t lane = (uint32_t)((off % 1024) / 16), n = lane % 16, g = lane / 16;
        uint4 v = {0u, 0u, 0u, 0u};
        if (off < L.gus) {
            const uint64_t k1 = off / 1024;
            const uint32_t T = (uint32_t)(k1 / nkt), kt = (uint32_t)(k1 % nkt);
            const uint32_t row = 8 * T + (n & 7);
            v = ref16(b, n < 8 ? 0 : 2, (uint64_t)row * (H / 2) + kt * 64 + 16 * g);
        } else if (off < L.dn) {
            const uint64_t k1 = (off - L.gus) / 1024;
            const uint32_t T = (uint32_t)(k1 / nsc), cc = (uint32_t)(k1 % nsc);
            const uint32_t row = 8 * T + (n & 7);
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            for (uint32_t i = 0; i < 16; i++) {
                const uint32_t kt = 16 * cc + i;
                if (kt < nkt) w[i / 4] |= ref1(b, n < 8 ? 1 : 3, (uint64_t)row * (H / 32) + kt * 4 + g) << (8 * (i % 4));
            }
            v = uint4{w[0], w[1], w[2], w[3]};
        } else if (off < L.dns) {
            const uint64_t k1 = (off - L.dn) / 1024;
            const uint32_t j = (uint32_t)(k1 / nq), q = (uint32_t)(k1 % nq);
            const uint32_t row = 32 * q + n + 16 * (g >> 1);
            v = ref16(b, 4, (uint64_t)row * (I / 2) + 32 * j + 16 * (g & 1));
        } else {
            const uint64_t k1 = (off - L.dns) / 1024;
            const uint32_t j = (uint32_t)(k1 / ndc), cc = (uint32_t)(k1 % ndc);
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            for (uint32_t i = 0; i < 16; i++) {
                const uint32_t q = 16 * cc + i;
                const uint32_t row = 32 * q + n + 16 * (g >> 1);
                if (q < nq) w[i / 4] |= ref1(b, 5, (uint64_t)row * (I / 32) + 2 * j + (g & 1)) << (8 * (i % 4));
            }
            v = uint4{w[0], w[1], w[2], w[3]};
        }
        *(uint4*)(dst + off) = v;
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

int launch_shared4_to_native(const uint8_t* const* parts, uint8_t* dst, uint32_t H, uint32_t SI, void* stream) {
    const RefBlock b = ref_block(parts, 0u);
    const uint64_t chunks = NativeLayout::make(H, SI).total / 16;
    uint64_t blocks = (chunks + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(expert_to_native_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, b,
                       dst + NativeShared4::make(H, SI).blk, H, SI);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    const uint64_t n = (uint64_t)(SI / 8) * H + (uint64_t)(SI / 32) * H;
    blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(shared4_down_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, b, dst, H, SI);
    return (int)hipGetLastError();
}

int launch_expert_to_native(const uint8_t* src, uint8_t* dst, uint32_t H, uint32_t I, uint32_t key, void* stream) {
    const uint8_t* parts[6];
    if (src) ref_parts(src, H, I, parts);
    const RefBlock b = ref_block(src ? parts : nullptr, key);
    const uint64_t chunks = NativeLayout::make(H, I).total / 16;
    uint64_t blocks = (chunks + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(expert_to_native_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, b, dst,
                       H, I);
    return (int)hipGetLastError();
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
