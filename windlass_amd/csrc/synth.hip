// synth.hip — counter-based synthetic expert blocks.
//
// Benchmark inputs have to fill tens of gigabytes of HBM quickly and still be
// reproducible on the CPU for the oracle, so every byte of a packed MXFP4
// expert block is a pure function of (seed, layer, expert, region, index):
//
//   mix32(x)      = lowbias32 integer hash (xor-shift-multiply, 2 rounds)
//   key           = mix32(mix32(seed ^ 0x9E3779B9) ^
//                         (layer * 0x85EBCA6B + expert * 0xC2B2AE35 + 0x27D4EB2F))
//   salt[r]       = mix32(0x632BE5AB * (r + 1)),  r = 0..5 in block order
//                   (gate_w, gate_s, up_w, up_s, down_w, down_s)
//   word(r, i)    = mix32(mix32(i ^ salt[r]) ^ key)
//   weight byte j = byte (j & 3) of word(r, j >> 2)   (little-endian)
//   scale byte j  = 118 + word(r, j) % 9              (E8M0 exponent in [118,126])
//
// The same formulas are restated in oracle/synth.py (numpy) and
// oracle/moe_oracle.c (C).
#include <hip/hip_runtime.h>
#include "internal.h"

namespace wl {

uint32_t synth_key(uint32_t seed, uint32_t layer, uint32_t expert) {
    return mix32(mix32(seed ^ 0x9E3779B9u) ^
                 (layer * 0x85EBCA6Bu + expert * 0xC2B2AE35u + 0x27D4EB2Fu));
}

struct SynthRegions {
    uint8_t* base;
    uint64_t off[6];
    uint64_t len[6];
    uint32_t salt[6];
    uint32_t key;
};

// One thread writes 16 bytes of a weight region or 4 bytes of a scale region.
__global__ void synth_kernel(const SynthRegions r, const uint64_t c1, const uint64_t c2,
                             const uint64_t c3, const uint64_t c4, const uint64_t c5,
                             const uint64_t c6) {
    const uint64_t cum[6] = {c1, c2, c3, c4, c5, c6};
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < c6; c += stride) {
        int reg = 0;
        while (c >= cum[reg]) reg++;
        const uint64_t local = c - (reg ? cum[reg - 1] : 0);
        const uint32_t salt = r.salt[reg];
        if ((reg & 1) == 0) {
            // 16 bytes = words 4*local .. 4*local+3
            uint4 v;
            const uint32_t w0 = (uint32_t)(local * 4);
            v.x = mix32(mix32((w0 + 0) ^ salt) ^ r.key);
            v.y = mix32(mix32((w0 + 1) ^ salt) ^ r.key);
            v.z = mix32(mix32((w0 + 2) ^ salt) ^ r.key);
            v.w = mix32(mix32((w0 + 3) ^ salt) ^ r.key);
            *(uint4*)(r.base + r.off[reg] + local * 16) = v;
        } else {
            // 4 scale bytes j = 4*local .. 4*local+3
            uint32_t packed = 0;
            const uint32_t j0 = (uint32_t)(local * 4);
            for (uint32_t b = 0; b < 4; b++) {
                const uint32_t s = 118u + mix32(mix32((j0 + b) ^ salt) ^ r.key) % 9u;
                packed |= s << (8 * b);
            }
            *(uint32_t*)(r.base + r.off[reg] + local * 4) = packed;
        }
    }
}

int launch_synth_expert(uint8_t* d_block, uint64_t gw_off, uint64_t gw_len, uint64_t gs_off,
                        uint64_t gs_len, uint64_t uw_off, uint64_t uw_len, uint64_t us_off,
                        uint64_t us_len, uint64_t dw_off, uint64_t dw_len, uint64_t ds_off,
                        uint64_t ds_len, uint32_t key, void* stream) {
    SynthRegions r;
    r.base = d_block;
    const uint64_t offs[6] = {gw_off, gs_off, uw_off, us_off, dw_off, ds_off};
    const uint64_t lens[6] = {gw_len, gs_len, uw_len, us_len, dw_len, ds_len};
    uint64_t cum[6];
    uint64_t acc = 0;
    for (int i = 0; i < 6; i++) {
        r.off[i] = offs[i];
        r.len[i] = lens[i];
        r.salt[i] = mix32(0x632BE5ABu * (uint32_t)(i + 1));
        acc += (i & 1) ? lens[i] / 4 : lens[i] / 16;
        cum[i] = acc;
    }
    r.key = key;
    const uint32_t threads = 256;
    uint64_t blocks = (acc + threads - 1) / threads;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(synth_kernel, dim3((uint32_t)blocks), dim3(threads), 0, (hipStream_t)stream,
                       r, cum[0], cum[1], cum[2], cum[3], cum[4], cum[5]);
    return (int)hipGetLastError();
}

}  // namespace wl
