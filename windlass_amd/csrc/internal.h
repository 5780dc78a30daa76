// internal.h — structures shared by the host code (moe_host.cpp) and the
// gfx950 kernels (moe_decode.hip). Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace wl {

// Work-group shape of every task kernel: 8 wave64s.
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;

// Counter words (device, zero at rest; the last work-group to leave a launch
// puts them back to zero). Per-tile arrival counters follow the fixed words.
enum CounterWord : uint32_t {
    C_CLAIM = 0,      // task queue head
    C_EXIT = 1,       // work-groups that have left the launch
    C_ROUTER = 2,     // router row tiles complete
    C_TOPK = 3,       // 1 once top-k ids/weights/block pointers are published
    C_SGU = 4,        // shared gate/up row tiles complete
    C_RGU = 5,        // routed gate/up row tiles complete
    C_SDOWN = 6,      // shared down row tiles complete
    C_ERROR = 7,      // sticky error bits, cleared by the host
    C_FIXED = 16      // first per-tile counter
};

// Error bits reported in C_ERROR.
enum : uint32_t {
    E_SPIN = 1u,          // a dependency wait exceeded its bound
    E_NOT_RESIDENT = 2u,  // a routed expert resolved to a null block
};

// Per-layer launch arguments; lives in device memory (one record per layer) so
// the kernel reads it through the scalar cache instead of holding ~60 kernel
// argument registers for its whole lifetime.
struct DecodeArgs {
    const uint16_t* ln_w;       // [H] bf16 or null (= ones)
    const uint16_t* router_w;   // [E][H] bf16
    const float* bias;          // [E] f32
    const uint16_t* sh_gate;    // [SI][H] bf16
    const uint16_t* sh_up;      // [SI][H] bf16
    const uint16_t* sh_down;    // [H][SI] bf16
    const uint8_t* const* slot_tab;  // [E] block pointers of this layer
    // context scratch
    float* norm;                // [H]
    float* logits;              // [E]
    int32_t* idx;               // [K]
    float* topw;                // [K]
    const uint8_t** sel;        // [K] block pointers of the selected experts
    float* rmid;                // [K][I]
    uint16_t* rmid_p;           // [K][3][I] bf16 pieces of rmid
    float* smid;                // [SI]
    uint16_t* smid_p;           // [3][SI]
    float* shared_out;          // [H]
    float* edown;               // [K][H] routed down outputs before weighting
    float* part_r;              // [E/16][4][16]
    float* part_s;              // [SI/16][4][32]
    uint32_t* ctr;              // counters
    // expert block layout (byte offsets)
    uint64_t gw_off, gs_off, uw_off, us_off, dw_off, ds_off;
    uint32_t H, I, E, K, SI;
    float eps, scaling;
    int32_t norm_topk;
};

// Per-call launch arguments (kernel arguments by value).
struct DecodeDyn {
    const float* hidden;        // [H] pre-norm residual stream
    const float* resid;         // [H] or null: out = resid + moe
    float* out;                 // [H]
    uint32_t task_lo, task_hi;  // task range of this launch
    int32_t wait_deps;          // 0 when stream order already satisfies dependencies
    int32_t write_norm_tap;     // 1 in the launch that owns task 0
};

// Row tiles (16 rows each) per routed-down task: one expert x 64 output rows.
constexpr uint32_t kDownRT = 4;

// Task index space of one decode layer, in dependency order.
struct TaskMap {
    uint32_t nR, nSG, nRG, nSD, nRD;
    uint32_t oSG, oRG, oSD, oRD, total;
    __host__ __device__ static TaskMap make(uint32_t H, uint32_t I, uint32_t E, uint32_t K, uint32_t SI) {
        TaskMap t;
        t.nR = (E / 16) * 4;
        t.nSG = (SI / 16) * 4;
        t.nRG = K * (I / 16);
        t.nSD = H / 16;
        t.nRD = K * (H / (16 * kDownRT));
        t.oSG = t.nR;
        t.oRG = t.oSG + t.nSG;
        t.oSD = t.oRG + t.nRG;
        t.oRD = t.oSD + t.nSD;
        t.total = t.oRD + t.nRD;
        return t;
    }
};

// Dynamic LDS of the decode kernel: three bf16 pieces of the normalised input
// (one padded row each), the cross-wave reduction area (kWaves x 64 floats),
// the per-expert row sums (32 x 16 floats) and the top-k staging (2E + 32 floats).
__host__ __device__ inline size_t decode_lds_xp_elems(uint32_t H) { return (size_t)3 * (H + 8); }
__host__ __device__ inline size_t decode_lds_bytes(uint32_t H, uint32_t E) {
    return decode_lds_xp_elems(H) * 2 + (size_t)kWaves * 64 * 4 + 32 * 16 * 4 + ((size_t)2 * E + 32) * 4;
}

// Launchers (moe_decode.hip).
int launch_decode(const DecodeArgs* d_args, const DecodeDyn& dyn, uint32_t H, uint32_t E,
                  uint32_t grid, void* stream);
int launch_dequant_matvec(const uint8_t* W, const uint8_t* S, const float* x, float* y, uint32_t N,
                          uint32_t K, void* stream);
int launch_expert_ffn(const uint8_t* blk, uint64_t gw_off, uint64_t gs_off, uint64_t uw_off,
                      uint64_t us_off, uint64_t dw_off, uint64_t ds_off, const float* x, uint32_t H,
                      uint32_t I, float* mid, uint16_t* mid_p, float* y, uint16_t* y_bf16,
                      void* stream);
int decode_occupancy(uint32_t H, uint32_t E, int* blocks_per_cu);
int launch_synth_expert(uint8_t* d_block, uint64_t gw_off, uint64_t gw_len, uint64_t gs_off,
                        uint64_t gs_len, uint64_t uw_off, uint64_t uw_len, uint64_t us_off,
                        uint64_t us_len, uint64_t dw_off, uint64_t dw_len, uint64_t ds_off,
                        uint64_t ds_len, uint32_t key, void* stream);
uint32_t synth_key(uint32_t seed, uint32_t layer, uint32_t expert);

}  // namespace wl
