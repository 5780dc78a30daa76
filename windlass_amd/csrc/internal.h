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

// Cross-work-group state of one decode layer lives in uncached device memory
// (MTYPE UC: loads and stores go to the memory side, never into a per-XCD L2),
// so a producer never needs an L2 write-back fence — measured on MI355X, one
// agent-scope release per task cut streaming from 5.2 to 0.9 TB/s — and a
// consumer's polling load always sees the latest value.
//
// Arrival counters (read-modify-write) each own a 128-byte line: RMWs on one
// line serialise at ~33 ns each. Completion flags hold the epoch of the call
// that set them, so they never need resetting.
constexpr uint32_t kLineWords = 32;

// Error bits reported in the error word.
enum : uint32_t {
    E_SPIN = 1u,          // a dependency wait exceeded its bound
    E_NOT_RESIDENT = 2u,  // a routed expert resolved to a null block
};

// Word offsets inside the uncached synchronisation block.
struct SyncMap {
    uint32_t c_rtile;   // [E/16] router tile arrivals (one line each)
    uint32_t c_sgtile;  // [SI/16] shared gate/up tile arrivals (one line each)
    uint32_t c_router;  // router tiles complete (one line)
    uint32_t c_rdblk;   // [H/64] routed-down block arrivals (one line each)
    uint32_t f_topk;    // epoch once top-k is published
    uint32_t f_sgu;     // [SI/16] epoch once shared SwiGLU tile t is published
    uint32_t f_rgu;     // [K][I/16] epoch once routed SwiGLU tile is published
    uint32_t f_sdown;   // [H/16] epoch once shared-down tile is published
    uint32_t error;     // sticky error bits
    uint32_t words;
    __host__ __device__ static SyncMap make(uint32_t H, uint32_t I, uint32_t E, uint32_t K, uint32_t SI) {
        SyncMap m;
        uint32_t o = 0;
        m.c_rtile = o;  o += (E / 16) * kLineWords;
        m.c_sgtile = o; o += (SI / 16) * kLineWords;
        m.c_router = o; o += kLineWords;
        m.c_rdblk = o;  o += (H / 64) * kLineWords;
        m.f_topk = o;   o += kLineWords;
        m.f_sgu = o;    o += SI / 16;
        m.f_rgu = o;    o += K * (I / 16);
        m.f_sdown = o;  o += H / 16;
        o = (o + kLineWords - 1) / kLineWords * kLineWords;
        m.error = o;    o += kLineWords;
        m.words = o;
        return m;
    }
};

struct DecodeArgs {
    const uint16_t* ln_w;       // [H] bf16 or null (= ones)
    const uint16_t* router_w;   // [E][H] bf16
    const float* bias;          // [E] f32
    const uint16_t* sh_gate;    // [SI][H] bf16
    const uint16_t* sh_up;      // [SI][H] bf16
    const uint16_t* sh_down;    // [H][SI] bf16
    const uint8_t* const* slot_tab;  // [E] block pointers of this layer
    // context scratch; the arrays marked (UC) are in uncached memory
    float* norm;                // [H]
    float* logits;              // [E] (UC)
    int32_t* idx;               // [K] (UC)
    float* topw;                // [K] (UC)
    const uint8_t** sel;        // [K] block pointers of the selected experts (UC)
    float* rmid;                // [K][I]
    uint16_t* rmid_p;           // [K][3][I] bf16 pieces of rmid (UC)
    float* smid;                // [SI]
    uint16_t* smid_p;           // [3][SI] (UC)
    float* shared_out;          // [H] (UC)
    float* edown;               // [K][H] routed down outputs before weighting (UC)
    float* part_r;              // [E/16][4][16] (UC)
    float* part_s;              // [SI/16][4][32] (UC)
    uint32_t* sync;             // uncached synchronisation block (SyncMap)
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
    uint32_t epoch;             // non-zero, different for every call of the context
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
