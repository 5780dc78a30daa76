// internal.h — structures shared by the host code (moe_host.cpp) and the
// gfx950 kernels (moe_decode.hip). Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace wl {

// Work-group shape of every kernel: 8 wave64s.
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;

// Rows of one routed-expert slice: a work-group computes 64 rows of an
// expert's SwiGLU output and applies the matching 64 columns of its down
// projection (8 waves x one 8-gate + 8-up row tile each).
constexpr uint32_t kSlice = 64;

// Largest grid the synchronisation block is sized for.
constexpr uint32_t kMaxGrid = 2048;

// Cross-work-group data of one decode layer lives in uncached device memory
// (MTYPE UC: loads and stores go to the memory side, never into a per-XCD L2),
// so a producer never needs an L2 write-back fence — measured on MI355X, one
// agent-scope release per work-group cut streaming from 5.2 to 0.9 TB/s — and
// a consumer's load always sees the latest value.
//
// Counters and release words each own a 128-byte line: read-modify-writes on
// one line serialise (about 15 ns each).
constexpr uint32_t kLineWords = 32;

// Error bits reported in the error word.
enum : uint32_t {
    E_SPIN = 1u,          // a grid barrier wait exceeded its bound
    E_NOT_RESIDENT = 2u,  // a routed expert resolved to a null block
};

// Word offsets inside the uncached synchronisation block.
struct SyncMap {
    uint32_t bar_grp;   // [8] arrival counters, one per group of work-groups (w % 8)
    uint32_t bar_all;   // arrivals of complete groups
    uint32_t bar_rel;   // [kMaxGrid] release words, one line per work-group
    uint32_t error;     // sticky error bits
    uint32_t words;
    __host__ __device__ static SyncMap make() {
        SyncMap m;
        uint32_t o = 0;
        m.bar_grp = o; o += 8 * kLineWords;
        m.bar_all = o; o += kLineWords;
        m.bar_rel = o; o += kMaxGrid * kLineWords;
        m.error = o;   o += kLineWords;
        m.words = o;
        return m;
    }
};

// Work decomposition of one layer over G work-groups (identical on host and
// device).
//   router rows      E rows, row r on work-group r mod G
//   shared gate/up   SI/8 tiles of 8 gate + 8 up rows, tile t on t mod G
//   shared down      (H/16 row tiles) x KS k-splits, unit v on v mod G
//   routed units     K experts x S = I/64 slices, unit u = (k = u mod K,
//                    j = u / K) on u mod G: rows [64j, 64j+64) of gate/up and
//                    columns [64j, 64j+64) of down; the partial down product
//                    of every unit is an H-vector in `part`
//   reduction        rows [RB*w, RB*w + RB) on work-group w
struct Plan {
    uint32_t G, S, U, KS, NSD, RB;
    __host__ __device__ static Plan make(uint32_t H, uint32_t I, uint32_t SI, uint32_t K, uint32_t G) {
        Plan p;
        p.G = G;
        p.S = I / kSlice;
        p.U = K * p.S;
        p.KS = (SI % 64u == 0u) ? 2u : 1u;
        p.NSD = (H / 16u) * p.KS;
        p.RB = (H + G - 1u) / G;
        return p;
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
    // intermediates kept for inspection (ordinary device memory)
    float* norm;                // [H]
    float* smid;                // [SI] shared SwiGLU output
    float* rmid;                // [K][I] routed SwiGLU outputs, slot order
    int32_t* idx;               // [K]
    float* topw;                // [K]
    float* shared_out;          // [H]
    float* edown;               // [K][H] routed down outputs before weighting
    // cross-work-group arrays (uncached)
    float* logits;              // [E]
    uint16_t* smid_p;           // [3][SI] bf16 pieces of smid
    float* part;                // [U][H] routed partial down products
    float* sdpart;              // [KS][H] shared-down partial sums
    uint32_t* sync;             // synchronisation block (SyncMap)
    // expert block layout (byte offsets)
    uint64_t gw_off, gs_off, uw_off, us_off, dw_off, ds_off, blk_bytes;
    uint32_t H, I, E, K, SI;
    float eps, scaling;
    int32_t norm_topk;
};

// Per-call launch arguments (kernel arguments by value). A layer runs as
// segments 0 (norm, router, shared gate/up), 1 (top-k, shared down, routed
// experts) and 2 (combine); a fused launch runs [0, 2] with grid barriers
// between segments, a phased schedule runs each segment as its own launch.
struct DecodeDyn {
    const float* hidden;        // [H] pre-norm residual stream
    const float* resid;         // [H] or null: out = resid + moe
    float* out;                 // [H]
    uint32_t seg_lo, seg_hi;
    uint32_t epoch;             // different for every call of the context
};

// Dynamic LDS layout of the decode kernel (byte offsets).
struct LdsMap {
    uint32_t xp, xn, smp, rmp, red, topk, slots, misc, bytes;
    __host__ __device__ static LdsMap make(uint32_t H, uint32_t SI, uint32_t E, uint32_t K, const Plan& p) {
        LdsMap m;
        auto al = [](uint32_t x) { return (x + 15u) & ~15u; };
        uint32_t o = 0;
        m.xp = o;   o += al(3u * (H + 8u) * 2u);
        m.xn = o;   // normalised input (f32); later the combine's staging
        const uint32_t fin = (p.U + p.KS + K) * p.RB * 4u;
        o += al(H * 4u > fin ? H * 4u : fin);
        m.smp = o;  o += al(3u * (SI + 8u) * 2u);
        m.rmp = o;  o += al(3u * (kSlice + 8u) * 2u);
        m.red = o;  o += kWaves * 64u * 4u;
        m.topk = o; o += al((2u * E + 64u) * 4u);
        m.slots = o; o += al(E * 8u);
        m.misc = o; o += 64u;
        m.bytes = o;
        return m;
    }
};

// Launchers (moe_decode.hip).
int launch_decode(const DecodeArgs* d_args, const DecodeDyn& dyn, uint32_t H, uint32_t I, uint32_t SI,
                  uint32_t E, uint32_t K, uint32_t grid, void* stream);
int decode_max_lds();
int launch_dequant_matvec(const uint8_t* W, const uint8_t* S, const float* x, float* y, uint32_t N,
                          uint32_t K, void* stream);
int launch_expert_ffn(const uint8_t* blk, uint64_t gw_off, uint64_t gs_off, uint64_t uw_off,
                      uint64_t us_off, uint64_t dw_off, uint64_t ds_off, const float* x, uint32_t H,
                      uint32_t I, float* mid, uint16_t* mid_p, float* y, uint16_t* y_bf16,
                      void* stream);
int launch_synth_expert(uint8_t* d_block, uint64_t gw_off, uint64_t gw_len, uint64_t gs_off,
                        uint64_t gs_len, uint64_t uw_off, uint64_t uw_len, uint64_t us_off,
                        uint64_t us_len, uint64_t dw_off, uint64_t dw_len, uint64_t ds_off,
                        uint64_t ds_len, uint32_t key, void* stream);
uint32_t synth_key(uint32_t seed, uint32_t layer, uint32_t expert);

}  // namespace wl
