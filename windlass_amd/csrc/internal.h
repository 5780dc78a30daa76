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

// Cross-work-group data of one layer (logits, shared SwiGLU values, partial
// sums) is ordinary device memory written with agent-scope (sc1) stores, which
// write through the writer's L2, and read with agent-scope (sc1) loads, which
// never return a line cached in a per-CU L1 or per-XCD L2 — measured on
// MI355X: plain loads after a grid barrier return stale data for the other
// XCDs, sc1 loads never did, and an L2 invalidate per work-group costs ~14 us.
// A release fence (L2 write-back) is never needed; one per work-group cut
// streaming from 5.2 to 0.9 TB/s.
//
// The error word lives in uncached memory so that read-modify-writes from
// all XCDs meet at one point; it owns a 128-byte line.
constexpr uint32_t kLineWords = 32;

// Error bits reported in the error word.
enum : uint32_t {
    E_SPIN = 1u,          // a wait for another work-group's data exceeded its bound
    E_NOT_RESIDENT = 2u,  // a routed expert resolved to a null block
    E_XCD = 4u,           // two-level combine: a work-group ran on another XCD than w mod 8
    E_TOKTAB = 8u,        // batched gate/up: a work-group's units needed more token-table entries than sized
};

// Word offsets inside the uncached synchronisation block.
//   error  sticky error bits, accumulated over calls until wl_check_error
//          reads and clears them
//   abort  the epoch of the last call that raised an error: a wait gives up
//          early only when this equals its own call's epoch, so an error of
//          one call never cuts short the waits of a later one
struct SyncMap {
    uint32_t error;
    uint32_t abort;
    uint32_t ticket;  // [3] combine-ticket counters, one per partial tag (tag t: ticket + t - 1)
    uint32_t words;
    __host__ __device__ static SyncMap make() {
        SyncMap m;
        m.error = 0;
        m.abort = kLineWords / 2;
        m.ticket = kLineWords;
        m.words = 2 * kLineWords;
        return m;
    }
};

// Work decomposition of one layer over G work-groups (identical on host and
// device).
//   router rows      E rows, row r on work-group r mod G
//   shared expert    SI/8 tiles of 8 gate + 8 up rows; the work-group of tile t
//                    also applies columns [8t, 8t+8) of the down projection
//   routed units     K experts x S = I/64 slices, unit u = (k = u mod K,
//                    j = u / K) on u mod G: rows [64j, 64j+64) of gate/up and
//                    columns [64j, 64j+64) of down
//   partials         every work-group's w_k-weighted routed and shared
//                    contributions, summed per output row in LDS, published as
//                    one H-vector per work-group of epoch-tagged words
//   combine          H/32 blocks of 32 rows; the work-group that takes ticket t
//                    (tickets in the order work-groups finish their own work)
//                    combines blocks t, t + G, ...
constexpr uint32_t kRowBlock = 32;  // rows per combine block (= rows per down item)
// Words of each partial-sum array (part, tsh): [H/32][G][32] for the
// one-level combine; the two-level combine uses the same H x G words as
// [8 XCDs][H/32][G/8][32] and the 8 x H words after them as [H/32][8][32]
// (each XCD's sum of its work-groups' partials).
__host__ __device__ inline size_t part_words(uint32_t H, uint32_t G) { return (size_t)H * (G + 8u); }
struct Plan {
    uint32_t G, S, U, NB;
    __host__ __device__ static Plan make(uint32_t H, uint32_t I, uint32_t SI, uint32_t K, uint32_t G) {
        (void)SI;
        Plan p;
        p.G = G;
        p.S = I / kSlice;
        p.U = K * p.S;
        p.NB = H / kRowBlock;
        return p;
    }
};

struct DecodeArgs {
    const uint16_t* ln_w;       // [H] bf16 or null (= ones)
    const uint16_t* router_w;   // [E][H] bf16
    const float* bias;          // [E] f32
    const uint8_t* sh_native;   // shared expert, NativeShared layout
    const uint8_t* const* slot_tab;  // [E] block pointers of this layer
    // intermediates kept for inspection (ordinary stores, read after the launch)
    float* norm;                // [H]
    float* logits;              // [E]
    float* smid;                // [SI] shared SwiGLU output
    float* rmid;                // [K][I] routed SwiGLU outputs, slot order
    int32_t* idx;               // [K]
    float* topw;                // [K]
    float* shared_out;          // [H] (written when taps are on)
    // cross-work-group arrays (agent-scope stores and loads)
    uint64_t* lslot;            // [E] logit of this call: epoch << 32 | f32 bits
    uint32_t* part;             // [H/32][G][32] partials, block-major: f32 at 21 mantissa bits | 2-bit call tag
    uint32_t* tsh;              // [H/32][G][32] shared-expert partials (taps on), tagged likewise
    uint32_t* sync;             // synchronisation block (SyncMap), uncached
    uint32_t H, I, E, K, SI;
    float eps, scaling;
    int32_t norm_topk;
};

// Per-call launch arguments. A layer runs as segment 0 (everything up to the
// published partials) and segment 1 (the combine); a fused launch runs both
// (the combine waits for the epoch tags of the partials it reads), the phased
// schedule runs each as its own launch. The decode kernel takes these as
// separate scalar kernel arguments, the record pointer and the first fields
// below up to `epoch` in front, and is built with kernarg preloading: those
// 14 dwords arrive in SGPRs, so the loads that start a layer (the hidden
// state, the norm weight, the router row, the shared expert and its logit
// polls) are issued without first waiting for a memory round trip to read
// their addresses. (A struct argument is not preloaded: its fields would be
// read from the kernarg segment with scalar loads, two dependent round trips
// before the first vector load.) The same pointers are also in the layer
// record (DecodeArgs) for the other kernels.
struct DecodeDyn {
    const float* hidden;        // [H] pre-norm residual stream
    const uint8_t* sh_native;   // the layer's shared expert (NativeShared)
    const uint16_t* router_w;   // [E][H] bf16
    const uint16_t* ln_w;       // [H] bf16 or null (= ones)
    uint64_t* lslot;            // [E] the context's epoch-tagged logit slots
    uint32_t seg;               // bits 0-7: first segment, 8-15: last segment, 16: shared-expert tap on,
                                // 24-25: the partials' tag of this call (1-3, differs from the previous call's)
    uint32_t epoch;             // different for every call of the context, never 0
    // not preloaded (read later in the layer)
    const float* bias;          // [E] f32
    const uint8_t* const* slot_tab;  // [E] block pointers of this layer
    const float* resid;         // [H] or null: out = resid + moe
    float* out;                 // [H]
    __host__ __device__ uint32_t seg_lo() const { return seg & 0xFFu; }
    __host__ __device__ uint32_t seg_hi() const { return (seg >> 8) & 0xFFu; }
    __host__ __device__ int32_t taps() const { return (int32_t)((seg >> 16) & 1u); }
    __host__ __device__ uint32_t ptag() const { return (seg >> 24) & 3u; }
    // bit 17: the two-level combine (partials summed per XCD through its L2 first)
    __host__ __device__ bool xl2() const { return ((seg >> 17) & 1u) != 0u; }
};
// Dwords of kernel arguments the decode kernel preloads into SGPRs (the
// record pointer, then hidden .. epoch).
constexpr int kPreloadDwords = 14;

// Dynamic LDS layout of the decode kernel (byte offsets).
struct LdsMap {
    uint32_t xp, pv, rmp, red, topk, slots, misc, bytes;
    __host__ __device__ static LdsMap make(uint32_t H, uint32_t SI, uint32_t E, uint32_t K, const Plan& p) {
        (void)SI;
        (void)K;
        LdsMap m;
        auto al = [](uint32_t x) { return (x + 15u) & ~15u; };
        uint32_t o = 0;
        m.xp = o;   o += al(3u * (H + 8u) * 2u);
        m.rmp = o;  o += al(3u * (kSlice + 8u) * 2u);
        m.red = o;  o += kWaves * 64u * 4u;
        m.topk = o; o += al((2u * E + 64u) * 4u);
        m.slots = o; o += al(E * 8u);
        m.misc = o; o += 128u;
        // last: its size depends on the grid, so no other offset does (the
        // kernel's first loads then need no wait for the grid size)
        m.pv = o;   // normalised input; this work-group's partial; combine staging
        uint32_t f32n = (p.G + 16u) * kRowBlock;
        if (f32n < H) f32n = H;
        // the two-level combine stages all first-level blocks of a work-group
        // at once: at most (H/32 + G/8) x 32 words
        if (f32n < H + 4u * p.G) f32n = H + 4u * p.G;
        o += al(f32n * 4u);
        m.bytes = o;
        return m;
    }
};

// lowbias32 integer hash of the synthetic-weight generator (synth.hip).
__host__ __device__ inline uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7FEB352Du;
    x ^= x >> 15;
    x *= 0x846CA68Bu;
    x ^= x >> 16;
    return x;
}

// ---- native (HBM) layouts ----------------------------------------------------
// Expert blocks bound to the decode kernel are stored so that every 16-byte
// load of a wave is one lane of a 1 KB contiguous chunk, in the lane order the
// MFMA operands want (lane l = (n, g) = (l % 16, l / 16)), and the E8M0 scales
// of 16 consecutive k tiles (or row pairs) of one lane are one 16-byte chunk.
// The reference layout (gate_w | gate_s | up_w | up_s | down_w | down_s, rows
// of packed nibbles) is what callers provide; wl_expert_to_native converts.
//
//   gu   [I/8 tiles][H/128 k tiles] 1 KB: lane (n,g) = row n<8 ? gate 8T+n :
//        up 8T+n-8, bytes [64kt + 16g, +16) of that row
//   gus  [I/8 tiles][ceil(H/2048)] 1 KB: lane byte i = scale of the lane's
//        row at k tile 16c + i, block 4kt + g (0 past the end)
//   dn   [I/64 slices][H/32 row pairs] 1 KB: lane (n,g) = down row
//        32q + n + 16(g>>1), bytes [32j + 16(g&1), +16)
//   dns  [I/64 slices][ceil(H/512)] 1 KB: lane byte i = scale of the lane's
//        row at pair 16c + i, block 2j + (g&1)
// The same scales again in the order of the batched GEMM kernels
// (moe_batched.hip: units of 4 slices or 16 row pairs, 8 waves, 256-column
// steps), so that a wave reads one 8-byte word per lane and step:
//   bgus [ceil(I/256) slice groups sg][8 waves v][ceil(H/256) steps s] 512 B:
//        lane (n,g) byte 2i + q = scale of the lane's row of tile
//        8(4sg + i) + v at k tile 2s + q, block 4kt + g
//   bdns [ceil(H/512) row blocks rb][8 waves v][ceil(I/256) steps st] 512 B:
//        lane (n,g) byte 2i + h = scale of down row 32q + n + 16(g>>1),
//        q = 16rb + 2v + h, at slice 4st + i, block 2j + (g&1)
// (0 past the end of either dimension).
struct NativeLayout {
    uint64_t gu, gus, dn, dns, bgus, bdns, total;
    __host__ __device__ static NativeLayout make(uint32_t H, uint32_t I) {
        NativeLayout m;
        uint64_t o = 0;
        m.gu = o;  o += (uint64_t)(I / 8) * (H / 128) * 1024;
        m.gus = o; o += (uint64_t)(I / 8) * ((H / 128 + 15) / 16) * 1024;
        m.dn = o;  o += (uint64_t)(I / 64) * (H / 32) * 1024;
        m.dns = o; o += (uint64_t)(I / 64) * ((H / 32 + 15) / 16) * 1024;
        m.bgus = o; o += (uint64_t)((I + 255) / 256) * 8 * ((H + 255) / 256) * 512;
        m.bdns = o; o += (uint64_t)((H + 511) / 512) * 8 * ((I + 255) / 256) * 512;
        m.total = o;
        return m;
    }
};
// The shared expert (bf16) per layer:
//   sgu  [SI/8 tiles][H/32 k tiles] 1 KB: lane (n,g) = row n<8 ? gate 8T+n :
//        up 8T+n-8, columns [32kt + 8g, +8)
//   sdn  [SI/8 tiles][H rows] 16 B: columns [8T, 8T+8) of down row r
struct NativeShared {
    uint64_t sgu, sdn, total;
    __host__ __device__ static NativeShared make(uint32_t H, uint32_t SI) {
        NativeShared m;
        m.sgu = 0;
        m.sdn = (uint64_t)(SI / 8) * (H / 32) * 1024;
        m.total = m.sdn + (uint64_t)(SI / 8) * H * 16;
        return m;
    }
};

// An MXFP4 shared expert (WL_SHARED_MXFP4; inter SI = moe_inter):
//   blk   the routed-expert native block (NativeLayout(H, SI)): gate/up of
//         the decode kernel, gate/up and down of the batched kernels
//   dn8   [SI/8 tiles][H rows] 4 bytes: the nibbles of columns [8T, 8T+8) of
//         down row r (the decode kernel's work-group of tile T applies them)
//   dns8  [SI/32][H rows] 1 byte: the scale of columns [32q, 32q+32) of row r
struct NativeShared4 {
    uint64_t blk, dn8, dns8, total;
    __host__ __device__ static NativeShared4 make(uint32_t H, uint32_t SI) {
        NativeShared4 m;
        m.blk = 0;
        m.dn8 = NativeLayout::make(H, SI).total;
        m.dns8 = m.dn8 + (uint64_t)(SI / 8) * H * 4;
        m.total = m.dns8 + (((uint64_t)(SI / 32) * H + 1023) & ~(uint64_t)1023);
        return m;
    }
};

// Batched (multi-token) layer, reference run_moe_batched
// (src/glm_layer_runner.cuh:818-928): per-token routing, tokens grouped by
// expert (stable: (token, slot) order), grouped GEMMs, per-token combine in
// slot order. Scratch is context-owned and sized for T tokens.
// BatchArgs::flags: experts whose slot-table entry is null get no GEMM units
// (a source-backed layer runs its routed set in chunks of experts); the
// shared expert's units are left out (they run with the first chunk only).
// kBatchShared4: the shared expert is MXFP4 and runs as expert E of the pass
// table (all T tokens, activations straight from norm3, outputs in the rows
// [T*K, T*K + T) of mid3 and expout).
// kBatchWideSharedUp / Down (set by launch_batched): the bf16 shared
// expert's gate/up (down) runs as 64-token units in the wide GEMM kernel.
enum : uint32_t {
    kBatchSkipUnbound = 1u,
    kBatchNoShared = 2u,
    kBatchShared4 = 4u,
    kBatchWideSharedUp = 8u,
    kBatchWideSharedDown = 16u
};
// Routed experts of few tokens run their gate/up and down projections in the
// GEMM kernels' streaming pipelines (run_small_up, run_small_down) when
// launch_batched takes those kernels' small-expert instantiations (at the
// shapes they fit): 1..kSmallT tokens in one MFMA row block, and at the GLM
// shape kSmallT+1..kSmallUpT (moe_batched.hip) in two; their pass tables leave
// them out of the other pipelines.
constexpr uint32_t kSmallT = 4;
// launch_batched phases: routing (norm .. scatter), the GEMMs, the combine.
enum : uint32_t { kPhaseRoute = 1u, kPhaseGemm = 2u, kPhaseCombine = 4u, kPhaseAll = 7u };
struct BatchArgs {
    uint32_t T;
    uint32_t flags;
    const float* hidden;   // [T][H] pre-norm residual stream
    const float* resid;    // [T][H] or null
    float* out;            // [T][H]
    float* norm;           // [T][H]
    uint16_t* norm3;       // [T][3][H] bf16 pieces of norm
    float* logits;         // [T][E]
    int32_t* idx;          // [T][K]
    float* wts;            // [T][K]
    uint32_t* counts;      // [E]
    uint32_t* offsets;     // [E+1]
    uint32_t* lists;       // [E][T] entries (token*K + slot) of expert e, ascending
    uint32_t* ent;         // [T*K] compact index -> token*K + slot (expert-major)
    uint32_t* pos;         // [T*K] token*K + slot -> compact index
    uint16_t* mid3;        // [T*K (+T)][3][I] routed (and MXFP4 shared) SwiGLU outputs (pieces), compact rows
    float* expout;         // [T*K (+T)][H] routed (and MXFP4 shared) expert outputs, compact rows
    uint16_t* smid3;       // [T][3][SI] shared SwiGLU outputs (pieces)
    float* shout;          // [T][H]
    uint32_t tcap;         // token-table entries per work-group in bup_kernel's LDS (set by launch_batched)
    uint32_t* wq;          // [kWqWords] work-queue counters of the streaming units: zero between launches
                           // (zeroed once when the scratch is made, reset by each launch's last work-group)
};
constexpr uint32_t kWqWords = 8;

// Launchers (moe_decode.hip).
int launch_decode(const DecodeArgs* d_args, const DecodeDyn& dyn, uint32_t H, uint32_t I, uint32_t SI,
                  uint32_t E, uint32_t K, uint32_t grid, bool sh4, void* stream);
// n consecutive resident layers (records recs[0..n)) in one launch, in place
// on d_h: epochs epoch0 .. epoch0 + n - 1, partial tags from seg0's; hx [H]
// u64 carries each layer's output to the next (tagged words).
int launch_chain(const DecodeArgs* recs, float* d_h, uint64_t* lslot, uint64_t* hx, uint32_t n, uint32_t epoch0,
                 uint32_t seg0, uint32_t H, uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid, bool sh4,
                 void* stream);
int decode_max_lds();
// Whether work-group w of a grid-sized launch runs on XCD w mod 8 (every
// work-group's XCC_ID register read back): *ok. Returns a hipError_t.
int probe_xcd_map(uint32_t grid, bool* ok);
// Work-groups of the decode / routing kernel one CU can hold at once
// (hipOccupancyMaxActiveBlocksPerMultiprocessor at the kernel's LDS size).
int decode_occupancy(uint32_t H, uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid, int* per_cu);
int route_occupancy(uint32_t H, uint32_t E, int* per_cu);
// Routing only (cache-backed layers): norm, router, top-k -> idx/topw/logits.
size_t route_lds_bytes(uint32_t H, uint32_t E);
int launch_route(const DecodeArgs* d_args, const float* hidden, uint32_t epoch, uint32_t H, uint32_t E,
                 uint32_t grid, void* stream);
// table[e] = ptrs[k] where ids[k] == e, null elsewhere (n <= 32).
int launch_slot_fill(const uint8_t** table, uint32_t E, const int32_t* ids, const uint8_t* const* ptrs, uint32_t n,
                     void* stream);
int launch_dequant_matvec(const uint8_t* W, const uint8_t* S, const float* x, float* y, uint32_t N,
                          uint32_t K, void* stream);
// The one-launch expert FFN (moe_decode.hip): its arguments.
struct FfnArgs {
    const uint8_t* blk;  // reference-layout block
    uint64_t gw_off, gs_off, uw_off, us_off, dw_off, ds_off;
    const float* x;      // [H]
    float* y;            // [H]
    uint16_t* y_bf16;    // [H] or null
    uint64_t* tag;       // [I] epoch-tagged SwiGLU values (context scratch, zeroed at creation)
    uint32_t* sync;      // synchronisation block (error and abort words)
    uint32_t H, I, epoch;
};
// Returns -1 (nothing launched) for a shape or grid it is not built for.
int launch_expert_ffn1(const FfnArgs& a, uint32_t grid, void* stream);
int launch_expert_ffn(const uint8_t* blk, uint64_t gw_off, uint64_t gs_off, uint64_t uw_off,
                      uint64_t us_off, uint64_t dw_off, uint64_t ds_off, const float* x, uint32_t H,
                      uint32_t I, float* mid, uint16_t* mid_p, float* y, uint16_t* y_bf16,
                      void* stream);
// Batched layer (moe_batched.hip): every stage on `stream`.
// The most routed experts the batched layer supports (its GEMM kernels keep
// the expert tables in LDS beside the activation slots).
uint32_t batched_max_experts();
// Largest batched chunk (tokens per launch) whose gate/up token table fits in
// LDS beside the activation slots and the expert tables, for a grid of at
// least `grid` work-groups.
uint32_t batched_max_tokens(uint32_t I, uint32_t SI, uint32_t E, uint32_t K, uint32_t grid);
int launch_batched(const DecodeArgs* d_args, const BatchArgs& b, uint32_t H, uint32_t I, uint32_t SI, uint32_t E,
                   uint32_t K, uint32_t n_cu, uint32_t phases, void* stream);
// The library's static device scratch (noalloc.hip): its device address on
// `device` (which must be current), looked up once per device and kept;
// and its size in bytes.
int noalloc_scratch(int device, void** ptr);
size_t noalloc_scratch_bytes();
// Reference-layout block -> native block (src null: synthesise the native
// block directly from the counter-based generator with `key`).
int launch_expert_to_native(const uint8_t* src, uint8_t* dst, uint32_t H, uint32_t I, uint32_t key, void* stream);
// n reference-layout packed blocks src[i] -> native blocks dst[i], up to 16
// per launch.
int launch_experts_to_native(const uint8_t* const* src, uint8_t* const* dst, uint32_t n, uint32_t H, uint32_t I,
                             void* stream);
int launch_shared_to_native(const uint16_t* src, uint16_t* dst, uint32_t H, uint32_t SI, void* stream);
// The six reference tensors of an MXFP4 shared expert (gate_w, gate_s, up_w,
// up_s, down_w, down_s) -> NativeShared4.
int launch_shared4_to_native(const uint8_t* const* parts, uint8_t* dst, uint32_t H, uint32_t SI, void* stream);
int launch_synth_expert(uint8_t* d_block, uint64_t gw_off, uint64_t gw_len, uint64_t gs_off,
                        uint64_t gs_len, uint64_t uw_off, uint64_t uw_len, uint64_t us_off,
                        uint64_t us_len, uint64_t dw_off, uint64_t dw_len, uint64_t ds_off,
                        uint64_t ds_len, uint32_t key, void* stream);
uint32_t synth_key(uint32_t seed, uint32_t layer, uint32_t expert);

}  // namespace wl
