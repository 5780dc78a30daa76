// moe_host.cpp — the C ABI of include/windlass_moe.h: context, layer binding,
// the HBM slot table and the launch schedule of the decode layer.
//
// Reference call surface this replaces: glm::run_moe + glm::ExpertSource +
// glm::ExpertLayout (src/glm_layer_runner.cuh:34-72,352-443) and the MoE part of
// glm::alloc_scratch (src/glm_loader.cuh:363-450).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/windlass_moe.h"
#include "attention.h"
#include "expert_files.h"
#include "host_internal.h"
#include "internal.h"
#include "lru.h"

struct LayerState {
    const uint16_t* router_w = nullptr;
    const float* bias = nullptr;
    const uint16_t* ln = nullptr;
    uint8_t* shared = nullptr;  // context-owned native copy of the shared expert
    size_t shared_bytes = 0;
    int32_t shared_dtype = WL_SHARED_BF16;
    bool set = false;
    std::vector<void*> owned;  // router / bias / norm buffers the context took over (wl_load_layer)
    // a dense MLP layer (wl_set_layer_dense): no router, no experts
    bool dense = false;
    const uint16_t *mlp_gate = nullptr, *mlp_up = nullptr, *mlp_down = nullptr;
    uint32_t dense_inter = 0;
};

// HBM expert cache (config 4): LRU slot pool filled from pinned host blocks.
struct CacheState {
    wl::SlotLru* lru = nullptr;
    wl_cache_policy policy{WL_POLICY_LRU, 0.5f, 0u};
    uint32_t transient = 0;          // slots [capacity, capacity + transient): misses not retained
    std::vector<uint32_t> pinned;    // pinned keys (kept across wl_cache_set_policy)
    uint64_t bypassed = 0;           // misses served from a transient slot
    uint8_t* pool = nullptr;
    uint32_t capacity = 0;
    wl_host_block_fn fn = nullptr;
    void* user = nullptr;
    hipStream_t copy[2] = {nullptr, nullptr};  // side streams for host-to-device copies
    uint32_t next_copy = 0;
    std::vector<hipEvent_t> slot_ev;  // per slot: the last copy into it
    std::vector<uint8_t> has_ev;      // slot_ev recorded at least once
    std::vector<uint8_t> spec;        // filled by a speculative copy, not yet requested
    // Decode calls read only a native block's decode regions (its first
    // decode_bytes); while prefix_only is set (the decode path's own fetches)
    // a miss copies just those and marks the slot partial; any other use of
    // a partial slot copies the rest first.
    std::vector<uint8_t> partial;
    bool prefix_only = false;
    hipEvent_t gate = nullptr;        // compute-stream point that copies into reused slots wait for
    hipEvent_t cur_gate = nullptr;    // the gate recorded by the last real resolve (gate, or a ring entry)
    bool gate_recorded = false;
    bool speculate = false;
    bool spec_pending = false;
    uint32_t spec_layer = 0;
    uint64_t spec_requests = 0, spec_copies = 0, spec_hits = 0, bytes_h2d = 0;
    std::vector<std::pair<uint32_t, uint32_t>> resolved;  // last wl_cache_prefetch: key -> slot
    std::vector<uint8_t*> blk;  // the block of each slot (a file-backed cache swaps them, below)
    // packed-file backing (wl_cache_create_files): the reads run on its
    // workers; task_of[slot] is the slot's read not yet waited for
    std::unique_ptr<wl::FileTier> files;
    std::vector<wl::FileTask*> task_of;
    hipEvent_t gates[4] = {nullptr, nullptr, nullptr, nullptr};  // per-resolve gates of file reads (a ring)
    uint32_t gate_i = 0;
    // A file read lands in its slot as the file's record (reference layout):
    // raw[slot] until wl_cache_get converts it on the caller's stream into
    // `spare` and swaps the two blocks, so no kernel runs beside the caller's
    // persistent kernels. spare_ev: the last conversion out of the block
    // that is now the spare (the next conversion into it waits for it).
    std::vector<uint8_t> raw;
    uint8_t* spare = nullptr;
    hipEvent_t spare_ev = nullptr;
    bool spare_rec = false;
};

// Scratch of the batched layer: one allocation sized for `cap` tokens
// (wl_run_moe_batched), or the library's static device array
// (wl_run_moe_batched_noalloc). `last` holds the buffers and token count of
// the last chunk either path ran (read by the test hooks).
struct BatchScratch {
    uint32_t cap = 0;
    bool sh4 = false;  // sized with the MXFP4 shared expert's rows
    void* buf = nullptr;
    wl::BatchArgs b{};
    wl::BatchArgs last{};
    bool ran = false;
};

struct wl_ctx {
    wl_moe_config cfg{};
    wl_expert_layout lay{};
    size_t native_bytes = 0;
    size_t decode_bytes = 0;  // the decode kernel's regions of a native block (its first bytes)
    uint32_t SI = 0;
    int device = 0;
    int n_cu = 0;
    int32_t sched = WL_SCHED_FUSED;
    std::vector<LayerState> layers;
    std::vector<const uint8_t*> h_slot;   // [L*E]
    std::vector<uint32_t> n_bound;        // bound experts per layer
    const uint8_t** d_slot = nullptr;     // [L*E]
    wl::DecodeArgs* d_largs = nullptr;    // [L] per-layer kernel records
    // intermediates kept for inspection (ordinary device memory)
    float* norm = nullptr;
    float* logits = nullptr;
    float* smid = nullptr;
    float* rmid = nullptr;
    int32_t* idx = nullptr;
    float* topw = nullptr;
    float* shared_out = nullptr;
    uint16_t* ffn_mid_p = nullptr;  // wl_expert_ffn's SwiGLU pieces
    uint64_t* ffn_tag = nullptr;    // wl_expert_ffn's epoch-tagged SwiGLU values [I] (agent-scope exchange)
    int32_t taps = 1;
    // cross-work-group arrays (agent-scope stores and loads)
    uint64_t* lslot = nullptr;
    uint32_t* part = nullptr;
    uint32_t* tsh = nullptr;
    uint64_t* hx = nullptr;  // [H] a chain launch's layer outputs, epoch-tagged words
    uint32_t ptag = 0;  // the partials' tag of the last decode call: 1, 2, 3, 1, ...
    bool xl2 = false;   // two-level combine (per-XCD sums through the XCDs' L2s first)
    bool stale_partials = false;  // a phased call's combine launch failed after its first segment ran
    uint32_t* sync = nullptr;   // barrier words (uncached)
    wl::SyncMap sm{};
    wl::Plan plan{};
    uint32_t grid = 0;
    uint32_t epoch = 0;
    void* uc_block = nullptr;   // uncached scratch (returned to the process pool on destroy)
    size_t uc_bytes = 0;
    // context-owned slot pool
    uint8_t* pool = nullptr;
    uint32_t pool_slots = 0;
    std::vector<void*> allocs;
    std::string err;
    CacheState cache;
    BatchScratch batch;
    void* scratch = nullptr;  // this device's static scratch (wl_run_moe_batched_noalloc)
    bool any_sh4 = false;     // some layer has an MXFP4 shared expert (the batched scratch keeps its rows)
    // the expert source of layers with no expert bound (src.get null: none)
    wl_expert_source src{};
    bool src_cache = false;        // src is the built-in cache
    wl_status src_status = WL_OK;  // a failure the built-in cache's callbacks reported
    uint8_t* stage = nullptr;      // native staging blocks for a reference-layout source
    uint32_t stage_n = 0;
    int32_t* h_pin = nullptr;      // pinned host words, PinMap layout
    std::vector<int32_t> uniq;     // a batched chunk's routed experts (capacity E, reserved once)
    hipEvent_t ids_ev = nullptr, pred_ev = nullptr;
    // dense MLP layers: gate / up outputs [dense_cap] f32, and an all-ones
    // norm weight [H] bf16 for a layer bound without one
    float *dense_g = nullptr, *dense_u = nullptr;
    uint32_t dense_cap = 0;
    uint16_t* ones_ln = nullptr;
};

// Word offsets in wl_ctx::h_pin: routed ids, the abort word, predicted ids of
// the next layer (speculation), the batched layer's per-expert counts.
struct PinMap {
    static constexpr uint32_t ids = 0, abort = 32, pred = 40, counts = 96;
    static size_t bytes(uint32_t E) { return 4u * ((size_t)counts + E); }
};

namespace {

wl_status fail(wl_ctx* c, wl_status s, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
wl_status fail(wl_ctx* c, wl_status s, const char* fmt, ...) {
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return s;
}

wl_status hip_fail(wl_ctx* c, hipError_t e, const char* what) {
    return fail(c, WL_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

template <typename T>
wl_status dalloc(wl_ctx* c, T** p, size_t bytes) {
    void* q = nullptr;
    hipError_t e = hipMalloc(&q, bytes ? bytes : 16);
    if (e != hipSuccess) return fail(c, WL_ERR_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    c->allocs.push_back(q);
    *p = (T*)q;
    return WL_OK;
}

// Uncached device memory is never returned to the runtime while the process
// lives (freeing it after a kernel has read it has corrupted later allocations
// on this platform); blocks of destroyed contexts are kept here for reuse.
struct UcBlock { int device; size_t bytes; void* ptr; };
std::mutex g_uc_mu;
std::vector<UcBlock> g_uc_free;

void* uc_acquire(int device, size_t bytes) {
    {
        std::lock_guard<std::mutex> lk(g_uc_mu);
        for (size_t i = 0; i < g_uc_free.size(); i++) {
            if (g_uc_free[i].device == device && g_uc_free[i].bytes >= bytes) {
                void* p = g_uc_free[i].ptr;
                g_uc_free.erase(g_uc_free.begin() + i);
                return p;
            }
        }
    }
    void* p = nullptr;
    if (hipExtMallocWithFlags(&p, bytes, hipDeviceMallocUncached) != hipSuccess) return nullptr;
    return p;
}

void uc_release(int device, size_t bytes, void* p) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(g_uc_mu);
    g_uc_free.push_back({device, bytes, p});
}

wl_status validate_cfg(const wl_moe_config* cfg, wl_ctx* c) {
    if (!cfg) return fail(c, WL_ERR_INVALID, "config is null");
    const uint32_t H = cfg->hidden, I = cfg->moe_inter, E = cfg->n_routed_experts,
                   K = cfg->n_experts_per_tok;
    if (H == 0 || H % 128) return fail(c, WL_ERR_INVALID, "hidden=%u must be a positive multiple of 128", H);
    if (I == 0 || I % 128) return fail(c, WL_ERR_INVALID, "moe_inter=%u must be a positive multiple of 128", I);
    if ((uint64_t)I * cfg->n_shared > 65536) return fail(c, WL_ERR_INVALID, "shared inter %u too large", I * cfg->n_shared);
    if (E == 0 || E % 16 || E > 4096) return fail(c, WL_ERR_INVALID, "n_routed_experts=%u must be a multiple of 16 in [16,4096]", E);
    if (K == 0 || K > WL_MAX_TOPK || K > E) return fail(c, WL_ERR_INVALID, "n_experts_per_tok=%u must be in [1,min(%d,E)]", K, WL_MAX_TOPK);
    if (cfg->n_shared == 0 || cfg->n_shared > 16) return fail(c, WL_ERR_INVALID, "n_shared=%u must be in [1,16]", cfg->n_shared);
    if (cfg->n_layers == 0 || cfg->n_layers > 4096) return fail(c, WL_ERR_INVALID, "n_layers=%u must be in [1,4096]", cfg->n_layers);
    if (H > 8192) return fail(c, WL_ERR_INVALID, "hidden=%u exceeds 8192", H);
    return WL_OK;
}

// The device-side launch record of one layer: its weights, its slot table
// row, the context scratch and the shapes.
wl::DecodeArgs layer_record(const wl_ctx* c, uint32_t layer) {
    const LayerState& L = c->layers[layer];
    const uint32_t H = c->cfg.hidden, E = c->cfg.n_routed_experts, SI = c->SI;
    wl::DecodeArgs a{};
    a.ln_w = L.ln;
    a.router_w = L.router_w;
    a.bias = L.bias;
    a.sh_native = L.shared;
    a.slot_tab = c->d_slot + (size_t)layer * E;
    a.norm = c->norm;
    a.logits = c->logits;
    a.smid = c->smid;
    a.rmid = c->rmid;
    a.idx = c->idx;
    a.topw = c->topw;
    a.shared_out = c->shared_out;
    a.lslot = c->lslot;
    a.part = c->part;
    a.tsh = c->tsh;
    a.sync = c->sync;
    a.H = H;
    a.I = c->cfg.moe_inter;
    a.E = E;
    a.K = c->cfg.n_experts_per_tok;
    a.SI = SI;
    a.eps = c->cfg.rms_eps;
    a.scaling = c->cfg.routed_scaling;
    a.norm_topk = c->cfg.norm_topk_prob ? 1 : 0;
    return a;
}

}  // namespace

extern "C" {

wl_status wl_expert_layout_of(const wl_moe_config* cfg, uint32_t inter, wl_expert_layout* out) {
    if (!cfg || !out) return WL_ERR_INVALID;
    const size_t H = cfg->hidden, I = inter ? inter : cfg->moe_inter;
    if (H % 32 || I % 32) return WL_ERR_INVALID;
    wl_expert_layout l{};
    size_t o = 0;
    l.gw_off = o; l.gw_len = I * H / 2;  o += l.gw_len;
    l.gs_off = o; l.gs_len = I * H / 32; o += l.gs_len;
    l.uw_off = o; l.uw_len = I * H / 2;  o += l.uw_len;
    l.us_off = o; l.us_len = I * H / 32; o += l.us_len;
    l.dw_off = o; l.dw_len = H * I / 2;  o += l.dw_len;
    l.ds_off = o; l.ds_len = H * I / 32; o += l.ds_len;
    l.total = o;
    *out = l;
    return WL_OK;
}

wl_status wl_create(const wl_moe_config* cfg, wl_ctx** out) {
    if (!out) return WL_ERR_INVALID;
    *out = nullptr;
    wl_status s = validate_cfg(cfg, nullptr);
    if (s != WL_OK) return s;
    wl_ctx* c = new wl_ctx();
    c->cfg = *cfg;
    c->SI = cfg->moe_inter * cfg->n_shared;
    wl_expert_layout_of(cfg, 0, &c->lay);
    c->native_bytes = wl::NativeLayout::make(cfg->hidden, cfg->moe_inter).total;
    c->decode_bytes = wl::NativeLayout::make(cfg->hidden, cfg->moe_inter).bgus;
    hipError_t e = hipGetDevice(&c->device);
    if (e != hipSuccess) { delete c; return WL_ERR_HIP; }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, c->device);
    if (e != hipSuccess) { delete c; return WL_ERR_HIP; }
    c->n_cu = prop.multiProcessorCount;
    const uint32_t H = cfg->hidden, I = cfg->moe_inter, E = cfg->n_routed_experts,
                   K = cfg->n_experts_per_tok, L = cfg->n_layers, SI = c->SI;
    // one work-group per CU, a multiple of 8 so every XCD holds the same
    // number. Work-groups of one launch wait for each other's data (logits,
    // partial sums), so all of them must be resident at once: checked below
    // against the occupancy the kernels' LDS and register use allow.
    uint32_t grid = (uint32_t)c->n_cu;
    if (const char* env = getenv("WL_DECODE_GRID")) {
        const int gv = atoi(env);
        if (gv > 0 && gv < (int)grid) grid = (uint32_t)gv;
    }
    if (grid > wl::kMaxGrid) grid = wl::kMaxGrid;
    if (grid >= 16) grid &= ~7u;
    c->grid = grid;
    c->plan = wl::Plan::make(H, I, SI, K, grid);
    const wl::LdsMap lm = wl::LdsMap::make(H, SI, E, K, c->plan);
    if ((int)lm.bytes > wl::decode_max_lds()) {
        delete c;
        return WL_ERR_INVALID;
    }
    {
        int per_cu_decode = 0, per_cu_route = 0;
        if (wl::decode_occupancy(H, I, SI, E, K, grid, &per_cu_decode) != 0 ||
            wl::route_occupancy(H, E, &per_cu_route) != 0) {
            delete c;
            return WL_ERR_HIP;
        }
        if ((uint64_t)per_cu_decode * (uint64_t)c->n_cu < grid || (uint64_t)per_cu_route * (uint64_t)c->n_cu < grid) {
            delete c;
            return WL_ERR_INVALID;  // the grid could not be co-resident
        }
    }

    c->layers.resize(L);
    c->h_slot.assign((size_t)L * E, nullptr);
    c->n_bound.assign(L, 0);
    c->sm = wl::SyncMap::make();
    if ((s = dalloc(c, &c->d_slot, sizeof(void*) * (size_t)L * E)) != WL_OK ||
        (s = dalloc(c, &c->d_largs, sizeof(wl::DecodeArgs) * (size_t)L)) != WL_OK ||
        (s = dalloc(c, &c->norm, 4 * (size_t)H)) != WL_OK ||
        (s = dalloc(c, &c->smid, 4 * (size_t)SI)) != WL_OK ||
        (s = dalloc(c, &c->rmid, 4 * (size_t)K * I)) != WL_OK ||
        (s = dalloc(c, &c->idx, 4 * (size_t)WL_MAX_TOPK)) != WL_OK ||
        (s = dalloc(c, &c->topw, 4 * (size_t)WL_MAX_TOPK)) != WL_OK ||
        (s = dalloc(c, &c->shared_out, 4 * (size_t)H)) != WL_OK ||
        (s = dalloc(c, &c->ffn_mid_p, 2 * 3 * (size_t)I)) != WL_OK ||
        (s = dalloc(c, &c->ffn_tag, 8 * (size_t)I)) != WL_OK ||
        (s = dalloc(c, &c->logits, 4 * (size_t)E)) != WL_OK ||
        (s = dalloc(c, &c->lslot, 8 * (size_t)E)) != WL_OK ||
        (s = dalloc(c, &c->part, 4 * wl::part_words(H, grid))) != WL_OK ||
        (s = dalloc(c, &c->tsh, 4 * wl::part_words(H, grid))) != WL_OK ||
        (s = dalloc(c, &c->hx, 8 * (size_t)H)) != WL_OK) {
        wl_destroy(c);
        return s;
    }
    // the uncached block holds only the barrier words
    c->uc_bytes = 4 * (size_t)c->sm.words;
    c->uc_block = uc_acquire(c->device, c->uc_bytes);
    if (!c->uc_block) {
        wl_destroy(c);
        return WL_ERR_OOM;
    }
    c->sync = (uint32_t*)c->uc_block;
    // the static scratch of this device (wl_run_moe_batched_noalloc), looked
    // up once per device, with the device current, at set-up
    if (wl::noalloc_scratch(c->device, &c->scratch) != 0) {
        wl_destroy(c);
        return WL_ERR_HIP;
    }

    e = hipMemset(c->d_slot, 0, sizeof(void*) * (size_t)L * E);
    // records of layers not yet bound are zero, not stale bytes
    if (e == hipSuccess) e = hipMemset(c->d_largs, 0, sizeof(wl::DecodeArgs) * (size_t)L);
    // epoch 0 is never a call's: zeroed tagged arrays hold no valid word (a
    // reused allocation could otherwise carry another context's tags)
    if (e == hipSuccess) e = hipMemset(c->lslot, 0, 8 * (size_t)E);
    if (e == hipSuccess) e = hipMemset(c->ffn_tag, 0, 8 * (size_t)I);
    // tag 0 is never a call's either
    if (e == hipSuccess) e = hipMemset(c->part, 0, 4 * wl::part_words(H, grid));
    if (e == hipSuccess) e = hipMemset(c->tsh, 0, 4 * wl::part_words(H, grid));
    if (e == hipSuccess) e = hipMemset(c->hx, 0, 8 * (size_t)H);
    if (e == hipSuccess) e = hipMemset(c->uc_block, 0, c->uc_bytes);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) { wl_destroy(c); return WL_ERR_HIP; }
    // The two-level combine (WL_DECODE_XL2=1; off by default: at config 1
    // its per-XCD first level takes as much time as it saves, see the
    // kernel) needs work-group w on XCD w mod 8 (the dispatcher's round
    // robin), checked here once with a probe launch of the decode grid and
    // by every decode launch (E_XCD).
    {
        const char* env = getenv("WL_DECODE_XL2");
        bool map_ok = false;
        if (grid >= 8 && grid % 8 == 0 && env && env[0] == '1' && wl::probe_xcd_map(grid, &map_ok) == 0)
            c->xl2 = map_ok;
    }
    *out = c;
    return WL_OK;
}

void wl_destroy(wl_ctx* c) {
    if (!c) return;
    // the file tier's workers first: a read still queued records the slot's
    // event and writes into the pool, so they are joined (and their streams
    // drained) before any event, stream or buffer goes
    c->cache.files.reset();
    if (c->uc_block || c->cache.lru) (void)hipDeviceSynchronize();
    {
        CacheState& C = c->cache;
        for (hipEvent_t e : C.slot_ev) (void)hipEventDestroy(e);
        if (C.gate) (void)hipEventDestroy(C.gate);
        for (hipEvent_t e : C.gates)
            if (e) (void)hipEventDestroy(e);
        if (C.spare_ev) (void)hipEventDestroy(C.spare_ev);
        for (hipStream_t st : C.copy)
            if (st) (void)hipStreamDestroy(st);
        delete C.lru;
    }
    if (c->batch.buf) (void)hipFree(c->batch.buf);
    if (c->stage) (void)hipFree(c->stage);
    for (LayerState& L : c->layers)
        for (void* p : L.owned) (void)hipFree(p);
    if (c->h_pin) (void)hipHostFree(c->h_pin);
    for (hipEvent_t e : {c->ids_ev, c->pred_ev})
        if (e) (void)hipEventDestroy(e);
    for (void* p : c->allocs) (void)hipFree(p);
    uc_release(c->device, c->uc_bytes, c->uc_block);
    delete c;
}

const char* wl_last_error(const wl_ctx* c) { return c ? c->err.c_str() : "null context"; }

// Binds a layer's router, bias and norm, and converts its shared expert into
// context-owned memory: bf16 (NativeShared) from `bf16`, or MXFP4
// (NativeShared4) from the six reference tensors `parts` (gate_w, gate_s,
// up_w, up_s, down_w, down_s).
static wl_status set_layer_checked(wl_ctx* c, uint32_t layer, const uint16_t* d_router_w, const float* d_router_bias,
                                   const uint16_t* d_post_attn_ln, const uint16_t* bf16, const uint8_t* const* parts,
                                   std::vector<void*>& take) {
    if (layer >= c->cfg.n_layers) return fail(c, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, c->cfg.n_layers);
    if (!d_router_w || !d_router_bias) return fail(c, WL_ERR_INVALID, "router weight and router bias are required");
    const uint32_t H = c->cfg.hidden, SI = c->SI;
    if (parts) {
        if (c->cfg.n_shared != 1)
            return fail(c, WL_ERR_INVALID, "an MXFP4 shared expert needs n_shared = 1 (inter %u), not %u",
                        c->cfg.moe_inter, c->cfg.n_shared);
        for (int r = 0; r < 6; r++)
            if (!parts[r]) return fail(c, WL_ERR_INVALID, "MXFP4 shared expert tensor %d is null", r);
    } else if (!bf16) {
        return fail(c, WL_ERR_INVALID, "the shared expert is required");
    }
    LayerState& L = c->layers[layer];
    const size_t need = parts ? wl::NativeShared4::make(H, SI).total : wl::NativeShared::make(H, SI).total;
    if (L.shared_bytes < need) {
        // a buffer too small for the new format stays owned by the context until it is destroyed
        wl_status st = dalloc(c, &L.shared, need);
        if (st != WL_OK) return st;
        L.shared_bytes = need;
    }
    const int le = parts ? wl::launch_shared4_to_native(parts, L.shared, H, SI, nullptr)
                         : wl::launch_shared_to_native(bf16, (uint16_t*)L.shared, H, SI, nullptr);
    if (le != 0) return fail(c, WL_ERR_HIP, "shared expert conversion launch failed");
    hipError_t se = hipDeviceSynchronize();
    if (se != hipSuccess) return hip_fail(c, se, "shared expert conversion");
    L.router_w = d_router_w;
    L.bias = d_router_bias;
    L.ln = d_post_attn_ln;
    L.shared_dtype = parts ? WL_SHARED_MXFP4 : WL_SHARED_BF16;
    L.dense = false;
    if (parts) c->any_sh4 = true;
    const wl::DecodeArgs a = layer_record(c, layer);
    hipError_t e = hipMemcpy(c->d_largs + layer, &a, sizeof(a), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(c, e, "layer record upload");
    L.set = true;
    // the device was synchronised above: no kernel still reads the buffers the layer used before
    for (void* p : L.owned) (void)hipFree(p);
    L.owned.clear();
    L.owned.swap(take);  // take is left empty: the caller frees nothing
    return WL_OK;
}

// set_layer_checked with the buffers in `take` (router, bias, norm) handed to
// the context: kept by the layer on success, freed on failure.
static wl_status set_layer(wl_ctx* c, uint32_t layer, const uint16_t* d_router_w, const float* d_router_bias,
                           const uint16_t* d_post_attn_ln, const uint16_t* bf16, const uint8_t* const* parts,
                           std::vector<void*> take = {}) {
    wl_status st = c ? set_layer_checked(c, layer, d_router_w, d_router_bias, d_post_attn_ln, bf16, parts, take)
                     : WL_ERR_INVALID;
    for (void* p : take) (void)hipFree(p);  // empty after a success
    return st;
}

wl_status wl_set_layer(wl_ctx* c, uint32_t layer, const uint16_t* d_router_w, const float* d_router_bias,
                       const uint16_t* d_post_attn_ln, const void* d_shared, int32_t shared_dtype) {
    if (!c) return WL_ERR_INVALID;
    if (!d_shared) return fail(c, WL_ERR_INVALID, "the shared expert is required");
    if (shared_dtype == WL_SHARED_BF16)
        return set_layer(c, layer, d_router_w, d_router_bias, d_post_attn_ln, (const uint16_t*)d_shared, nullptr);
    if (shared_dtype != WL_SHARED_MXFP4) return fail(c, WL_ERR_INVALID, "unknown shared_dtype %d", shared_dtype);
    wl_expert_layout l;
    if (wl_expert_layout_of(&c->cfg, c->SI, &l) != WL_OK) return fail(c, WL_ERR_INVALID, "shared expert layout");
    const uint8_t* b = (const uint8_t*)d_shared;
    const uint8_t* parts[6] = {b + l.gw_off, b + l.gs_off, b + l.uw_off, b + l.us_off, b + l.dw_off, b + l.ds_off};
    return set_layer(c, layer, d_router_w, d_router_bias, d_post_attn_ln, nullptr, parts);
}

wl_status wl_set_layer_mxfp4(wl_ctx* c, uint32_t layer, const uint16_t* d_router_w, const float* d_router_bias,
                             const uint16_t* d_post_attn_ln, const uint8_t* d_sh_gate_w, const uint8_t* d_sh_gate_s,
                             const uint8_t* d_sh_up_w, const uint8_t* d_sh_up_s, const uint8_t* d_sh_down_w,
                             const uint8_t* d_sh_down_s) {
    const uint8_t* parts[6] = {d_sh_gate_w, d_sh_gate_s, d_sh_up_w, d_sh_up_s, d_sh_down_w, d_sh_down_s};
    return set_layer(c, layer, d_router_w, d_router_bias, d_post_attn_ln, nullptr, parts);
}

wl_status wl_set_layer_dense(wl_ctx* c, uint32_t layer, const uint16_t* d_post_ln, const uint16_t* d_gate,
                             const uint16_t* d_up, const uint16_t* d_down, uint32_t dense_inter) {
    if (!c) return WL_ERR_INVALID;
    if (layer >= c->cfg.n_layers) return fail(c, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, c->cfg.n_layers);
    if (!d_gate || !d_up || !d_down) return fail(c, WL_ERR_INVALID, "gate, up and down are required");
    if (dense_inter == 0 || dense_inter % 8 || dense_inter > 16384)
        return fail(c, WL_ERR_INVALID, "dense_inter=%u must be a positive multiple of 8, at most 16384", dense_inter);
    if (((uintptr_t)d_gate | (uintptr_t)d_up | (uintptr_t)d_down | (uintptr_t)d_post_ln) % 16)
        return fail(c, WL_ERR_INVALID, "dense MLP tensors must be 16-byte aligned");
    const uint32_t H = c->cfg.hidden;
    // no kernel may still read what the layer held before (owned router /
    // bias / norm copies, or the dense scratch being replaced)
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(c, e, "dense layer bind");
    if (dense_inter > c->dense_cap) {
        wl_status st;
        if ((st = dalloc(c, &c->dense_g, 4 * (size_t)dense_inter)) != WL_OK ||
            (st = dalloc(c, &c->dense_u, 4 * (size_t)dense_inter)) != WL_OK)
            return st;  // a smaller pair stays owned by the context until it is destroyed
        c->dense_cap = dense_inter;
    }
    if (!d_post_ln && !c->ones_ln) {
        wl_status st = dalloc(c, &c->ones_ln, 2 * (size_t)H);
        if (st != WL_OK) return st;
        const std::vector<uint16_t> ones(H, 0x3F80u);  // bf16 1.0
        if ((e = hipMemcpy(c->ones_ln, ones.data(), 2 * (size_t)H, hipMemcpyHostToDevice)) != hipSuccess)
            return hip_fail(c, e, "norm weight upload");
    }
    LayerState& L = c->layers[layer];
    for (void* p : L.owned) (void)hipFree(p);
    L.owned.clear();
    L.router_w = nullptr;
    L.bias = nullptr;
    L.ln = d_post_ln ? d_post_ln : c->ones_ln;
    L.mlp_gate = d_gate;
    L.mlp_up = d_up;
    L.mlp_down = d_down;
    L.dense_inter = dense_inter;
    L.dense = true;
    L.set = true;
    return WL_OK;
}

}  // extern "C"

namespace wl {

const wl_moe_config& ctx_config(const wl_ctx* c) { return c->cfg; }
uint32_t ctx_shared_inter(const wl_ctx* c) { return c->SI; }

wl_status ctx_fail(wl_ctx* c, wl_status s, const std::string& msg) { return fail(c, s, "%s", msg.c_str()); }

wl_status ctx_set_layer_owned(wl_ctx* c, uint32_t layer, uint16_t* router_w, float* bias, uint16_t* ln,
                              const uint16_t* bf16_shared, const uint8_t* const* mxfp4_parts) {
    return set_layer(c, layer, router_w, bias, ln, bf16_shared, mxfp4_parts, {router_w, bias, ln});
}

}  // namespace wl

extern "C" {

wl_status wl_slot_bind(wl_ctx* c, uint32_t layer, uint32_t expert, const uint8_t* d_block) {
    if (!c) return WL_ERR_INVALID;
    if (layer >= c->cfg.n_layers || expert >= c->cfg.n_routed_experts)
        return fail(c, WL_ERR_INVALID, "slot (%u,%u) out of range", layer, expert);
    if (!d_block) return fail(c, WL_ERR_INVALID, "null block for (%u,%u)", layer, expert);
    const size_t i = (size_t)layer * c->cfg.n_routed_experts + expert;
    if (!c->h_slot[i]) c->n_bound[layer]++;
    c->h_slot[i] = d_block;
    hipError_t e = hipMemcpy(c->d_slot + i, &c->h_slot[i], sizeof(void*), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(c, e, "slot table update");
    return WL_OK;
}

wl_status wl_slot_unbind(wl_ctx* c, uint32_t layer, uint32_t expert) {
    if (!c) return WL_ERR_INVALID;
    if (layer >= c->cfg.n_layers || expert >= c->cfg.n_routed_experts)
        return fail(c, WL_ERR_INVALID, "slot (%u,%u) out of range", layer, expert);
    const size_t i = (size_t)layer * c->cfg.n_routed_experts + expert;
    if (c->h_slot[i]) c->n_bound[layer]--;
    c->h_slot[i] = nullptr;
    hipError_t e = hipMemcpy(c->d_slot + i, &c->h_slot[i], sizeof(void*), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(c, e, "slot table update");
    return WL_OK;
}

wl_status wl_slot_pool_create(wl_ctx* c, uint32_t n_slots) {
    if (!c) return WL_ERR_INVALID;
    if (c->pool) return fail(c, WL_ERR_STATE, "slot pool already created");
    if (n_slots == 0) return fail(c, WL_ERR_INVALID, "n_slots must be positive");
    const size_t bytes = (size_t)n_slots * c->native_bytes;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(c, WL_ERR_OOM, "slot pool of %u x %zu B: %s", n_slots, c->native_bytes, hipGetErrorString(e));
    c->allocs.push_back(p);
    c->pool = (uint8_t*)p;
    c->pool_slots = n_slots;
    return WL_OK;
}

wl_status wl_slot_pool_ptr(wl_ctx* c, uint32_t slot, uint8_t** d_block) {
    if (!c || !d_block) return WL_ERR_INVALID;
    if (!c->pool) return fail(c, WL_ERR_STATE, "no slot pool");
    if (slot >= c->pool_slots) return fail(c, WL_ERR_INVALID, "slot %u >= %u", slot, c->pool_slots);
    *d_block = c->pool + (size_t)slot * c->native_bytes;
    return WL_OK;
}

// ---- expert cache ------------------------------------------------------------
// Resolves n ids of `layer`: hits bump the LRU, misses take a slot (evicting
// the least-recent key) and start a host-to-device copy on a side stream that
// waits for the last gate (so no kernel enqueued before it still reads the
// reused slot) and for the slot's previous copy. Real requests order `s`
// after the copy of their slot; speculative ones only start copies (their
// victims are never among the last real batch's experts: capacity >= 2K).
static wl_status cache_resolve(wl_ctx* c, uint32_t layer, const int32_t* ids, uint32_t n, hipStream_t s,
                               bool speculative, uint32_t* slots) {
    CacheState& C = c->cache;
    const uint32_t E = c->cfg.n_routed_experts;
    const size_t nb = c->native_bytes;
    hipError_t e;
    if (!speculative) {
        hipEvent_t g = C.gate;
        if (C.files) {  // file reads wait on a ring of gates (a read issued late waits for its own resolve)
            C.gate_i = (C.gate_i + 1) % 4u;
            g = C.gates[C.gate_i];
        }
        if ((e = hipEventRecord(g, s)) != hipSuccess) return hip_fail(c, e, "cache gate");
        C.cur_gate = g;
        C.gate_recorded = true;
    }
    C.lru->begin_batch();  // no key of this batch is evicted by another of it
    for (uint32_t k = 0; k < n; k++) {
        if (ids[k] < 0 || (uint32_t)ids[k] >= E)
            return fail(c, WL_ERR_INVALID, "expert id %d of layer %u out of range", ids[k], layer);
        bool dup = false;
        for (uint32_t j = 0; j < k; j++)
            if (ids[j] == ids[k]) {
                dup = true;
                if (slots) slots[k] = slots[j];
            }
        if (dup) continue;
        const uint32_t key = layer * E + (uint32_t)ids[k];
        const wl::SlotLru::Result r = C.lru->request(key, !speculative);
        uint8_t* dst = C.blk[r.slot];
        if (r.transient) {
            if (speculative) continue;  // a prediction the policy would not retain: nothing to fetch early
            if (!C.transient) return fail(c, WL_ERR_STATE, "no transient slot for a miss that is not retained");
            C.bypassed++;
        }
        if (r.evicted) {  // a block wl_cache_get could still hand out is gone
            auto& R = C.resolved;
            R.erase(std::remove_if(R.begin(), R.end(), [&](const auto& x) { return x.first == r.evicted_key; }), R.end());
        }
        if (speculative) C.spec_requests++;
        if (r.hit) {
            if (!speculative && C.spec[r.slot]) {
                C.spec_hits++;
                C.spec[r.slot] = 0;
            }
            if (C.partial[r.slot] && !C.prefix_only && !speculative) {  // the rest of the block
                const uint8_t* src = C.fn(C.user, layer, (uint32_t)ids[k]);
                if (!src) return fail(c, WL_ERR_IO, "no host block for layer %u expert %d", layer, ids[k]);
                hipStream_t cs = C.copy[C.next_copy++ & 1u];
                const size_t db = c->decode_bytes;
                if (C.gate_recorded && (e = hipStreamWaitEvent(cs, C.cur_gate, 0)) != hipSuccess)
                    return hip_fail(c, e, "copy gate");
                if (C.has_ev[r.slot] && (e = hipStreamWaitEvent(cs, C.slot_ev[r.slot], 0)) != hipSuccess)
                    return hip_fail(c, e, "slot order");
                if ((e = hipMemcpyAsync(dst + db, src + db, nb - db, hipMemcpyHostToDevice, cs)) != hipSuccess)
                    return hip_fail(c, e, "expert copy");
                if ((e = hipEventRecord(C.slot_ev[r.slot], cs)) != hipSuccess) return hip_fail(c, e, "copy event");
                C.has_ev[r.slot] = 1;
                C.partial[r.slot] = 0;
                C.bytes_h2d += nb - db;
            }
        } else if (C.files) {
            // a read still pending on this slot (its key was evicted before it
            // was waited for) lands first
            if (wl::FileTask* old = C.task_of[r.slot]) {
                const bool ok = C.files->wait_issued(old);
                const std::string why = old->why;
                C.files->release(old);
                C.task_of[r.slot] = nullptr;
                if (!ok) {
                    C.lru->forget(key);
                    return fail(c, WL_ERR_IO, "an earlier read into slot %u failed: %s", r.slot, why.c_str());
                }
            }
            wl::FileTask* t = C.files->submit(layer, (uint32_t)ids[k], dst, C.gate_recorded ? C.cur_gate : nullptr,
                                              C.slot_ev[r.slot]);
            if (!t) {  // every task in flight: release the issued ones and retry once
                for (wl::FileTask*& q : C.task_of)
                    if (q && q->issued.load()) {
                        C.files->wait_issued(q);
                        C.files->release(q);
                        q = nullptr;
                    }
                t = C.files->submit(layer, (uint32_t)ids[k], dst, C.gate_recorded ? C.cur_gate : nullptr,
                                    C.slot_ev[r.slot]);
            }
            if (!t) {
                C.lru->forget(key);
                return fail(c, WL_ERR_STATE, "file read queue full");
            }
            C.task_of[r.slot] = t;
            C.raw[r.slot] = 1;
            C.partial[r.slot] = 0;  // the conversion writes the whole native block
            C.has_ev[r.slot] = 1;
            C.spec[r.slot] = speculative ? 1 : 0;
            C.bytes_h2d += C.files->ref_bytes();
            if (speculative) C.spec_copies++;
        } else {
            const uint8_t* src = C.fn(C.user, layer, (uint32_t)ids[k]);
            if (!src) {
                C.lru->forget(key);
                return fail(c, WL_ERR_IO, "no host block for layer %u expert %d", layer, ids[k]);
            }
            hipStream_t cs = C.copy[C.next_copy++ & 1u];
            if (C.gate_recorded && (e = hipStreamWaitEvent(cs, C.cur_gate, 0)) != hipSuccess) return hip_fail(c, e, "copy gate");
            if (C.has_ev[r.slot] && (e = hipStreamWaitEvent(cs, C.slot_ev[r.slot], 0)) != hipSuccess)
                return hip_fail(c, e, "slot order");
            const bool part = C.prefix_only || speculative;  // speculation runs for decode only
            const size_t n_copy = part ? c->decode_bytes : nb;
            if ((e = hipMemcpyAsync(dst, src, n_copy, hipMemcpyHostToDevice, cs)) != hipSuccess)
                return hip_fail(c, e, "expert copy");
            if ((e = hipEventRecord(C.slot_ev[r.slot], cs)) != hipSuccess) return hip_fail(c, e, "copy event");
            C.has_ev[r.slot] = 1;
            C.spec[r.slot] = speculative ? 1 : 0;
            C.partial[r.slot] = part ? 1 : 0;
            C.bytes_h2d += n_copy;
            if (speculative) C.spec_copies++;
        }
        // (file reads: the stream waits in wl_cache_get, once the read is issued)
        if (!speculative && !C.files && C.has_ev[r.slot] && (e = hipStreamWaitEvent(s, C.slot_ev[r.slot], 0)) != hipSuccess)
            return hip_fail(c, e, "wait for expert copy");
        if (slots) slots[k] = r.slot;
    }
    return WL_OK;
}

// The pinned words and events of the source path (allocated once).
static wl_status ensure_pin(wl_ctx* c) {
    hipError_t e;
    if (!c->h_pin && (e = hipHostMalloc((void**)&c->h_pin, PinMap::bytes(c->cfg.n_routed_experts),
                                        hipHostMallocDefault)) != hipSuccess) {
        c->h_pin = nullptr;
        return fail(c, WL_ERR_OOM, "pinned id buffer: %s", hipGetErrorString(e));
    }
    for (hipEvent_t* ev : {&c->ids_ev, &c->pred_ev})
        if (!*ev && (e = hipEventCreateWithFlags(ev, hipEventDisableTiming)) != hipSuccess) {
            *ev = nullptr;
            return hip_fail(c, e, "source event");
        }
    c->uniq.reserve(c->cfg.n_routed_experts);
    return WL_OK;
}

// At least n native staging blocks for a reference-layout source (growing
// synchronises the device: blocks in use by queued work are freed).
static wl_status ensure_stage(wl_ctx* c, uint32_t n) {
    if (n <= c->stage_n) return WL_OK;
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(c, e, "staging resize");
    if (c->stage) (void)hipFree(c->stage);
    c->stage = nullptr;
    c->stage_n = 0;
    void* p = nullptr;
    if ((e = hipMalloc(&p, (size_t)n * c->native_bytes)) != hipSuccess)
        return fail(c, WL_ERR_OOM, "%u staging blocks: %s", n, hipGetErrorString(e));
    c->stage = (uint8_t*)p;
    c->stage_n = n;
    return WL_OK;
}

// The blocks of n experts of `layer` through the source: get_async (or get)
// each, in order; a reference-layout block is converted on `s` into staging
// block k. ptrs[k] = the native block of ids[k].
static wl_status source_fetch(wl_ctx* c, uint32_t layer, const int32_t* ids, uint32_t n, hipStream_t s,
                              const uint8_t** ptrs) {
    const wl_expert_source& S = c->src;
    if (!S.native && n > c->stage_n) return fail(c, WL_ERR_STATE, "%u staging blocks for %u experts", c->stage_n, n);
    for (uint32_t k = 0; k < n; k++) {
        c->src_status = WL_OK;
        const uint8_t* p = S.get_async ? S.get_async(S.user, layer, (uint32_t)ids[k], (void*)s)
                                       : S.get(S.user, layer, (uint32_t)ids[k]);
        if (!p) {
            if (c->src_status != WL_OK) return c->src_status;
            return fail(c, WL_ERR_IO, "expert source returned no block for layer %u expert %d", layer, ids[k]);
        }
        ptrs[k] = p;
    }
    if (S.native) return WL_OK;
    // every block of the call is valid until the call's work has run (the
    // source contract), so all n convert in one launch (16 per launch)
    uint8_t* dst[64];
    for (uint32_t k0 = 0; k0 < n; k0 += 64) {
        const uint32_t m = std::min(64u, n - k0);
        for (uint32_t k = 0; k < m; k++) dst[k] = c->stage + (size_t)(k0 + k) * c->native_bytes;
        if (wl::launch_experts_to_native(ptrs + k0, dst, m, c->cfg.hidden, c->cfg.moe_inter, s) != 0)
            return fail(c, WL_ERR_HIP, "expert conversion launch failed");
        for (uint32_t k = 0; k < m; k++) ptrs[k0 + k] = dst[k];
    }
    return WL_OK;
}

// Announces n experts of `layer` to the source (its prefetch, if any).
static wl_status source_prefetch(wl_ctx* c, uint32_t layer, const int32_t* ids, uint32_t n, hipStream_t s) {
    if (!c->src.prefetch) return WL_OK;
    c->src_status = WL_OK;
    c->src.prefetch(c->src.user, layer, ids, n, (void*)s);
    return c->src_status;
}

// A layer with no expert bound, through the expert source (run_moe's pattern,
// src/glm_layer_runner.cuh:391-418): route it on the device, read its ids back
// (the reference's one host round trip per layer), announce them, fetch each
// and fill the layer's slot table with the blocks (every other entry null, so
// a routing mismatch raises E_NOT_RESIDENT instead of reading a stale slot).
// With the built-in cache and speculation on, also routes layer `next` on the
// same input and copies its predicted ids back (resolved after the layer's
// launch, by cache_speculate).
static wl_status source_prepare(wl_ctx* c, uint32_t layer, const float* d_hidden, uint32_t next, hipStream_t s) {
    const uint32_t H = c->cfg.hidden, E = c->cfg.n_routed_experts, K = c->cfg.n_experts_per_tok;
    int32_t* pin = c->h_pin;
    hipError_t e;
    if (++c->epoch >= 0x7FFFFFFFu) c->epoch = 1;
    const uint32_t route_epoch = c->epoch;
    int le = wl::launch_route(c->d_largs + layer, d_hidden, route_epoch, H, E, c->grid, s);
    if (le != 0) return hip_fail(c, (hipError_t)le, "route launch");
    // the abort word names the last call that raised an error: only an error of
    // this routing launch fails this call (older ones stay for wl_check_error)
    if ((e = hipMemcpyAsync(pin + PinMap::ids, c->idx, 4 * (size_t)K, hipMemcpyDeviceToHost, s)) != hipSuccess ||
        (e = hipMemcpyAsync(pin + PinMap::abort, c->sync + c->sm.abort, 4, hipMemcpyDeviceToHost, s)) != hipSuccess ||
        (e = hipEventRecord(c->ids_ev, s)) != hipSuccess || (e = hipEventSynchronize(c->ids_ev)) != hipSuccess)
        return hip_fail(c, e, "routing read-back");
    if ((uint32_t)pin[PinMap::abort] == route_epoch)
        return fail(c, WL_ERR_DEVICE, "the routing kernel of layer %u reported an error (see wl_check_error)", layer);
    // the built-in cache copies only the decode regions of a missing block
    struct PrefixOnly {
        CacheState& C;
        PrefixOnly(CacheState& cs, bool on) : C(cs) { C.prefix_only = on; }
        ~PrefixOnly() { C.prefix_only = false; }
    } prefix_only(c->cache, c->src_cache);
    wl_status st = source_prefetch(c, layer, pin + PinMap::ids, K, s);
    if (st != WL_OK) return st;
    const uint8_t* ptrs[WL_MAX_TOPK];
    if ((st = source_fetch(c, layer, pin + PinMap::ids, K, s, ptrs)) != WL_OK) return st;
    le = wl::launch_slot_fill(c->d_slot + (size_t)layer * E, E, pin + PinMap::ids, ptrs, K, s);
    if (le != 0) return hip_fail(c, (hipError_t)le, "slot table fill");
    CacheState& C = c->cache;
    C.spec_pending = false;
    if (c->src_cache && C.speculate && next < c->cfg.n_layers && c->n_bound[next] == 0 && c->layers[next].set &&
        !c->layers[next].dense) {
        if (++c->epoch >= 0x7FFFFFFFu) c->epoch = 1;
        le = wl::launch_route(c->d_largs + next, d_hidden, c->epoch, H, E, c->grid, s);
        if (le != 0) return hip_fail(c, (hipError_t)le, "speculative route launch");
        if ((e = hipMemcpyAsync(pin + PinMap::pred, c->idx, 4 * (size_t)K, hipMemcpyDeviceToHost, s)) != hipSuccess ||
            (e = hipEventRecord(c->pred_ev, s)) != hipSuccess)
            return hip_fail(c, e, "prediction read-back");
        C.spec_pending = true;
        C.spec_layer = next;
    }
    return WL_OK;
}

static wl_status cache_speculate(wl_ctx* c, hipStream_t s) {
    CacheState& C = c->cache;
    if (!C.spec_pending) return WL_OK;
    C.spec_pending = false;
    hipError_t e = hipEventSynchronize(c->pred_ev);
    if (e != hipSuccess) return hip_fail(c, e, "prediction wait");
    return cache_resolve(c, C.spec_layer, c->h_pin + PinMap::pred, c->cfg.n_experts_per_tok, s, true, nullptr);
}

// A dense MLP layer (the dense branch of run_moe, src/glm_layer_runner.cuh:
// 373-384): out = resid + down(silu(gate x) * up x), x = RMSNorm(hidden), in
// two stream-ordered GEMV launches; the norm goes to the norm tap. d_out may
// alias d_hidden and d_resid exactly (launch_dense_mlp reads hidden in its
// first launch and each resid row before writing it).
static wl_status run_dense(wl_ctx* c, uint32_t layer, const float* d_hidden, const float* d_resid, float* d_out,
                           void* stream) {
    const LayerState& L = c->layers[layer];
    if (((uintptr_t)d_hidden | (uintptr_t)d_out | (uintptr_t)d_resid) % 16)
        return fail(c, WL_ERR_INVALID, "a dense layer's hidden, residual and output must be 16-byte aligned");
    const wl::attn::DenseMlp m{L.ln, L.mlp_gate, L.mlp_up, L.mlp_down, c->cfg.hidden, L.dense_inter,
                               c->cfg.rms_eps};
    const int e = wl::attn::launch_dense_mlp(m, d_hidden, d_resid, d_out, c->dense_g, c->dense_u, c->norm, nullptr,
                                             stream);
    if (e != 0) return hip_fail(c, (hipError_t)e, "dense MLP launch");
    return WL_OK;
}

// in_place: d_out == d_hidden == d_resid is allowed (h <- h + moe(h)): every
// work-group reads all of h for its norm before it publishes any partial, and
// a combine block is written only after every partial of it is in, so no
// read of h can see a written value.
static wl_status run_layer(wl_ctx* c, uint32_t layer, const float* d_hidden, const float* d_resid,
                           float* d_out, void* stream, uint32_t next = 0xFFFFFFFFu, bool in_place = false) {
    if (!c) return WL_ERR_INVALID;
    if (layer >= c->cfg.n_layers) return fail(c, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, c->cfg.n_layers);
    const LayerState& L = c->layers[layer];
    if (!L.set) return fail(c, WL_ERR_STATE, "layer %u has no weights (wl_set_layer)", layer);
    if (!d_hidden || !d_out) return fail(c, WL_ERR_INVALID, "null hidden/out");
    if (in_place ? (d_out != d_hidden || d_resid != d_hidden)
                 : (d_out == d_hidden || (d_resid && d_out == d_resid)))
        return fail(c, WL_ERR_INVALID, "d_out must not alias the inputs");
    if (L.dense) return run_dense(c, layer, d_hidden, d_resid, d_out, stream);
    {
        // Each decode launch carries a new epoch and partial tag from the
        // host; a captured launch replayed would reuse them and could take an
        // earlier call's logits or partials as this call's.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
            return fail(c, WL_ERR_STATE, "a MoE decode layer cannot be captured into a graph (per-call epochs)");
    }
    const uint32_t H = c->cfg.hidden, I = c->cfg.moe_inter, E = c->cfg.n_routed_experts,
                   K = c->cfg.n_experts_per_tok, SI = c->SI;
    const bool cached = c->n_bound[layer] == 0 && c->src.get != nullptr;
    if (!cached && c->n_bound[layer] != E)
        return fail(c, WL_ERR_NOT_RESIDENT, "layer %u has %u of %u experts bound%s", layer, c->n_bound[layer], E,
                    c->n_bound[layer] == 0 ? " and the context has no expert source" : "");
    if (cached) {
        wl_status s = source_prepare(c, layer, d_hidden, next, (hipStream_t)stream);
        if (s != WL_OK) return s;
    }

    wl::DecodeDyn dyn{};
    if (++c->epoch >= 0x7FFFFFFFu) c->epoch = 1;
    dyn.epoch = c->epoch;
    // per decode call (the routing launches also take epochs), so consecutive
    // calls' partials never share a tag. The tag is kept only once every
    // launch of the call is enqueued: a launch that fails enqueues nothing,
    // so the next call reuses the tag (the combine's ticket counter for it
    // was cleared by the last call that ran a combine).
    if (c->stale_partials) {
        // a segment-0 launch ran without its combine: its words carry a tag
        // the next calls will use, and the next tag's ticket was not cleared
        hipError_t e = hipDeviceSynchronize();
        if (e == hipSuccess) e = hipMemset(c->sync + c->sm.ticket, 0, 4 * 3);
        if (e == hipSuccess) e = hipMemset(c->part, 0, 4 * wl::part_words(H, c->grid));
        if (e == hipSuccess) e = hipMemset(c->tsh, 0, 4 * wl::part_words(H, c->grid));
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_fail(c, e, "partial-sum reset");
        c->stale_partials = false;
    }
    const uint32_t ptag = c->ptag % 3u + 1u;
    dyn.hidden = d_hidden;
    dyn.sh_native = L.shared;
    dyn.router_w = L.router_w;
    dyn.ln_w = L.ln;
    dyn.lslot = c->lslot;
    dyn.bias = L.bias;
    dyn.slot_tab = c->d_slot + (size_t)layer * E;
    dyn.resid = d_resid;
    dyn.out = d_out;
    auto launch = [&](uint32_t lo, uint32_t hi) -> wl_status {
        dyn.seg = lo | (hi << 8) | ((c->taps ? 1u : 0u) << 16) | ((c->xl2 ? 1u : 0u) << 17) | (ptag << 24);
        int e = wl::launch_decode(c->d_largs + layer, dyn, H, I, SI, E, K, c->grid,
                                  L.shared_dtype == WL_SHARED_MXFP4, stream);
        if (e != 0) return hip_fail(c, (hipError_t)e, "decode launch");
        return WL_OK;
    };
    if (c->sched == WL_SCHED_FUSED) {
        wl_status s = launch(0, 1);
        if (s != WL_OK) return s;
        c->ptag = ptag;
        if (!cached) return s;
        return cache_speculate(c, (hipStream_t)stream);
    }
    wl_status s;
    if ((s = launch(0, 0)) != WL_OK) return s;
    if ((s = launch(1, 1)) != WL_OK) {
        c->stale_partials = true;
        return s;
    }
    c->ptag = ptag;
    if (!cached) return s;
    return cache_speculate(c, (hipStream_t)stream);
}

}  // extern "C"

namespace wl {
// One MoE layer with its residual, in place: h <- h + moe(h) (wl_run_layer
// holds a single hidden buffer).
wl_status run_moe_in_place(wl_ctx* c, uint32_t layer, float* d_h, void* stream) {
    return run_layer(c, layer, d_h, d_h, d_h, stream, 0xFFFFFFFFu, true);
}
}  // namespace wl

extern "C" {

wl_status wl_run_moe(wl_ctx* c, uint32_t layer, const float* d_hidden, float* d_out, void* stream) {
    return run_layer(c, layer, d_hidden, nullptr, d_out, stream);
}

wl_status wl_run_moe_residual(wl_ctx* c, uint32_t layer, const float* d_hidden, const float* d_resid,
                              float* d_out, void* stream) {
    if (!d_resid) return fail(c, WL_ERR_INVALID, "null residual");
    return run_layer(c, layer, d_hidden, d_resid, d_out, stream);
}

wl_status wl_run_chain(wl_ctx* c, uint32_t first_layer, uint32_t n_layers, float* d_h, float* d_tmp,
                       void* stream) {
    if (!c) return WL_ERR_INVALID;
    if (!d_h || !d_tmp || d_h == d_tmp) return fail(c, WL_ERR_INVALID, "chain needs two distinct buffers");
    if (first_layer + (uint64_t)n_layers > c->cfg.n_layers)
        return fail(c, WL_ERR_INVALID, "layers [%u,%u) exceed n_layers %u", first_layer,
                    first_layer + n_layers, c->cfg.n_layers);
    if (n_layers == 0) return WL_OK;
    // Resident MoE layers under the fused schedule run in one launch
    // (moe_chain_kernel): a work-group starts layer l + 1 as soon as it has
    // finished its part of layer l, so the next layer's weight loads overlap
    // this layer's combine, with no launch boundary between layers. The
    // arithmetic is the per-layer launch's, so results are bit-identical.
    bool one_launch = c->sched == WL_SCHED_FUSED && c->hx != nullptr && !c->stale_partials;
    for (uint32_t l = 0; one_launch && l < n_layers; l++) {
        const LayerState& L = c->layers[first_layer + l];
        one_launch = L.set && !L.dense && c->n_bound[first_layer + l] == c->cfg.n_routed_experts &&
                     L.shared_dtype == c->layers[first_layer].shared_dtype;
    }
    if (one_launch) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
            return fail(c, WL_ERR_STATE, "a MoE decode chain cannot be captured into a graph (per-call epochs)");
        if ((uintptr_t)d_h % 16) return fail(c, WL_ERR_INVALID, "d_h must be 16-byte aligned");
        // layer l takes epoch epoch0 + l and the l-th partial tag after the last call's
        if (c->epoch + (uint64_t)n_layers >= 0x7FFFFFFFu) c->epoch = 0;
        const uint32_t epoch0 = c->epoch + 1, ptag0 = c->ptag % 3u + 1u;
        const uint32_t seg0 = 0u | (1u << 8) | ((c->taps ? 1u : 0u) << 16) | ((c->xl2 ? 1u : 0u) << 17) | (ptag0 << 24);
        const int e = wl::launch_chain(c->d_largs + first_layer, d_h, c->lslot, c->hx, n_layers, epoch0, seg0,
                                       c->cfg.hidden, c->cfg.moe_inter, c->SI, c->cfg.n_routed_experts,
                                       c->cfg.n_experts_per_tok, c->grid,
                                       c->layers[first_layer].shared_dtype == WL_SHARED_MXFP4, stream);
        if (e != 0) return hip_fail(c, (hipError_t)e, "chain launch");
        c->epoch += n_layers;
        c->ptag = (ptag0 - 1u + n_layers - 1u) % 3u + 1u;
        return WL_OK;
    }
    // every layer in place (see run_layer); d_tmp is not written
    for (uint32_t l = 0; l < n_layers; l++) {
        const uint32_t next = l + 1 < n_layers ? first_layer + l + 1 : 0xFFFFFFFFu;
        wl_status s = run_layer(c, first_layer + l, d_h, d_h, d_h, stream, next, true);
        if (s != WL_OK) return s;
    }
    return WL_OK;
}

wl_status wl_taps(wl_ctx* c, wl_taps_out* out) {
    if (!c || !out) return WL_ERR_INVALID;
    out->norm = c->norm;
    out->logits = c->logits;
    out->topk_idx = c->idx;
    out->topk_w = c->topw;
    out->mid = c->rmid;
    out->shared = c->shared_out;
    return WL_OK;
}

// Tokens per batched launch (longer calls run in chunks of this many).
constexpr uint32_t kBatchChunk = 4096;

// Byte layout of the batched layer's scratch for T tokens, every buffer
// 256-byte aligned. With base null only the size is computed; otherwise the
// pointers of *b are set into [base, base + size).
static size_t batch_layout(const wl_ctx* c, uint32_t T, uint8_t* base, wl::BatchArgs* b) {
    const size_t H = c->cfg.hidden, I = c->cfg.moe_inter, E = c->cfg.n_routed_experts, K = c->cfg.n_experts_per_tok,
                 SI = c->SI, t = T;
    size_t o = 0;
    auto take = [&](auto** p, size_t bytes) {
        o = (o + 255u) & ~(size_t)255u;
        if (base) *p = (std::remove_reference_t<decltype(*p)>)(base + o);
        o += bytes ? bytes : 16u;
    };
    wl::BatchArgs d{};
    wl::BatchArgs& x = b ? *b : d;
    take(&x.wq, 4 * wl::kWqWords);  // first: the same offset in every layout of the shared static scratch
    take(&x.norm, 4 * t * H);
    take(&x.norm3, 6 * t * H);
    take(&x.logits, 4 * t * E);
    take(&x.idx, 4 * t * K);
    take(&x.wts, 4 * t * K);
    take(&x.counts, 4 * E);
    take(&x.offsets, 4 * (E + 1));
    take(&x.lists, 4 * E * t);
    take(&x.ent, 4 * t * K);
    take(&x.pos, 4 * t * K);
    const size_t Kr = K + (c->any_sh4 ? 1u : 0u);  // + the MXFP4 shared expert's rows
    take(&x.mid3, 6 * t * Kr * I);
    take(&x.expout, 4 * t * Kr * H);
    take(&x.smid3, 6 * t * SI);
    take(&x.shout, 4 * t * H);
    return (o + 255u) & ~(size_t)255u;
}

// Largest chunk of tokens whose scratch fits in `bytes` (0 if none).
static uint32_t batch_tokens_fitting(const wl_ctx* c, size_t bytes) {
    uint32_t lo = 0, hi = kBatchChunk;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1u) / 2u;
        if (batch_layout(c, mid, nullptr, nullptr) <= bytes) lo = mid;
        else hi = mid - 1u;
    }
    return lo;
}

static wl_status batch_reserve(wl_ctx* c, uint32_t T) {
    BatchScratch& B = c->batch;
    if (T <= B.cap && B.sh4 == c->any_sh4) return WL_OK;
    hipError_t e = hipDeviceSynchronize();  // launches in flight may still use the old buffers
    if (e != hipSuccess) return hip_fail(c, e, "batched scratch resize");
    if (B.buf) (void)hipFree(B.buf);
    B.buf = nullptr;
    B.cap = 0;
    const size_t bytes = batch_layout(c, T, nullptr, nullptr);
    if (hipMalloc(&B.buf, bytes) != hipSuccess) {
        B.buf = nullptr;
        return fail(c, WL_ERR_OOM, "batched scratch for %u tokens (%zu B)", T, bytes);
    }
    batch_layout(c, T, (uint8_t*)B.buf, &B.b);
    if ((e = hipMemset(B.b.wq, 0, 4 * wl::kWqWords)) != hipSuccess || (e = hipDeviceSynchronize()) != hipSuccess)
        return hip_fail(c, e, "batched work-queue words");
    B.cap = T;
    B.sh4 = c->any_sh4;
    return WL_OK;
}

// Argument checks of the batched layer.
static wl_status batched_check(wl_ctx* c, uint32_t layer, uint32_t n_tokens, const float* d_hidden,
                               const float* d_resid, float* d_out) {
    if (layer >= c->cfg.n_layers) return fail(c, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, c->cfg.n_layers);
    if (!c->layers[layer].set) return fail(c, WL_ERR_STATE, "layer %u has no weights (wl_set_layer)", layer);
    if (n_tokens == 0 || n_tokens > 65535) return fail(c, WL_ERR_INVALID, "n_tokens=%u must be in [1,65535]", n_tokens);
    if (!d_hidden || !d_out) return fail(c, WL_ERR_INVALID, "null batched buffers");
    // d_out may be d_hidden and/or d_resid exactly (the reference adds the
    // block output into b.hidden in place, src/glm_layer_runner.cuh:918-920):
    // every chunk's rows are read before its combine writes them, each by the
    // thread that writes them. Partial overlaps are rejected.
    const size_t bytes = (size_t)n_tokens * c->cfg.hidden * 4;
    auto overlap = [&](const void* a, const void* b) {
        const char *x = (const char*)a, *y = (const char*)b;
        return a && b && a != b && x < y + bytes && y < x + bytes;
    };
    if (overlap(d_out, d_hidden) || overlap(d_out, d_resid))
        return fail(c, WL_ERR_INVALID, "d_out partly overlaps an input (only exact aliasing is allowed)");
    if (((uintptr_t)d_hidden | (uintptr_t)d_out | (uintptr_t)d_resid) % 16u)
        return fail(c, WL_ERR_INVALID, "batched buffers must be 16-byte aligned");
    if (c->layers[layer].dense) return WL_OK;
    const uint32_t E = c->cfg.n_routed_experts;
    if (E > wl::batched_max_experts())
        return fail(c, WL_ERR_INVALID, "the batched layer supports at most %u routed experts (config: %u)",
                    wl::batched_max_experts(), E);
    if (c->n_bound[layer] != E && !(c->n_bound[layer] == 0 && c->src.get))
        return fail(c, WL_ERR_NOT_RESIDENT, "batched layer %u has %u of %u experts bound%s", layer, c->n_bound[layer],
                    E, c->n_bound[layer] == 0 ? " and the context has no expert source" : "");
    return WL_OK;
}

// Chunk cap that keeps every piece array of the kernels under 2 GB (they
// address them with 32-bit buffer offsets) and the gate/up kernel's token
// table within its LDS.
static uint32_t batch_offset_cap(const wl_ctx* c) {
    const uint64_t H = c->cfg.hidden, K = c->cfg.n_experts_per_tok + (c->any_sh4 ? 1u : 0u);
    const uint64_t row = 6ull * K * std::max<uint64_t>(std::max<uint64_t>(H, c->cfg.moe_inter), c->SI);
    const uint32_t lds = wl::batched_max_tokens(c->cfg.moe_inter, c->SI, c->cfg.n_routed_experts,
                                                c->cfg.n_experts_per_tok, (uint32_t)c->n_cu);
    return (uint32_t)std::min<uint64_t>(std::min<uint64_t>(kBatchChunk, lds), ((1ull << 31) - 1) / row);
}

// The GEMMs of a source-backed batched chunk (routing already enqueued): read
// the per-expert counts back, then fetch the routed set through the source,
// every unique expert once, in ascending order and in chunks of at most 32
// (run_moe_batched's chunking, src/glm_layer_runner.cuh:869-902): announce
// the chunk, fetch its blocks, point the slot table at them (null elsewhere)
// and run the GEMMs of that chunk's experts (the shared expert's with the
// first chunk). may_grow: reference-layout staging may grow to 32 blocks
// (the allocation-free entry point keeps the staging it has).
static wl_status batched_source_gemms(wl_ctx* c, uint32_t layer, wl::BatchArgs b, bool may_grow, hipStream_t s) {
    const uint32_t E = c->cfg.n_routed_experts;
    uint32_t* counts = (uint32_t*)(c->h_pin + PinMap::counts);
    hipError_t e;
    if ((e = hipMemcpyAsync(counts, b.counts, 4 * (size_t)E, hipMemcpyDeviceToHost, s)) != hipSuccess ||
        (e = hipEventRecord(c->ids_ev, s)) != hipSuccess || (e = hipEventSynchronize(c->ids_ev)) != hipSuccess)
        return hip_fail(c, e, "batched routing read-back");
    std::vector<int32_t>& uniq = c->uniq;  // reserved for E ids: no allocation here
    uniq.clear();
    for (uint32_t x = 0; x < E; x++)
        if (counts[x]) uniq.push_back((int32_t)x);
    uint32_t ech = 32;
    // the cache: a chunk's misses that are not retained each need a distinct
    // transient slot while the chunk's GEMMs run
    if (c->src_cache) ech = std::min(ech, std::min(c->cache.capacity / 2u, c->cache.transient));
    if (!c->src.native) {
        if (may_grow) {
            wl_status st = ensure_stage(c, ech);
            if (st != WL_OK) return st;
        }
        ech = std::min(ech, c->stage_n);
    }
    if (ech == 0) return fail(c, WL_ERR_STATE, "no room to fetch experts");
    for (size_t i = 0; i < uniq.size(); i += ech) {
        const uint32_t n = (uint32_t)std::min<size_t>(ech, uniq.size() - i);
        const int32_t* ids = uniq.data() + i;
        wl_status st = source_prefetch(c, layer, ids, n, s);
        if (st != WL_OK) return st;
        const uint8_t* ptrs[32];
        if ((st = source_fetch(c, layer, ids, n, s, ptrs)) != WL_OK) return st;
        int le = wl::launch_slot_fill(c->d_slot + (size_t)layer * E, E, ids, ptrs, n, s);
        if (le != 0) return hip_fail(c, (hipError_t)le, "slot table fill");
        b.flags = (b.flags & wl::kBatchShared4) | wl::kBatchSkipUnbound | (i == 0 ? 0u : wl::kBatchNoShared);
        le = wl::launch_batched(c->d_largs + layer, b, c->cfg.hidden, c->cfg.moe_inter, c->SI, E,
                                c->cfg.n_experts_per_tok, (uint32_t)c->n_cu, wl::kPhaseGemm, s);
        if (le != 0) return hip_fail(c, (hipError_t)le, "batched GEMM launch");
    }
    return WL_OK;
}

// The batched layer in chunks of at most `chunk` tokens, every chunk on the
// buffers of `scratch` (sized for `chunk` tokens). A layer with no expert
// bound fetches its experts through the context's source.
static wl_status batched_run(wl_ctx* c, uint32_t layer, uint32_t n_tokens, const float* d_hidden,
                             const float* d_resid, float* d_out, const wl::BatchArgs& scratch, uint32_t chunk,
                             bool may_grow, void* stream) {
    const uint64_t H = c->cfg.hidden;
    const uint32_t E = c->cfg.n_routed_experts, K = c->cfg.n_experts_per_tok;
    const bool via_src = c->n_bound[layer] == 0;
    for (uint32_t t0 = 0; t0 < n_tokens; t0 += chunk) {
        wl::BatchArgs b = scratch;
        b.T = std::min(chunk, n_tokens - t0);
        b.flags = c->layers[layer].shared_dtype == WL_SHARED_MXFP4 ? wl::kBatchShared4 : 0u;
        b.hidden = d_hidden + (size_t)t0 * H;
        b.resid = d_resid ? d_resid + (size_t)t0 * H : nullptr;
        b.out = d_out + (size_t)t0 * H;
        c->batch.last = b;
        c->batch.ran = true;
        auto launch = [&](uint32_t phases) -> wl_status {
            const int e = wl::launch_batched(c->d_largs + layer, b, c->cfg.hidden, c->cfg.moe_inter, c->SI, E, K,
                                             (uint32_t)c->n_cu, phases, stream);
            return e == 0 ? WL_OK : hip_fail(c, (hipError_t)e, "batched launch");
        };
        wl_status s;
        if (!via_src) {
            if ((s = launch(wl::kPhaseAll)) != WL_OK) return s;
            continue;
        }
        if ((s = launch(wl::kPhaseRoute)) != WL_OK) return s;
        if ((s = batched_source_gemms(c, layer, b, may_grow, (hipStream_t)stream)) != WL_OK) return s;
        if ((s = launch(wl::kPhaseCombine)) != WL_OK) return s;
    }
    return WL_OK;
}

// A dense layer of a batched call: the dense MLP per position (the reference
// has nothing to amortise there either and runs run_moe + residual_add per
// position, src/glm_layer_runner.cuh:985-994). No scratch beyond the layer's.
static wl_status batched_dense(wl_ctx* c, uint32_t layer, uint32_t n_tokens, const float* d_hidden,
                               const float* d_resid, float* d_out, void* stream) {
    const size_t H = c->cfg.hidden;
    for (uint32_t t = 0; t < n_tokens; t++) {
        wl_status s = run_dense(c, layer, d_hidden + t * H, d_resid ? d_resid + t * H : nullptr, d_out + t * H, stream);
        if (s != WL_OK) return s;
    }
    return WL_OK;
}

wl_status wl_run_moe_batched(wl_ctx* c, uint32_t layer, uint32_t n_tokens, const float* d_hidden,
                             const float* d_resid, float* d_out, void* stream) {
    if (!c) return WL_ERR_INVALID;
    wl_status s = batched_check(c, layer, n_tokens, d_hidden, d_resid, d_out);
    if (s != WL_OK) return s;
    if (c->layers[layer].dense) return batched_dense(c, layer, n_tokens, d_hidden, d_resid, d_out, stream);
    // Tokens run in chunks: bounded scratch, and every piece array stays under
    // 2 GB.
    const uint32_t chunk = batch_offset_cap(c);
    if (chunk == 0) return fail(c, WL_ERR_INVALID, "batched rows too large for 32-bit offsets");
    if ((s = batch_reserve(c, std::min(n_tokens, chunk))) != WL_OK) return s;
    return batched_run(c, layer, n_tokens, d_hidden, d_resid, d_out, c->batch.b, chunk, true, stream);
}

wl_status wl_run_moe_batched_noalloc(wl_ctx* c, uint32_t layer, uint32_t n_tokens, const float* d_hidden,
                                     const float* d_resid, float* d_out, void* stream) {
    if (!c) return WL_ERR_INVALID;
    wl_status s = batched_check(c, layer, n_tokens, d_hidden, d_resid, d_out);
    if (s != WL_OK) return s;
    if (c->layers[layer].dense) return batched_dense(c, layer, n_tokens, d_hidden, d_resid, d_out, stream);
    if (c->n_bound[layer] == 0) {
        // a source-backed layer reads its routing back on the host (a
        // synchronisation), which a stream under capture does not allow
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
            return fail(c, WL_ERR_STATE, "layer %u runs through the expert source: it cannot be captured", layer);
    }
    if (!c->scratch) return fail(c, WL_ERR_STATE, "static scratch of device %d not resolved", c->device);
    const uint32_t chunk = std::min(batch_offset_cap(c), batch_tokens_fitting(c, wl::noalloc_scratch_bytes()));
    if (chunk == 0)
        return fail(c, WL_ERR_INVALID, "one token's batched scratch (%zu B) exceeds the static scratch (%zu B)",
                    batch_layout(c, 1, nullptr, nullptr), wl::noalloc_scratch_bytes());
    wl::BatchArgs scratch{};
    batch_layout(c, chunk, (uint8_t*)c->scratch, &scratch);
    return batched_run(c, layer, n_tokens, d_hidden, d_resid, d_out, scratch, chunk, false, stream);
}

wl_status wl_batched_counts(wl_ctx* c, uint32_t* h_counts) {
    if (!c || !h_counts) return WL_ERR_INVALID;
    if (!c->batch.ran) return fail(c, WL_ERR_STATE, "no batched call yet");
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess)
        e = hipMemcpy(h_counts, c->batch.last.counts, 4 * (size_t)c->cfg.n_routed_experts, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(c, e, "batched counts");
    return WL_OK;
}

wl_status wl_batched_routing(wl_ctx* c, uint32_t max_tokens, uint32_t* h_n_tokens, float* h_logits, int32_t* h_idx,
                             float* h_w) {
    if (!c || !h_n_tokens) return WL_ERR_INVALID;
    if (!c->batch.ran) return fail(c, WL_ERR_STATE, "no batched call yet");
    const wl::BatchArgs& b = c->batch.last;
    const uint32_t T = b.T;
    *h_n_tokens = T;
    if (T > max_tokens) return fail(c, WL_ERR_INVALID, "the last chunk has %u tokens > max_tokens %u", T, max_tokens);
    const size_t E = c->cfg.n_routed_experts, K = c->cfg.n_experts_per_tok;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess && h_logits) e = hipMemcpy(h_logits, b.logits, 4 * (size_t)T * E, hipMemcpyDeviceToHost);
    if (e == hipSuccess && h_idx) e = hipMemcpy(h_idx, b.idx, 4 * (size_t)T * K, hipMemcpyDeviceToHost);
    if (e == hipSuccess && h_w) e = hipMemcpy(h_w, b.wts, 4 * (size_t)T * K, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(c, e, "batched routing");
    return WL_OK;
}

// The built-in cache as an expert source (the reference's ExpertCache is an
// ExpertSource too, src/glm_expert_cache.cuh:99): prefetch resolves the
// experts (hits and misses counted, copies of the misses started on the side
// streams), get_async hands out a resolved block with the caller's stream
// ordered after its copy, get does the same and waits for the copy.
// Failures are reported through wl_ctx::src_status (the message in c->err).
static void cache_src_prefetch(void* u, uint32_t layer, const int32_t* ids, uint32_t n, void* stream) {
    wl_ctx* c = (wl_ctx*)u;
    const wl_status s = wl_cache_prefetch(c, layer, ids, n, stream);
    if (s != WL_OK) c->src_status = s;
}
static const uint8_t* cache_src_get_async(void* u, uint32_t layer, uint32_t expert, void* stream) {
    wl_ctx* c = (wl_ctx*)u;
    uint8_t* p = nullptr;
    const wl_status s = wl_cache_get(c, layer, expert, stream, &p);
    if (s != WL_OK) {
        c->src_status = s;
        return nullptr;
    }
    return p;
}
static const uint8_t* cache_src_get(void* u, uint32_t layer, uint32_t expert) {
    wl_ctx* c = (wl_ctx*)u;
    const uint8_t* p = cache_src_get_async(u, layer, expert, nullptr);
    if (p) {
        const hipError_t e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) {
            c->src_status = hip_fail(c, e, "expert copy wait");
            return nullptr;
        }
    }
    return p;
}

wl_status wl_set_expert_source(wl_ctx* c, const wl_expert_source* src) {
    if (!c) return WL_ERR_INVALID;
    if (c->src_cache) return fail(c, WL_ERR_STATE, "the context's built-in cache is its expert source");
    if (!src) {
        c->src = wl_expert_source{};
        return WL_OK;
    }
    if (!src->get) return fail(c, WL_ERR_INVALID, "an expert source needs get");
    wl_status s = ensure_pin(c);
    if (s != WL_OK) return s;
    if (!src->native && (s = ensure_stage(c, c->cfg.n_experts_per_tok)) != WL_OK) return s;
    c->src = *src;
    return WL_OK;
}

wl_status wl_make_resident(wl_ctx* c, uint32_t layer, void* stream) {
    if (!c) return WL_ERR_INVALID;
    if (layer >= c->cfg.n_layers) return fail(c, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, c->cfg.n_layers);
    if (c->layers[layer].dense) return fail(c, WL_ERR_INVALID, "layer %u is a dense layer: it has no experts", layer);
    if (!c->src.get) return fail(c, WL_ERR_STATE, "the context has no expert source");
    if (c->src_cache) return fail(c, WL_ERR_STATE, "the built-in cache is the context's source");
    const uint32_t E = c->cfg.n_routed_experts;
    if (c->n_bound[layer] == E) return WL_OK;
    if (c->n_bound[layer] != 0)
        return fail(c, WL_ERR_STATE, "layer %u has %u of %u experts bound", layer, c->n_bound[layer], E);
    const size_t nb = c->native_bytes;
    void* mem = nullptr;
    hipError_t e = hipMalloc(&mem, (size_t)E * nb);
    if (e != hipSuccess)
        return fail(c, WL_ERR_OOM, "%u native blocks for layer %u: %s", E, layer, hipGetErrorString(e));
    c->allocs.push_back(mem);
    uint8_t* blocks = (uint8_t*)mem;
    const wl_expert_source& S = c->src;
    hipStream_t s = (hipStream_t)stream;
    // K experts at a time: a source holds the blocks of one call (K) valid
    // until that call's work has run, as run_moe needs
    const uint32_t K = c->cfg.n_experts_per_tok;
    std::vector<const uint8_t*> src(K);
    std::vector<uint8_t*> dst(K);
    for (uint32_t x0 = 0; x0 < E; x0 += K) {
        const uint32_t m = std::min(K, E - x0);
        for (uint32_t i = 0; i < m; i++) {
            const uint32_t x = x0 + i;
            c->src_status = WL_OK;
            const uint8_t* p = S.get_async ? S.get_async(S.user, layer, x, (void*)s) : S.get(S.user, layer, x);
            if (!p) {
                if (c->src_status != WL_OK) return c->src_status;
                return fail(c, WL_ERR_IO, "expert source returned no block for layer %u expert %u", layer, x);
            }
            src[i] = p;
            dst[i] = blocks + (size_t)x * nb;
            if (S.native && (e = hipMemcpyAsync(dst[i], p, nb, hipMemcpyDeviceToDevice, s)) != hipSuccess)
                return hip_fail(c, e, "resident block copy");
        }
        if (!S.native && wl::launch_experts_to_native(src.data(), dst.data(), m, c->cfg.hidden, c->cfg.moe_inter, s) != 0)
            return fail(c, WL_ERR_HIP, "expert conversion launch failed");
    }
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(c, e, "resident fill");
    const size_t row = (size_t)layer * E;
    for (uint32_t x = 0; x < E; x++) c->h_slot[row + x] = blocks + (size_t)x * nb;
    c->n_bound[layer] = E;
    e = hipMemcpy(c->d_slot + row, &c->h_slot[row], sizeof(void*) * E, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(c, e, "slot table update");
    return WL_OK;
}

// The slot pool, LRU, side streams and events of a cache, and the cache as
// the context's expert source.
static wl_status cache_init(wl_ctx* c, uint32_t capacity) {
    CacheState& C = c->cache;
    if (C.lru) return fail(c, WL_ERR_STATE, "the context already has a cache");
    if (c->src.get) return fail(c, WL_ERR_STATE, "the context already has an expert source");
    if (capacity < 2u * c->cfg.n_experts_per_tok)
        return fail(c, WL_ERR_INVALID, "capacity %u < 2 x n_experts_per_tok", capacity);
    // 2K transient slots beyond the capacity: a miss the policy does not
    // retain (or that finds no evictable key) still needs its block in HBM
    C.transient = 2u * c->cfg.n_experts_per_tok;
    const uint32_t nslots = capacity + C.transient;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, (size_t)nslots * c->native_bytes);
    if (e != hipSuccess)
        return fail(c, WL_ERR_OOM, "cache pool of %u x %zu B: %s", nslots, c->native_bytes, hipGetErrorString(e));
    c->allocs.push_back(p);
    C.pool = (uint8_t*)p;
    C.capacity = capacity;
    wl_status ps = ensure_pin(c);
    if (ps != WL_OK) return ps;
    for (hipStream_t& st : C.copy)
        if ((e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking)) != hipSuccess) return hip_fail(c, e, "copy stream");
    if ((e = hipEventCreateWithFlags(&C.gate, hipEventDisableTiming)) != hipSuccess) return hip_fail(c, e, "cache event");
    C.slot_ev.assign(nslots, nullptr);
    for (hipEvent_t& ev : C.slot_ev)
        if ((e = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess) return hip_fail(c, e, "slot event");
    C.has_ev.assign(nslots, 0);
    C.spec.assign(nslots, 0);
    C.partial.assign(nslots, 0);
    C.task_of.assign(nslots, nullptr);
    C.raw.assign(nslots, 0);
    C.blk.resize(nslots);
    for (uint32_t i = 0; i < nslots; i++) C.blk[i] = C.pool + (size_t)i * c->native_bytes;
    C.lru = new wl::SlotLru(capacity, WL_POLICY_LRU, 0.5f, 0u, C.transient);
    c->src = wl_expert_source{c, cache_src_get, cache_src_prefetch, cache_src_get_async, 1};
    c->src_cache = true;
    return WL_OK;
}

wl_status wl_cache_create(wl_ctx* c, uint32_t capacity, wl_host_block_fn host_block, void* user) {
    if (!c) return WL_ERR_INVALID;
    if (!host_block) return fail(c, WL_ERR_INVALID, "host_block is null");
    wl_status s = cache_init(c, capacity);
    if (s != WL_OK) return s;
    c->cache.fn = host_block;
    c->cache.user = user;
    return WL_OK;
}

wl_status wl_cache_create_files(wl_ctx* c, uint32_t capacity, const char* dir, uint32_t first_layer,
                                uint32_t io_threads) {
    return wl_cache_create_files_ex(c, capacity, dir, first_layer, io_threads, 0u);
}

wl_status wl_cache_create_files_ex(wl_ctx* c, uint32_t capacity, const char* dir, uint32_t first_layer,
                                   uint32_t io_threads, uint32_t flags) {
    if (!c) return WL_ERR_INVALID;
    if (!dir) return fail(c, WL_ERR_INVALID, "dir is null");
    if (flags & ~(uint32_t)WL_FILES_DIRECT) return fail(c, WL_ERR_INVALID, "unknown flags 0x%x", flags);
    if ((flags & WL_FILES_DIRECT) && c->lay.total % 4096u)
        return fail(c, WL_ERR_INVALID, "WL_FILES_DIRECT needs records of a multiple of 4096 bytes, not %zu",
                    c->lay.total);
    if (io_threads > 64) return fail(c, WL_ERR_INVALID, "io_threads %u > 64", io_threads);
    if (c->cache.lru) return fail(c, WL_ERR_STATE, "the context already has a cache");
    std::unique_ptr<wl::FileTier> files(new wl::FileTier());
    if (c->lay.total > c->native_bytes)  // a record lands in its slot before it is converted
        return fail(c, WL_ERR_INVALID, "a file record (%zu B) exceeds a slot (%zu B)", c->lay.total, c->native_bytes);
    const std::string err = files->open(dir, first_layer, c->cfg.n_layers, c->cfg.n_routed_experts, c->lay.total,
                                        io_threads, c->device, (flags & WL_FILES_DIRECT) != 0u);
    if (!err.empty()) return fail(c, WL_ERR_IO, "%s", err.c_str());
    wl_status s = cache_init(c, capacity);
    if (s != WL_OK) return s;
    CacheState& C = c->cache;
    for (hipEvent_t& ev : C.gates) {
        const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(c, e, "gate event");
    }
    hipError_t e = hipEventCreateWithFlags(&C.spare_ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(c, e, "spare event");
    if ((e = hipMalloc((void**)&C.spare, c->native_bytes)) != hipSuccess) {
        C.spare = nullptr;
        return fail(c, WL_ERR_OOM, "spare block: %s", hipGetErrorString(e));
    }
    c->allocs.push_back(C.spare);  // (swapped into the pool and back: freed with the pool's allocation list)
    C.files = std::move(files);
    return WL_OK;
}

wl_status wl_cache_set_speculation(wl_ctx* c, int32_t enable) {
    if (!c) return WL_ERR_INVALID;
    if (!c->cache.lru) return fail(c, WL_ERR_STATE, "no cache (wl_cache_create)");
    c->cache.speculate = enable != 0;
    return WL_OK;
}

wl_status wl_cache_get_stats(wl_ctx* c, wl_cache_stats* out) {
    if (!c || !out) return WL_ERR_INVALID;
    const CacheState& C = c->cache;
    if (!C.lru) return fail(c, WL_ERR_STATE, "no cache (wl_cache_create)");
    out->hits = C.lru->hits();
    out->misses = C.lru->misses();
    out->evictions = C.lru->evictions();
    out->spec_requests = C.spec_requests;
    out->spec_copies = C.spec_copies;
    out->spec_hits = C.spec_hits;
    out->bytes_h2d = C.bytes_h2d;
    out->used = C.lru->used();
    out->capacity = C.capacity;
    out->bypassed = C.bypassed;
    return WL_OK;
}

wl_status wl_cache_reset_stats(wl_ctx* c) {
    if (!c) return WL_ERR_INVALID;
    CacheState& C = c->cache;
    if (!C.lru) return fail(c, WL_ERR_STATE, "no cache (wl_cache_create)");
    C.lru->reset_stats();
    C.spec_requests = C.spec_copies = C.spec_hits = C.bytes_h2d = C.bypassed = 0;
    return WL_OK;
}

wl_status wl_cache_prefetch(wl_ctx* c, uint32_t layer, const int32_t* experts, uint32_t n, void* stream) {
    if (!c) return WL_ERR_INVALID;
    CacheState& C = c->cache;
    if (!C.lru) return fail(c, WL_ERR_STATE, "no cache (wl_cache_create)");
    if (layer >= c->cfg.n_layers || (n && !experts) || n > WL_MAX_TOPK || n > C.capacity / 2u)
        return fail(c, WL_ERR_INVALID, "bad prefetch request (layer %u, n %u)", layer, n);
    uint32_t slots[WL_MAX_TOPK];
    wl_status s = cache_resolve(c, layer, experts, n, (hipStream_t)stream, false, slots);
    if (s != WL_OK) return s;
    C.resolved.clear();
    for (uint32_t k = 0; k < n; k++) C.resolved.push_back({layer * c->cfg.n_routed_experts + (uint32_t)experts[k], slots[k]});
    return WL_OK;
}

wl_status wl_cache_get(wl_ctx* c, uint32_t layer, uint32_t expert, void* stream, uint8_t** d_block) {
    if (!c || !d_block) return WL_ERR_INVALID;
    CacheState& C = c->cache;
    if (!C.lru) return fail(c, WL_ERR_STATE, "no cache (wl_cache_create)");
    if (layer >= c->cfg.n_layers || expert >= c->cfg.n_routed_experts)
        return fail(c, WL_ERR_INVALID, "(%u,%u) out of range", layer, expert);
    const uint32_t key = layer * c->cfg.n_routed_experts + expert;
    uint32_t slot = 0;
    bool found = false;
    for (const auto& r : C.resolved)
        if (r.first == key) {  // the prefetch ordered the stream after a host copy
            slot = r.second;
            found = true;
        }
    if (!found) {
        const int32_t id = (int32_t)expert;
        wl_status s = cache_resolve(c, layer, &id, 1, (hipStream_t)stream, false, &slot);
        if (s != WL_OK) return s;
    }
    if (C.files) {  // the slot's read: wait until its worker has issued it, then order the stream after it
        hipStream_t st = (hipStream_t)stream;
        if (wl::FileTask* t = C.task_of[slot]) {
            const bool ok = C.files->wait_issued(t);
            const std::string why = t->why;
            C.files->release(t);
            C.task_of[slot] = nullptr;
            if (!ok) {
                C.raw[slot] = 0;
                return fail(c, WL_ERR_IO, "read of layer %u expert %u failed: %s", layer, expert, why.c_str());
            }
        }
        hipError_t e;
        if (C.has_ev[slot] && (e = hipStreamWaitEvent(st, C.slot_ev[slot], 0)) != hipSuccess)
            return hip_fail(c, e, "wait for expert read");
        if (C.raw[slot]) {
            // the file's record -> the native layout, into the spare block, on
            // the caller's stream (ordered with its other kernels); the two
            // blocks then trade places
            if (C.spare_rec && (e = hipStreamWaitEvent(st, C.spare_ev, 0)) != hipSuccess)
                return hip_fail(c, e, "wait for the spare block");
            if (wl::launch_expert_to_native(C.blk[slot], C.spare, c->cfg.hidden, c->cfg.moe_inter, 0, st) != 0)
                return fail(c, WL_ERR_HIP, "expert conversion launch failed");
            std::swap(C.blk[slot], C.spare);
            if ((e = hipEventRecord(C.spare_ev, st)) != hipSuccess || (e = hipEventRecord(C.slot_ev[slot], st)) != hipSuccess)
                return hip_fail(c, e, "conversion event");
            C.spare_rec = true;
            C.raw[slot] = 0;
        }
    }
    *d_block = C.blk[slot];
    return WL_OK;
}

// An online policy (offline = true also admits the Belady bounds).
static bool policy_ok(const wl_cache_policy* p, bool offline = false) {
    return p && p->kind >= WL_POLICY_LRU && p->kind <= (offline ? WL_POLICY_BELADY_BYPASS : WL_POLICY_TINYLFU) &&
           p->protected_frac >= 0.f && p->protected_frac <= 1.f;
}

wl_status wl_policy_replay(const wl_cache_policy* policy, uint32_t capacity, const uint32_t* keys, uint32_t n_keys,
                           uint32_t batch, const uint32_t* pinned, uint32_t n_pinned, uint8_t* hit_out, uint64_t* hits,
                           uint64_t* misses, uint64_t* evictions) {
    if (!policy_ok(policy, true) || capacity == 0 || (n_keys && !keys) || batch == 0 || (n_pinned && !pinned))
        return WL_ERR_INVALID;
    if (policy->kind == WL_POLICY_BELADY || policy->kind == WL_POLICY_BELADY_BYPASS) {
        if (n_pinned) return WL_ERR_INVALID;  // the bound has no pinned keys (it bounds pinned policies too)
        wl::belady_replay(capacity, keys, n_keys, batch, policy->kind == WL_POLICY_BELADY_BYPASS, hit_out, hits,
                          misses, evictions);
        return WL_OK;
    }
    wl::SlotLru lru(capacity, policy->kind, policy->protected_frac, policy->ghost, 2u * batch);
    for (uint32_t i = 0; i < n_pinned; i++) lru.pin(pinned[i], true);
    for (uint32_t b0 = 0; b0 < n_keys; b0 += batch) {
        const uint32_t b1 = b0 + batch < n_keys ? b0 + batch : n_keys;
        lru.begin_batch();
        for (uint32_t i = b0; i < b1; i++) {
            bool dup = false;
            for (uint32_t j = b0; j < i; j++) dup = dup || keys[j] == keys[i];
            if (dup) {
                if (hit_out) hit_out[i] = 2;
                continue;
            }
            const wl::SlotLru::Result r = lru.request(keys[i]);
            if (hit_out) hit_out[i] = r.hit ? 1 : r.transient ? 3 : 0;
        }
    }
    if (hits) *hits = lru.hits();
    if (misses) *misses = lru.misses();
    if (evictions) *evictions = lru.evictions();
    return WL_OK;
}

wl_status wl_lru_replay(uint32_t capacity, const uint32_t* keys, uint32_t n_keys, uint32_t batch, uint8_t* hit_out,
                        uint64_t* hits, uint64_t* misses, uint64_t* evictions) {
    const wl_cache_policy lru{WL_POLICY_LRU, 0.5f, 0u};
    return wl_policy_replay(&lru, capacity, keys, n_keys, batch, nullptr, 0, hit_out, hits, misses, evictions);
}

// Empties the cache (every slot free, counters zero) under a new policy;
// pinned keys stay pinned. Waits for the device and for every pending read.
wl_status wl_cache_set_policy(wl_ctx* c, const wl_cache_policy* policy) {
    if (!c) return WL_ERR_INVALID;
    CacheState& C = c->cache;
    if (!C.lru) return fail(c, WL_ERR_STATE, "no cache (wl_cache_create)");
    if (!policy_ok(policy)) return fail(c, WL_ERR_INVALID, "bad cache policy");
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(c, e, "cache flush");
    if (C.files)
        for (wl::FileTask*& t : C.task_of)
            if (t) {
                C.files->wait_issued(t);
                C.files->release(t);
                t = nullptr;
            }
    if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail(c, e, "cache flush");
    delete C.lru;
    C.lru = new wl::SlotLru(C.capacity, policy->kind, policy->protected_frac, policy->ghost, C.transient);
    for (uint32_t k : C.pinned) C.lru->pin(k, true);
    C.policy = *policy;
    std::fill(C.spec.begin(), C.spec.end(), 0);
    std::fill(C.partial.begin(), C.partial.end(), 0);
    std::fill(C.raw.begin(), C.raw.end(), 0);  // the keys are gone; a slot is read again before it is handed out
    C.resolved.clear();
    C.spec_pending = false;
    C.spec_requests = C.spec_copies = C.spec_hits = C.bytes_h2d = C.bypassed = 0;
    return WL_OK;
}

wl_status wl_cache_pin(wl_ctx* c, uint32_t layer, uint32_t expert, int32_t pinned) {
    if (!c) return WL_ERR_INVALID;
    CacheState& C = c->cache;
    if (!C.lru) return fail(c, WL_ERR_STATE, "no cache (wl_cache_create)");
    if (layer >= c->cfg.n_layers || expert >= c->cfg.n_routed_experts)
        return fail(c, WL_ERR_INVALID, "(%u,%u) out of range", layer, expert);
    const uint32_t key = layer * c->cfg.n_routed_experts + expert;
    const bool on = pinned != 0;
    auto it = std::find(C.pinned.begin(), C.pinned.end(), key);
    if (on && it == C.pinned.end()) {
        if (C.pinned.size() + 2u * c->cfg.n_experts_per_tok >= C.capacity)
            return fail(c, WL_ERR_INVALID, "pinning more than capacity - 2 x n_experts_per_tok keys");
        C.pinned.push_back(key);
    } else if (!on && it != C.pinned.end()) {
        C.pinned.erase(it);
    }
    C.lru->pin(key, on);
    return WL_OK;
}

wl_status wl_check_error(wl_ctx* c, void* stream) {
    if (!c) return WL_ERR_INVALID;
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(c, e, "stream synchronize");
    uint32_t flag = 0;
    e = hipMemcpy(&flag, c->sync + c->sm.error, 4, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(c, e, "error flag read");
    if (flag) {
        // a launch that gave up may have left barrier counters mid-count, and
        // partial words of an older call whose tag a later call would reuse
        (void)hipMemset(c->sync, 0, 4 * (size_t)c->sm.words);
        (void)hipMemset(c->part, 0, 4 * wl::part_words(c->cfg.hidden, c->grid));
        (void)hipMemset(c->tsh, 0, 4 * wl::part_words(c->cfg.hidden, c->grid));
        (void)hipDeviceSynchronize();
        return fail(c, WL_ERR_DEVICE, "device error bits 0x%x%s%s%s%s", flag,
                    (flag & wl::E_SPIN) ? " [dependency wait expired]" : "",
                    (flag & wl::E_NOT_RESIDENT) ? " [routed expert not resident]" : "",
                    (flag & wl::E_XCD) ? " [work-group not on XCD w mod 8: set WL_DECODE_XL2=0]" : "",
                    (flag & wl::E_TOKTAB) ? " [batched token table overflow]" : "");
    }
    return WL_OK;
}

wl_status wl_set_taps(wl_ctx* c, int32_t enable) {
    if (!c) return WL_ERR_INVALID;
    c->taps = enable ? 1 : 0;
    return WL_OK;
}

wl_status wl_set_schedule(wl_ctx* c, int32_t sched) {
    if (!c) return WL_ERR_INVALID;
    if (sched != WL_SCHED_FUSED && sched != WL_SCHED_PHASED)
        return fail(c, WL_ERR_INVALID, "unknown schedule %d", sched);
    c->sched = sched;
    return WL_OK;
}

wl_status wl_dequant_matvec_mxfp4(const uint8_t* d_W, const uint8_t* d_S, const float* d_x, float* d_y,
                                  uint32_t N, uint32_t K, void* stream) {
    if (!d_W || !d_S || !d_x || !d_y) return WL_ERR_INVALID;
    if (N == 0 || N % 16 || K == 0 || K % 128 || K > 16384) return WL_ERR_INVALID;
    return wl::launch_dequant_matvec(d_W, d_S, d_x, d_y, N, K, stream) == 0 ? WL_OK : WL_ERR_HIP;
}

wl_status wl_expert_ffn(wl_ctx* c, const uint8_t* d_block, const float* d_x, float* d_y, uint16_t* d_y_bf16,
                        void* stream) {
    if (!c) return WL_ERR_INVALID;
    if (!d_block || !d_x || !d_y) return fail(c, WL_ERR_INVALID, "null block/x/y");
    if (++c->epoch >= 0x7FFFFFFFu) c->epoch = 1;
    const wl::FfnArgs a{d_block,  c->lay.gw_off, c->lay.gs_off, c->lay.uw_off, c->lay.us_off, c->lay.dw_off,
                        c->lay.ds_off, d_x,      d_y,           d_y_bf16,      c->ffn_tag,    c->sync,
                        c->cfg.hidden, c->cfg.moe_inter, c->epoch};
    int e = wl::launch_expert_ffn1(a, c->grid, stream);
    if (e < 0)  // a shape the one-launch kernel is not built for: gate/up, then down
        e = wl::launch_expert_ffn(d_block, c->lay.gw_off, c->lay.gs_off, c->lay.uw_off, c->lay.us_off,
                                  c->lay.dw_off, c->lay.ds_off, d_x, c->cfg.hidden, c->cfg.moe_inter, c->rmid,
                                  c->ffn_mid_p, d_y, d_y_bf16, stream);
    if (e != 0) return hip_fail(c, (hipError_t)e, "expert ffn launch");
    return WL_OK;
}

size_t wl_native_block_bytes(const wl_moe_config* cfg) {
    if (!cfg) return 0;
    return (size_t)wl::NativeLayout::make(cfg->hidden, cfg->moe_inter).total;
}

wl_status wl_expert_to_native(const wl_moe_config* cfg, const uint8_t* d_ref_block, uint8_t* d_native_block,
                              void* stream) {
    if (!cfg || !d_ref_block || !d_native_block) return WL_ERR_INVALID;
    if (validate_cfg(cfg, nullptr) != WL_OK) return WL_ERR_INVALID;
    return wl::launch_expert_to_native(d_ref_block, d_native_block, cfg->hidden, cfg->moe_inter, 0, stream) == 0
               ? WL_OK
               : WL_ERR_HIP;
}

wl_status wl_synth_expert_native(const wl_moe_config* cfg, uint32_t seed, uint32_t layer, uint32_t expert,
                                 uint8_t* d_native_block, void* stream) {
    if (!cfg || !d_native_block) return WL_ERR_INVALID;
    if (validate_cfg(cfg, nullptr) != WL_OK) return WL_ERR_INVALID;
    return wl::launch_expert_to_native(nullptr, d_native_block, cfg->hidden, cfg->moe_inter,
                                       wl::synth_key(seed, layer, expert), stream) == 0
               ? WL_OK
               : WL_ERR_HIP;
}

wl_status wl_synth_expert(const wl_moe_config* cfg, uint32_t inter, uint32_t seed, uint32_t layer,
                          uint32_t expert, uint8_t* d_block, void* stream) {
    if (!cfg || !d_block) return WL_ERR_INVALID;
    wl_expert_layout l;
    if (wl_expert_layout_of(cfg, inter, &l) != WL_OK) return WL_ERR_INVALID;
    if ((cfg->hidden % 128) || ((inter ? inter : cfg->moe_inter) % 128)) return WL_ERR_INVALID;
    const uint32_t key = wl::synth_key(seed, layer, expert);
    int e = wl::launch_synth_expert(d_block, l.gw_off, l.gw_len, l.gs_off, l.gs_len, l.uw_off, l.uw_len,
                                    l.us_off, l.us_len, l.dw_off, l.dw_len, l.ds_off, l.ds_len, key,
                                    stream);
    return e == 0 ? WL_OK : WL_ERR_HIP;
}

}  // extern "C"
