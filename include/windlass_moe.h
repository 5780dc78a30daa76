/*
 * windlass_moe.h — C ABI of the MI355X (gfx950) MoE-layer hot path.
 *
 * This is the drop-in boundary for windlass's MoE layer: the functions below
 * replace, one for one, the C++ entry points the reference binds for this
 * path. Every pointer argument named d_* is a device pointer; sizes are in
 * elements unless stated. No torch or HIP C++ types appear in the signatures:
 * the stream is passed as an opaque `void*` holding a hipStream_t (NULL = the
 * null stream).
 *
 * Error model: every call returns a wl_status. WL_OK is 0. On failure the
 * context keeps a human-readable message, read with wl_last_error(). Nothing
 * in this library calls exit() or abort() (the reference exits on CUDA and
 * I/O errors: src/glm_expert_cache.cuh:91-95, src/glm_loader.cuh:24-26).
 *
 * Threading: one host thread per context. All device work of a call is
 * enqueued on the stream passed to that call, in call order.
 *
 * Co-residency: the decode and routing kernels run one work-group per CU, and
 * those work-groups wait for each other's data (router logits, partial sums)
 * with bounded polls. wl_create checks that the chip can hold the whole grid
 * at once. While a layer runs, no other kernel may occupy the device's CUs
 * (a kernel on another stream, another process's context): a work-group left
 * unscheduled makes the others' waits expire, and the call reports
 * WL_ERR_DEVICE (E_SPIN) through wl_check_error instead of hanging. An error
 * aborts only the call that raised it; later calls run normally, while the
 * error bits stay set until wl_check_error reads them.
 */
#ifndef WINDLASS_MOE_H
#define WINDLASS_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum wl_status {
    WL_OK = 0,
    WL_ERR_INVALID = 1,      /* bad argument or unsupported shape */
    WL_ERR_HIP = 2,          /* a HIP runtime call failed */
    WL_ERR_OOM = 3,          /* device or pinned-host allocation failed */
    WL_ERR_NOT_RESIDENT = 4, /* a routed expert has no HBM slot bound */
    WL_ERR_STATE = 5,        /* call made in the wrong state (e.g. layer not set) */
    WL_ERR_DEVICE = 6,       /* the device kernel reported an error (see wl_check_error) */
    WL_ERR_IO = 7,           /* host backing store or checkpoint read failed */
    WL_ERR_NOT_FOUND = 8,    /* a checkpoint tensor is absent */
    WL_ERR_FORMAT = 9        /* a checkpoint file is malformed or does not match the config */
} wl_status;

/* MoE fields of glm::Config (reference src/glm_loader.cuh:35-47). */
typedef struct wl_moe_config {
    uint32_t hidden;             /* hidden_size                 6144 */
    uint32_t moe_inter;          /* moe_intermediate_size       2048 */
    uint32_t n_routed_experts;   /* n_routed_experts             256 */
    uint32_t n_experts_per_tok;  /* num_experts_per_tok            8 (<= WL_MAX_TOPK) */
    uint32_t n_shared;           /* n_shared_experts               1 */
    uint32_t n_layers;           /* MoE layers served by the context  */
    float    routed_scaling;     /* routed_scaling_factor        2.5 */
    int32_t  norm_topk_prob;     /* 1: renormalise the top-k weights */
    float    rms_eps;            /* rms_norm_eps                1e-5 */
} wl_moe_config;

#define WL_MAX_TOPK 32           /* reference MAX_TOPK, src/glm_loader.cuh:86 */

/* Sub-offsets inside one packed expert block (reference ExpertLayout,
 * src/glm_layer_runner.cuh:52-72; tools/repack_experts_glm.py:46-55):
 * gate_w | gate_s | up_w | up_s | down_w | down_s, MXFP4 nibbles (low nibble =
 * even column) with one E8M0 scale byte per 32 values. */
typedef struct wl_expert_layout {
    size_t gw_off, gw_len, gs_off, gs_len;
    size_t uw_off, uw_len, us_off, us_len;
    size_t dw_off, dw_len, ds_off, ds_len;
    size_t total;                /* 20,054,016 at hidden 6144 / inter 2048 */
} wl_expert_layout;

/* Replaces ExpertLayout::from(Config) (src/glm_layer_runner.cuh:60-72). */
wl_status wl_expert_layout_of(const wl_moe_config* cfg, uint32_t inter, wl_expert_layout* out);

typedef struct wl_ctx wl_ctx;

/* Creates a context on the current HIP device. Replaces the MoE part of
 * glm::alloc_scratch (src/glm_loader.cuh:363-450): all per-layer scratch
 * (norm, logits, top-k, SwiGLU intermediates, partial sums, counters) is owned
 * by the context. */
wl_status wl_create(const wl_moe_config* cfg, wl_ctx** out);
void      wl_destroy(wl_ctx* ctx);
const char* wl_last_error(const wl_ctx* ctx);

/* Shared-expert storage formats for wl_set_layer. */
#define WL_SHARED_BF16  0   /* [gate SI*H | up SI*H | down H*SI] bf16, row-major */
#define WL_SHARED_MXFP4 1   /* one packed block in wl_expert_layout order, inter = SI (n_shared = 1) */

/* Binds the non-expert weights of MoE layer `layer` (0-based within the
 * context). Router, bias and norm pointers are caller-owned and must stay
 * valid while the layer is run; the shared expert is copied (into the native
 * layout, in context-owned memory) during the call, which synchronises the
 * device. Replaces the MoE fields of glm::LayerWeights (src/glm_loader.cuh:
 * 259-339): router_w [E,H] bf16, router_bias [E] f32 (e_score_correction_bias,
 * kept f32 on purpose), post_attn_ln [H] bf16 (NULL = all ones), shared expert
 * block as above. */
wl_status wl_set_layer(wl_ctx* ctx, uint32_t layer, const uint16_t* d_router_w,
                       const float* d_router_bias, const uint16_t* d_post_attn_ln,
                       const void* d_shared, int32_t shared_dtype);

/* The same with the shared expert given as the six MXFP4 tensors of
 * glm::LayerWeights (sh_gate_w / sh_gate_s / sh_up_w / sh_up_s / sh_down_w /
 * sh_down_s, src/glm_loader.cuh:271-273,608-610): gate/up [SI, H/2] nibbles +
 * [SI, H/32] E8M0, down [H, SI/2] + [H, SI/32]. Requires n_shared = 1. */
wl_status wl_set_layer_mxfp4(wl_ctx* ctx, uint32_t layer, const uint16_t* d_router_w, const float* d_router_bias,
                             const uint16_t* d_post_attn_ln, const uint8_t* d_sh_gate_w, const uint8_t* d_sh_gate_s,
                             const uint8_t* d_sh_up_w, const uint8_t* d_sh_up_s, const uint8_t* d_sh_down_w,
                             const uint8_t* d_sh_down_s);

/* Binds layer `layer` as a dense MLP layer, the dense branch of run_moe for
 * the layers below first_k_dense_replace (src/glm_layer_runner.cuh:373-384;
 * glm::LayerWeights' post_attn_ln / mlp_gate / mlp_up / mlp_down,
 * src/glm_loader.cuh:259-339): post_attention_layernorm [H] bf16 (NULL = all
 * ones), gate / up [dense_inter, H] and down [H, dense_inter] bf16 row-major,
 * caller-owned, 16-byte aligned, valid while the layer is run. wl_run_moe on
 * the layer writes down(silu(gate x) * up x), x = RMSNorm(d_hidden), without
 * the residual (two GEMV launches, no host round trip); wl_run_moe_residual,
 * wl_run_chain and wl_run_moe_batched (one position at a time, as the
 * reference's layer-major prefill does for these layers, :985-994) add the
 * residual. The norm tap holds x. Synchronises the device. dense_inter: a
 * multiple of 8, at most 16384. */
wl_status wl_set_layer_dense(wl_ctx* ctx, uint32_t layer, const uint16_t* d_post_ln, const uint16_t* d_gate,
                             const uint16_t* d_up, const uint16_t* d_down, uint32_t dense_inter);

/* ---- HBM slot table (replaces the pointer-returning ExpertSource::get of a
 * fully resident model, src/glm_layer_runner.cuh:34-48) ---------------------
 * The device keeps a table slot_of[layer][expert] -> block pointer, and the
 * decode kernel resolves routed ids through it on the device, so no host
 * round-trip (src/glm_layer_runner.cuh:393-396) is needed when every expert
 * of the layer is bound.
 *
 * Bound blocks are in the NATIVE layout (wl_native_block_bytes bytes,
 * 21,233,664 at the GLM shape): the same bytes as the reference's packed
 * block, reordered so that each 16-byte load of a GPU wave is one lane of a
 * contiguous 1 KB chunk and the E8M0 scales of 16 k tiles of one lane are
 * one 16-byte chunk, plus a second copy of the scales in the batched
 * kernels' order (one 8-byte word per lane and step). Convert a
 * reference-layout block with wl_expert_to_native (the conversion the
 * reference's loader would run when it fills a VRAM slot,
 * src/glm_expert_cache.cuh:394-433). */
size_t    wl_native_block_bytes(const wl_moe_config* cfg);
wl_status wl_expert_to_native(const wl_moe_config* cfg, const uint8_t* d_ref_block, uint8_t* d_native_block,
                              void* stream);
wl_status wl_slot_bind(wl_ctx* ctx, uint32_t layer, uint32_t expert, const uint8_t* d_native_block);
wl_status wl_slot_unbind(wl_ctx* ctx, uint32_t layer, uint32_t expert);
/* Allocates a context-owned pool of n_slots native expert blocks (one
 * hipMalloc, like ExpertCache's pool, src/glm_expert_cache.cuh:150-156). */
wl_status wl_slot_pool_create(wl_ctx* ctx, uint32_t n_slots);
wl_status wl_slot_pool_ptr(wl_ctx* ctx, uint32_t slot, uint8_t** d_block);

/* ---- expert source (the C form of glm::ExpertSource,
 * src/glm_layer_runner.cuh:34-48) ------------------------------------------
 * A caller-supplied provider of expert blocks in DEVICE memory, for layers
 * whose experts are not bound in the slot table. `get` returns the block of
 * (layer, expert) (required); `prefetch` announces the n experts a layer is
 * about to read, so the source can start every fetch at once (optional, NULL
 * = nothing to overlap); `get_async` returns a block and orders `stream` after
 * its arrival (optional, NULL = get). A NULL return fails the call with
 * WL_ERR_IO. `native` = 1: blocks are in the native layout
 * (wl_native_block_bytes); 0: in the reference's packed layout
 * (wl_expert_layout, the layer_N.bin record), which the library converts on
 * `stream` into context-owned staging blocks before use.
 *
 * How the library calls it (run_moe's pattern, :391-418): a layer with no
 * expert bound is routed on the device, its K ids are read back on the host
 * (one host round trip per layer), then prefetch(layer, ids, K) and one
 * get_async per id, in slot order. A batched layer (wl_run_moe_batched) reads
 * back the routed set once, then fetches every unique expert exactly once, in
 * ascending id order and in chunks of at most 32 (prefetch of the chunk, then
 * get_async of each), running the chunk's GEMMs before the next chunk is
 * announced (run_moe_batched, :862-902).
 *
 * A returned block must stay valid until the work this call enqueued on
 * `stream` has completed; a source that reuses its buffers orders the reuse
 * after `stream` (the reference's ExpertCache records a gate event on the
 * caller's stream at prefetch for this, src/glm_expert_cache.cuh:204-208).
 * `user` is passed back unchanged. All calls come from the thread that calls
 * the library. */
typedef struct wl_expert_source {
    void* user;
    const uint8_t* (*get)(void* user, uint32_t layer, uint32_t expert);
    void (*prefetch)(void* user, uint32_t layer, const int32_t* experts, uint32_t n, void* stream);
    const uint8_t* (*get_async)(void* user, uint32_t layer, uint32_t expert, void* stream);
    int32_t native;
} wl_expert_source;

/* Attaches `src` (copied; NULL detaches) as the source of every layer of the
 * context that has no expert bound. A reference-layout source gets
 * n_experts_per_tok staging blocks (allocated here; the batched layer grows
 * them to 32 on first use). WL_ERR_STATE if the context has a built-in cache
 * (wl_cache_create installs the cache as the context's source). */
wl_status wl_set_expert_source(wl_ctx* ctx, const wl_expert_source* src);

/* Makes layer `layer` resident from the context's expert source: one
 * context-owned allocation of n_routed_experts native blocks (held until
 * wl_destroy), filled with every expert's block from the source (get_async,
 * else get, in id order; reference-layout blocks are converted on `stream`),
 * then bound in the slot table, so the layer runs from then on with no host
 * round trip and no per-call conversion. Synchronises `stream`. For the
 * reference's resident models, whose ExpertSource hands out the same VRAM
 * blocks on every call (src/glm_layer_runner.cuh:34-48). WL_ERR_STATE if the
 * context has no source, the built-in cache is its source, or the layer is
 * partly bound; WL_ERR_OOM if the blocks do not fit. */
wl_status wl_make_resident(wl_ctx* ctx, uint32_t layer, void* stream);

/* ---- the MoE layer ------------------------------------------------------
 * Replaces glm::run_moe (src/glm_layer_runner.cuh:352-443): post-attention
 * RMSNorm -> router GEMV -> sigmoid + bias -> top-k -> renorm ->
 * x routed_scaling -> K MXFP4 SwiGLU experts -> shared expert ->
 * out = sum_k w_k e_k + shared. d_hidden [H] f32 is the pre-norm residual
 * stream; d_out [H] f32 receives the block output WITHOUT the residual and must
 * not alias d_hidden. A layer with every expert bound runs with no host
 * round trip; a layer with none bound runs through the context's expert
 * source (wl_set_expert_source, or the built-in cache). Returns
 * WL_ERR_NOT_RESIDENT for a partly bound layer, or an unbound one without a
 * source. A MoE decode layer cannot be captured into a HIP graph (each launch
 * carries a new call epoch from the host): on a stream under capture this,
 * wl_run_moe_residual and wl_run_chain return WL_ERR_STATE. */
wl_status wl_run_moe(wl_ctx* ctx, uint32_t layer, const float* d_hidden, float* d_out,
                     void* stream);

/* Same layer with the residual fused: d_out = d_resid + moe(d_hidden). Used
 * by the decode chain (reference run_layer's residual_add,
 * src/glm_layer_runner.cuh:675). d_out must alias neither input. */
wl_status wl_run_moe_residual(wl_ctx* ctx, uint32_t layer, const float* d_hidden,
                              const float* d_resid, float* d_out, void* stream);

/* n_layers consecutive layers starting at first_layer, h <- h + moe(h) per
 * layer (the MoE half of run_chain's per-layer loop, src/glm_layer_runner.cuh:
 * 1065-1068). d_h [H] is updated in place (each layer reads all of h before
 * any of it is written); d_tmp [H] is accepted for the reference's calling
 * shape and not written. */
wl_status wl_run_chain(wl_ctx* ctx, uint32_t first_layer, uint32_t n_layers, float* d_h,
                       float* d_tmp, void* stream);

/* The layer for n_tokens positions at once (prefill; reference
 * run_moe_batched, src/glm_layer_runner.cuh:818-928). d_hidden [n_tokens][H]
 * f32 pre-norm residual stream; d_out [n_tokens][H] = d_resid + moe(d_hidden)
 * row by row (d_resid may be NULL: moe only; d_out may be d_hidden and/or
 * d_resid exactly, the reference's in-place update of b.hidden, but must not
 * partly overlap them; all three 16-byte aligned). Each token is routed exactly as wl_run_moe routes
 * it (same ids); tokens are then
 * grouped by expert (stable, (token, slot) order) and every selected expert's
 * weights are streamed once per 32 of its tokens; the per-token combine sums
 * the slots in slot order, then the shared expert (the reference's pass 3).
 * A layer with every expert bound runs with no host round trip; a layer with
 * none bound fetches its routed set through the context's expert source (see
 * wl_expert_source: one host round trip per chunk of tokens, each unique
 * expert fetched once). n_tokens <= 65535, run in chunks of up to 4096 tokens.
 * At most 816 routed experts (the GEMM kernels keep the expert tables in LDS
 * beside the activation slots); a wider config fails with WL_ERR_INVALID.
 * Scratch grows to the largest chunk seen (context-owned; growing
 * synchronises the device). */
wl_status wl_run_moe_batched(wl_ctx* ctx, uint32_t layer, uint32_t n_tokens, const float* d_hidden,
                             const float* d_resid, float* d_out, void* stream);

/* The batched layer for callers that cannot allocate: no counterpart in the
 * reference. It is for code that may not call hipMalloc during a call (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation): the same arguments, kernels and results as wl_run_moe_batched,
 * but the scratch comes from a static 64 MiB device array of the library
 * (one per GPU, held until the process ends) instead of context memory that
 * wl_run_moe_batched grows on demand, so the call performs no hipMalloc,
 * hipFree or other allocation. Tokens run in chunks of as many as the array
 * holds (169 at hidden 6144 / inter 2048 / 8 of 256 experts); a shape whose
 * single token does not fit returns WL_ERR_INVALID. Every call on one GPU
 * shares that GPU's array, which keeps the last call's contents: calls that
 * overlap on one GPU (two streams, two contexts, two host threads) race.
 * A layer with every expert bound, or a dense layer, enqueues kernels only
 * and can be captured into a HIP graph and replayed; a layer that runs
 * through the expert source reads its routing back on the host per chunk,
 * and fails with WL_ERR_STATE on a stream under capture. */
wl_status wl_run_moe_batched_noalloc(wl_ctx* ctx, uint32_t layer, uint32_t n_tokens, const float* d_hidden,
                                     const float* d_resid, float* d_out, void* stream);

/* Tokens routed to each expert by the last chunk of the last wl_run_moe_batched
 * call (all of it when n_tokens <= 4096) (h_counts:
 * host array of n_routed_experts; synchronises the device). The grouping the
 * reference keeps in run_moe_batched's where[] (src/glm_layer_runner.cuh:
 * 855-868). */
wl_status wl_batched_counts(wl_ctx* ctx, uint32_t* h_counts);

/* Test hook, no reference counterpart: the routing of the last chunk of the
 * last wl_run_moe_batched call. *h_n_tokens = its token count T (WL_ERR_INVALID
 * if T > max_tokens, nothing copied); then, for each non-null array (host,
 * sized for max_tokens), the router logits [T][n_routed_experts], the selected
 * ids [T][n_experts_per_tok] (descending biased score) and their weights
 * [T][n_experts_per_tok]; synchronises the device. Per token these equal
 * wl_taps' logits / topk_idx / topk_w after wl_run_moe on the same hidden
 * state. */
wl_status wl_batched_routing(wl_ctx* ctx, uint32_t max_tokens, uint32_t* h_n_tokens, float* h_logits,
                             int32_t* h_idx, float* h_w);

/* Device pointers to the last layer's intermediates (the substeps
 * test_glm_chain reads through SubstepHook, src/test_glm_chain.cu:434-441). */
typedef struct wl_taps_out {
    const float*   norm;     /* [H]  post_attention_layernorm output */
    const float*   logits;   /* [E]  router logits */
    const int32_t* topk_idx; /* [K]  selected experts, descending biased score */
    const float*   topk_w;   /* [K]  routing weights */
    const float*   mid;      /* [K, I] routed SwiGLU outputs */
    const float*   shared;   /* [H]  shared expert output (when taps are on) */
} wl_taps_out;
wl_status wl_taps(wl_ctx* ctx, wl_taps_out* out);

/* Synchronises `stream`, then returns WL_ERR_DEVICE (and clears the flag) if a
 * kernel of this context reported an error since the last check. */
wl_status wl_check_error(wl_ctx* ctx, void* stream);

/* Execution schedule of wl_run_moe: WL_SCHED_FUSED runs one persistent
 * kernel per layer, whose combine waits for the epoch-tagged partial sums of
 * the other work-groups (no grid barrier); WL_SCHED_PHASED runs the combine as
 * a second stream-ordered launch. Both compute identical results. */
#define WL_SCHED_FUSED  0
#define WL_SCHED_PHASED 1
wl_status wl_set_schedule(wl_ctx* ctx, int32_t sched);

/* Whether wl_run_moe also produces the shared-expert output tap (wl_taps_out.
 * shared). The other taps are always written. The shared expert's
 * contribution is otherwise only kept summed into the layer output, so the tap
 * costs one extra H-vector per work-group; off for benchmarking. Default: on
 * (the reference's run_moe leaves every intermediate in its scratch,
 * src/glm_layer_runner.cuh:431-436). */
wl_status wl_set_taps(wl_ctx* ctx, int32_t enable);

/* ---- HBM expert cache (config 4: more experts than HBM holds) -------------
 * Replaces the reference's ExpertCache (src/glm_expert_cache.cuh:99-509): an
 * LRU pool of `capacity` native expert blocks in HBM, keyed by (layer,
 * expert), filled from host memory on a miss. Where the reference reads
 * packed files with pread into pinned staging, this cache copies directly
 * from pinned host blocks that the caller provides through `host_block`
 * (native layout, wl_native_block_bytes bytes each, allocated with
 * hipHostMalloc; NULL for an unknown expert fails the call with WL_ERR_IO).
 *
 * A layer with no experts bound through wl_slot_bind runs through the cache:
 * wl_run_moe routes it (norm, router, top-k on the device), waits for the
 * ids on the host (the reference's one host round trip per layer,
 * src/glm_layer_runner.cuh:391-396), resolves them (hits bump the LRU,
 * misses evict the least-recent key and start a host-to-device copy on a
 * side stream), orders the caller's stream after those copies and runs the
 * layer. Requires capacity >= 2 x n_experts_per_tok.
 *
 * With speculation on, wl_run_chain also applies layer l+1's router to layer
 * l's input while layer l runs and starts the copies of the predicted
 * misses then (cross-layer prefetch); those requests update the LRU order but
 * are counted in spec_* only. */
typedef const uint8_t* (*wl_host_block_fn)(void* user, uint32_t layer, uint32_t expert);
wl_status wl_cache_create(wl_ctx* ctx, uint32_t capacity, wl_host_block_fn host_block, void* user);
/* The reference's file tier (ExpertCache::init, src/glm_expert_cache.cuh:
 * 139-183): the same cache, its misses read from the packed expert files
 * `dir`/layer_N.bin, N = first_layer + context layer (256 records of
 * wl_expert_layout.total bytes in the reference layout, record e at offset
 * e x total; tools/repack_experts_glm.py:5-14,46-55). A pool of io_threads
 * workers pread each miss into one of its two pinned buffers and copies it,
 * as it is, into the slot on its own non-blocking stream (after the gate
 * event of the resolve that took the slot, so no kernel enqueued before still
 * reads it). The workers launch no kernel: a copy engine moves the block, so
 * nothing shares the CUs with the persistent kernels (see Co-residency).
 * wl_cache_get (and the layer run) waits until the read is issued, orders the
 * stream after it and, the first time the slot is handed out, converts it
 * into the native layout on that stream (one kernel, ~13 us at the GLM
 * shape, into a spare block that then takes the slot's place). io_threads = 0
 * reads on the calling thread. Every file must exist and hold all
 * n_routed_experts records (WL_ERR_IO otherwise); a short read fails the call
 * that needs the block with WL_ERR_IO. Each worker (one for io_threads = 0)
 * holds two reference blocks of pinned memory; the cache holds one spare
 * device block. */
wl_status wl_cache_create_files(wl_ctx* ctx, uint32_t capacity, const char* dir, uint32_t first_layer,
                                uint32_t io_threads);
/* The same with flags: WL_FILES_DIRECT reads with O_DIRECT (bypassing the
 * host page cache; the record size must be a multiple of 4096 bytes, as it is
 * at the GLM shape: 20,054,016 = 4,896 x 4,096). No reference counterpart:
 * the reference reads through the page cache. */
#define WL_FILES_DIRECT 1
wl_status wl_cache_create_files_ex(wl_ctx* ctx, uint32_t capacity, const char* dir, uint32_t first_layer,
                                   uint32_t io_threads, uint32_t flags);
wl_status wl_cache_set_speculation(wl_ctx* ctx, int32_t enable);

typedef struct wl_cache_stats {
    uint64_t hits, misses, evictions;  /* reference ExpertCache counters (:334-336) */
    uint64_t spec_requests;            /* speculative (predicted) requests */
    uint64_t spec_copies;              /* speculative requests that started a copy */
    uint64_t spec_hits;                /* real requests served by a speculative copy */
    uint64_t bytes_h2d;                /* bytes copied host -> device */
    uint32_t used, capacity;           /* occupied / total slots */
    uint64_t bypassed;                 /* misses served from a transient slot, not retained */
} wl_cache_stats;
wl_status wl_cache_get_stats(wl_ctx* ctx, wl_cache_stats* out);
wl_status wl_cache_reset_stats(wl_ctx* ctx);

/* ExpertCache::prefetch + get_async (src/glm_expert_cache.cuh:186-275):
 * resolve n experts of `layer` at once (hits and misses counted), starting
 * the copies of the misses; wl_cache_get then returns the device block of one
 * resolved expert and orders `stream` after its copy. wl_cache_get on an
 * expert that was not resolved resolves it alone. */
wl_status wl_cache_prefetch(wl_ctx* ctx, uint32_t layer, const int32_t* experts, uint32_t n, void* stream);
wl_status wl_cache_get(wl_ctx* ctx, uint32_t layer, uint32_t expert, void* stream, uint8_t** d_block);

/* Replacement and admission policy of the cache (no reference counterpart
 * except WL_POLICY_LRU, the reference's ExpertCache semantics and the
 * default):
 *   WL_POLICY_LFU      evict the key requested least often so far (ties: the
 *                      least recent)
 *   WL_POLICY_SLRU     segmented LRU: a miss enters a probationary segment, a
 *                      hit there promotes the key to a protected segment of
 *                      protected_frac x capacity slots (its least recent key
 *                      demoted back); victims come from the probationary end
 *   WL_POLICY_2Q       admission on a second miss: a key missing for the first
 *                      time (not among the last `ghost` first misses; 0 =
 *                      capacity) is served but not retained
 *   WL_POLICY_TINYLFU  frequency admission: a missing key is retained only if
 *                      it has been requested more often than its victim
 * Victims are never keys of the request batch being resolved, nor pinned
 * keys. A miss that is not retained is copied into one of 2 x
 * n_experts_per_tok transient slots beyond `capacity` (allocated with the
 * cache) and counted in wl_cache_stats.bypassed. */
#define WL_POLICY_LRU     0
#define WL_POLICY_LFU     1
#define WL_POLICY_SLRU    2
#define WL_POLICY_2Q      3
#define WL_POLICY_TINYLFU 4
/* Offline bounds, accepted by wl_policy_replay only, without pinned keys
 * (they read every future request of the replayed sequence;
 * wl_cache_set_policy refuses them):
 *   WL_POLICY_BELADY         Belady's MIN: evict the key whose next request
 *                            comes last; every miss is retained
 *   WL_POLICY_BELADY_BYPASS  MIN with bypass: a missing key whose own next
 *                            request comes after the victim's is not retained
 * Both drop the rule that a batch's misses do not evict the keys the batch
 * has already requested, which makes them the optimum of plain paging, and
 * an upper bound on the hits of every policy of the same kind (retaining
 * every miss, or free to decline one) under the batch rule, pinned or not. */
#define WL_POLICY_BELADY        5
#define WL_POLICY_BELADY_BYPASS 6
typedef struct wl_cache_policy {
    int32_t  kind;            /* WL_POLICY_* */
    float    protected_frac;  /* SLRU: share of the slots in the protected segment (0.5) */
    uint32_t ghost;           /* 2Q: first misses remembered (0 = capacity) */
} wl_cache_policy;
/* Empties the cache (every slot free, counters zero) and sets its policy;
 * synchronises the device and waits for pending reads. */
wl_status wl_cache_set_policy(wl_ctx* ctx, const wl_cache_policy* policy);
/* Pins (pinned != 0) or unpins the key (layer, expert): a pinned key is always
 * admitted and never evicted (popularity pinning: pin the most requested keys of a profile). At
 * most capacity - 2 x n_experts_per_tok keys may be pinned. */
wl_status wl_cache_pin(wl_ctx* ctx, uint32_t layer, uint32_t expert, int32_t pinned);
/* Replay hook (no device use): wl_lru_replay under `policy` (an online
 * policy, or one of the offline bounds), with `n_pinned` pinned keys;
 * hit_out[i] is 1 for a hit, 0 for a retained miss, 3 for a miss not
 * retained, 2 for a skipped duplicate. */
wl_status wl_policy_replay(const wl_cache_policy* policy, uint32_t capacity, const uint32_t* keys, uint32_t n_keys,
                           uint32_t batch, const uint32_t* pinned, uint32_t n_pinned, uint8_t* hit_out,
                           uint64_t* hits, uint64_t* misses, uint64_t* evictions);

/* Test hook (no device use): replays `n_keys` requests through the cache's
 * LRU bookkeeping with `capacity` slots, in batches of `batch` keys (keys
 * repeated within a batch are skipped, as in a prefetch batch). hit_out[i]
 * (optional) is 1 for a hit, 0 for a miss, 2 for a skipped duplicate. */
wl_status wl_lru_replay(uint32_t capacity, const uint32_t* keys, uint32_t n_keys, uint32_t batch,
                        uint8_t* hit_out, uint64_t* hits, uint64_t* misses, uint64_t* evictions);

/* ---- checkpoint loader (safetensors) -------------------------------------
 * A sharded safetensors checkpoint: model.safetensors.index.json maps each
 * tensor name to a shard file; a shard is an 8-byte little-endian header
 * length, a JSON header {name: {dtype, shape, data_offsets}} and the data.
 * Host-only: these calls use no device. One thread per wl_st. */
typedef struct wl_st wl_st;

#define WL_ST_MAX_DIMS 8
typedef struct wl_st_tensor {
    char     dtype[16];          /* "BF16", "F32", "U8", ... as in the header */
    uint32_t ndim;
    uint64_t shape[WL_ST_MAX_DIMS];
    uint64_t nbytes;
    uint64_t file_offset;        /* absolute offset of its first byte in its shard */
    uint32_t shard;              /* index of its shard file */
} wl_st_tensor;

/* Replaces st::open (src/safetensors_io.cuh:89-186). `path` is a checkpoint
 * directory (with model.safetensors.index.json, or a single
 * model.safetensors) or one .safetensors file. Every tensor the index names
 * must be in its shard's header; allow_missing_shards != 0 skips shard files
 * that do not exist (their tensors are then absent, as in st::open). Each
 * tensor's byte range must lie inside its shard, and for the fixed-width
 * dtypes match its shape (WL_ERR_FORMAT otherwise). On failure *out is NULL
 * and wl_st_last_error(NULL) gives this thread's message. */
wl_status   wl_st_open(const char* path, int32_t allow_missing_shards, wl_st** out);
void        wl_st_close(wl_st* st);                                      /* st::close */
const char* wl_st_last_error(const wl_st* st);
uint32_t    wl_st_count(const wl_st* st);                                /* tensors, */
const char* wl_st_name(const wl_st* st, uint32_t i);                     /* in name order */
/* Replaces st::info (src/safetensors_io.cuh:194-197): WL_ERR_NOT_FOUND for
 * an absent tensor. */
wl_status   wl_st_info(const wl_st* st, const char* name, wl_st_tensor* out);
/* Replaces st::read_bytes (src/safetensors_io.cuh:199-229): the tensor's raw
 * bytes into h_dst (capacity >= nbytes), by positional reads. */
wl_status   wl_st_read(wl_st* st, const char* name, void* h_dst, size_t capacity);

/* Replaces the MoE fields of glm::load_layer (src/glm_loader.cuh:524-620):
 * loads checkpoint layer `ckpt_layer`'s
 *   model.layers.N.post_attention_layernorm.weight       BF16 [H]
 *   model.layers.N.mlp.gate.weight                       BF16 [E, H]
 *   model.layers.N.mlp.gate.e_score_correction_bias      F32  [E]
 *   model.layers.N.mlp.shared_experts.{gate,up,down}_proj.weight
 * into context layer `layer`. A tensor is MXFP4 when "<name>_scale" exists
 * (as in the reference): then the weight is U8 [rows, cols/2] and the scale
 * U8 [rows, cols/32] (gate/up: rows SI, cols H; down: rows H, cols SI), and
 * the shared expert is bound as by wl_set_layer_mxfp4; without scales the
 * shared projections are BF16 [rows, cols] and bound as WL_SHARED_BF16. The
 * router, bias and norm copies are owned by the context (freed when the layer
 * is bound again or the context destroyed). Errors: WL_ERR_NOT_FOUND for a
 * missing tensor, WL_ERR_FORMAT for a dtype or size that does not match the
 * config, WL_ERR_IO for a failed read. Synchronises the device. */
wl_status wl_load_layer(wl_ctx* ctx, wl_st* st, uint32_t ckpt_layer, uint32_t layer);

/* Populates the slot table from the checkpoint: routed experts experts[i]
 * (experts NULL: expert i), i < n, of checkpoint layer `ckpt_layer`
 * (model.layers.N.mlp.experts.e.{gate,up,down}_proj.weight and
 * .weight_scale, MXFP4 as above) are read into pinned buffers, copied to the
 * device, converted into the native layout in context pool slot first_slot +
 * i (wl_slot_pool_create) and bound to (layer, experts[i]). Every tensor is
 * checked before any slot is written. Reads of one expert overlap the copy
 * and conversion of the previous one on `stream`; the call returns after the
 * stream has drained and the slots are bound. Reference: the packed block of
 * tools/repack_experts_glm.py:46-55 filled into an ExpertCache slot
 * (src/glm_expert_cache.cuh:394-433), here straight from the shards. */
wl_status wl_load_experts(wl_ctx* ctx, wl_st* st, uint32_t ckpt_layer, uint32_t layer, const uint32_t* experts,
                          uint32_t n, uint32_t first_slot, void* stream);

/* Writes `path` as the packed expert file of checkpoint layer `ckpt_layer`
 * (the input of wl_cache_create_files): n_routed_experts records of
 * wl_expert_layout_of(cfg, 0).total bytes, record e the six tensors of expert
 * e in layout order (tools/repack_experts_glm.py:5-14,46-55). Host-only;
 * errors in wl_st_last_error(st); a failed call removes the partial file. */
wl_status wl_st_pack_layer(wl_st* st, const wl_moe_config* cfg, uint32_t ckpt_layer, const char* path);

/* ---- the caller side of a decoder layer: MLA attention and dense MLP ------
 * Replaces run_attention / run_layer (src/glm_layer_runner.cuh:525-675) and
 * the dense branch of run_moe (:373-384) at decode (one position per call).
 * A wl_attn holds the attention weights of n_layers decoder layers (caller-
 * owned device pointers), their KV caches (context-owned, max_seq positions:
 * kv_c [L] and k_rot [qk_rope] f32 per position, the absorbed-MLA form, plus
 * the indexer keys [index_head_dim] f32 on indexer-owning layers) and the
 * scratch. One host thread per wl_attn; work is enqueued on the given stream. */
typedef struct wl_attn_config {
    uint32_t hidden;          /* hidden_size               6144 */
    uint32_t n_heads;         /* num_attention_heads         64 */
    uint32_t q_lora_rank;     /*                           2048 */
    uint32_t kv_lora_rank;    /*                            512 */
    uint32_t qk_nope;         /* qk_nope_head_dim           192 */
    uint32_t qk_rope;         /* qk_rope_head_dim            64 */
    uint32_t v_head;          /* v_head_dim                 256 */
    uint32_t index_n_heads;   /* DSA indexer heads           32 */
    uint32_t index_head_dim;  /*                            128 */
    uint32_t index_topk;      /* keys kept per query       2048 */
    uint32_t dense_inter;     /* intermediate_size (dense MLP) 12288 */
    uint32_t n_layers;        /* decoder layers served by the context */
    uint32_t max_seq;         /* KV-cache capacity in positions */
    float    rms_eps;         /* rms_norm_eps of input / post-attention norms 1e-5 */
    float    rope_theta;
} wl_attn_config;

typedef struct wl_attn wl_attn;

/* Attention weights of one layer (glm::LayerWeights' attention fields,
 * src/glm_loader.cuh:259-339), bf16 [out, in] row-major unless stated. The
 * five idx_* pointers are all set on an indexer-owning ("full") layer and all
 * NULL on a "shared" layer, which reuses the selection the last owning layer
 * made at the same position (IndexShare, src/glm_layer_runner.cuh:461-519). */
typedef struct wl_attn_weights {
    const uint16_t* input_ln;          /* [H] */
    const uint16_t* q_a_proj;          /* [q_lora, H] */
    const uint16_t* q_a_ln;            /* [q_lora] */
    const uint16_t* q_b_proj;          /* [n_heads * (qk_nope + qk_rope), q_lora] */
    const uint16_t* kv_a_proj;         /* [kv_lora + qk_rope, H] (kv_a_proj_with_mqa) */
    const uint16_t* kv_a_ln;           /* [kv_lora] */
    const uint16_t* kv_b_proj;         /* [n_heads * (qk_nope + v_head), kv_lora] */
    const uint16_t* o_proj;            /* [H, n_heads * v_head] */
    const uint16_t* idx_wq_b;          /* [index_n_heads * index_head_dim, q_lora] */
    const uint16_t* idx_wk;            /* [index_head_dim, H] */
    const uint16_t* idx_k_norm_w;      /* [index_head_dim] (LayerNorm weight) */
    const uint16_t* idx_k_norm_b;      /* [index_head_dim] (LayerNorm bias) */
    const float*    idx_weights_proj;  /* [index_n_heads, H] f32 */
} wl_attn_weights;

/* Creates the context on the current device (KV caches zeroed). Shapes:
 * hidden, q_lora_rank, kv_lora_rank, n_heads * v_head and dense_inter are
 * multiples of 8 and at most 16384; kv_lora_rank <= 512; qk_rope a multiple
 * of 4 and <= index_head_dim <= 256; index_n_heads * index_head_dim <= 16384;
 * n_heads a multiple of 16 or at most 16; v_head a multiple of 8. On
 * failure wl_attn_last_error(NULL) gives this thread's message. */
wl_status   wl_attn_create(const wl_attn_config* cfg, wl_attn** out);
void        wl_attn_destroy(wl_attn* a);
const char* wl_attn_last_error(const wl_attn* a);
wl_status   wl_attn_set_layer(wl_attn* a, uint32_t layer, const wl_attn_weights* w);
/* A dense MLP layer (layer < dense_first): post_attention_layernorm [H],
 * gate / up [dense_inter, H], down [H, dense_inter], bf16. */
wl_status   wl_attn_set_dense_mlp(wl_attn* a, uint32_t layer, const uint16_t* d_post_ln, const uint16_t* d_gate,
                                  const uint16_t* d_up, const uint16_t* d_down);
/* run_attention: d_hidden [H] f32 <- d_hidden + o_proj(attention(input_ln(
 * d_hidden))) at position pos (< max_seq), writing the layer's cache row pos;
 * the keys attended are 0..pos (those of the DSA selection when pos + 1 >
 * index_topk). A "shared" layer with no selection published at pos by an
 * owning layer fails with WL_ERR_STATE (the reference raises, M:418). */
wl_status   wl_run_attention(wl_attn* a, uint32_t layer, uint32_t pos, float* d_hidden, void* stream);
/* d_hidden <- d_hidden + down(silu(gate(x)) * up(x)), x = post_ln(d_hidden). */
wl_status   wl_run_dense_mlp(wl_attn* a, uint32_t layer, float* d_hidden, void* stream);
/* run_layer: attention, then the dense MLP (a layer set with
 * wl_attn_set_dense_mlp) or the MoE layer moe_layer of `moe` (wl_run_moe +
 * residual), d_hidden updated in place. */
wl_status   wl_run_layer(wl_attn* a, wl_ctx* moe, uint32_t layer, uint32_t moe_layer, uint32_t pos, float* d_hidden,
                         void* stream);
/* Device pointers to the last call's intermediates (test hook): the input
 * norm [H], q_resid [q_lora], the attention context before o_proj
 * [n_heads * v_head], the o_proj output [H], the index scores [pos + 1] and
 * keep mask [pos + 1] (uint8, 1 = attended) of the last owning layer. */
typedef struct wl_attn_taps_out {
    void* norm;
    void* q_resid;
    void* attn;
    void* attn_out;
    void* index_score;
    void* keep;
} wl_attn_taps_out;
wl_status   wl_attn_taps(wl_attn* a, wl_attn_taps_out* out);

/* ---- single-expert building blocks ---------------------------------------
 * y[N] = W . x for MXFP4 W ([N,K/2] packed nibbles + [N,K/32] E8M0 scales) and
 * f32 x [K]. Replaces launch_dequant_matvec_mxfp4 (src/glm_kernels.cuh:104-110).
 * Requires N % 16 == 0, K % 128 == 0, K <= 16384. */
wl_status wl_dequant_matvec_mxfp4(const uint8_t* d_W, const uint8_t* d_S, const float* d_x, float* d_y,
                                  uint32_t N, uint32_t K, void* stream);

/* y[N] = W . x for bf16 W [N, K] row-major and f32 x [K] (K % 8 == 0,
 * K <= 16384, 16-byte aligned pointers): the GEMV kernel of the attention
 * and dense-MLP projections. Replaces launch_matvec_bf16
 * (src/glm_primitives.cuh:87-116). */
wl_status wl_matvec_bf16(const uint16_t* d_W, const float* d_x, float* d_y, uint32_t N, uint32_t K, void* stream);

/* One routed expert applied to one position, without the routing weight:
 * y = down(silu(gate x) * up x), d_block in wl_expert_layout order, x f32 [H],
 * y f32 [H] and, if d_y_bf16 is not NULL, its bf16 (round-to-nearest-even)
 * copy. The per-expert sequence of run_moe (3 x dequant_matvec_mxfp4 +
 * silu_mul, src/glm_layer_runner.cuh:424-427) and expert_slot
 * (tools/ref_glm_chain.py:679-685). Uses the context's scratch. */
wl_status wl_expert_ffn(wl_ctx* ctx, const uint8_t* d_block, const float* d_x, float* d_y,
                        uint16_t* d_y_bf16, void* stream);

/* ---- synthetic weights (test and benchmark inputs; no reference
 * counterpart: the reference loads real checkpoints) -----------------------
 * Fills one expert block with the counter-based generator: packed weight
 * bytes = bytes of mix32(mix32(i ^ salt_r) ^ key), scale bytes = 118 +
 * (mix32(...) % 9), key = f(seed, layer, expert). The CPU oracle regenerates
 * the same bytes. */
wl_status wl_synth_expert(const wl_moe_config* cfg, uint32_t inter, uint32_t seed,
                          uint32_t layer, uint32_t expert, uint8_t* d_block, void* stream);
/* The same synthetic expert written directly in the native layout (equal to
 * wl_expert_to_native of wl_synth_expert's block). */
wl_status wl_synth_expert_native(const wl_moe_config* cfg, uint32_t seed, uint32_t layer, uint32_t expert,
                                 uint8_t* d_native_block, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* WINDLASS_MOE_H */
