// attn_host.cpp — the C ABI of the caller side of a decoder layer
// (wl_attn_*, wl_run_attention, wl_run_dense_mlp, wl_run_layer): context,
// KV caches, the DSA selection shared across layers, and the launch
// sequence. Reference: run_attention / run_layer / IndexShare
// (src/glm_layer_runner.cuh:461-675), the attention part of alloc_scratch
// (src/glm_loader.cuh:363-450).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/windlass_moe.h"
#include "attention.h"

namespace wl {
wl_status run_moe_in_place(wl_ctx* c, uint32_t layer, float* d_h, void* stream);  // moe_host.cpp
}

namespace {

constexpr uint32_t kMaxSplits = 64;

struct AttnLayer {
    wl_attn_weights w{};
    bool set = false;
    bool owner = false;
    bool dense = false;
    const uint16_t *post_ln = nullptr, *gate = nullptr, *up = nullptr, *down = nullptr;
    float* kv_c = nullptr;   // [max_seq][L]
    float* k_rot = nullptr;  // [max_seq][RP]
    float* idx_k = nullptr;  // [max_seq][ID] (owner)
    uint8_t* keep = nullptr; // [max_seq] (owner)
    uint32_t* klist = nullptr;  // [max_seq + 1] (owner): kept keys, then their count
};

}  // namespace

struct wl_attn {
    wl_attn_config cfg{};
    wl::attn::Shape sh{};
    std::vector<AttnLayer> layers;
    std::vector<void*> allocs;
    std::string err;
    float *x_norm = nullptr, *qa_raw = nullptr, *q_resid = nullptr, *kv_raw = nullptr, *ik_raw = nullptr,
          *iw = nullptr, *q = nullptr, *iq = nullptr, *iqr = nullptr, *q_abs = nullptr, *q_rope = nullptr,
          *rope_cs = nullptr, *isc = nullptr, *part_m = nullptr, *part_l = nullptr, *part_ctx = nullptr,
          *ctx = nullptr, *attn = nullptr, *attn_out = nullptr, *g = nullptr, *u = nullptr;
    int32_t share_layer = -1;          // the owning layer whose selection is current
    uint32_t share_pos = 0xFFFFFFFFu;  // the position it was made at
    int32_t last_owner = -1;
};

namespace {
thread_local std::string t_create_err;  // wl_attn_create's message when no context exists
}  // namespace

namespace {

wl_status fail(wl_attn* a, wl_status s, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
wl_status fail(wl_attn* a, wl_status s, const char* fmt, ...) {
    if (a) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        a->err = buf;
    }
    return s;
}

template <typename T>
wl_status dalloc(wl_attn* a, T** p, size_t bytes, bool zero = false) {
    void* q = nullptr;
    hipError_t e = hipMalloc(&q, bytes ? bytes : 16);
    if (e != hipSuccess) return fail(a, WL_ERR_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    a->allocs.push_back(q);
    if (zero && (e = hipMemset(q, 0, bytes ? bytes : 16)) != hipSuccess)
        return fail(a, WL_ERR_HIP, "hipMemset: %s", hipGetErrorString(e));
    *p = (T*)q;
    return WL_OK;
}

wl_status validate(const wl_attn_config* c, wl_attn* a) {
    if (!c) return fail(a, WL_ERR_INVALID, "config is null");
    auto k_ok = [](uint32_t k) { return k > 0 && k % 8 == 0 && k <= 16384; };
    if (!k_ok(c->hidden) || !k_ok(c->q_lora_rank) || !k_ok(c->kv_lora_rank) || !k_ok(c->n_heads * c->v_head) ||
        (c->dense_inter && !k_ok(c->dense_inter)))
        return fail(a, WL_ERR_INVALID, "hidden, q_lora_rank, kv_lora_rank, n_heads x v_head and dense_inter must be "
                                       "multiples of 8 in [8, 16384]");
    if (c->kv_lora_rank > 512) return fail(a, WL_ERR_INVALID, "kv_lora_rank %u exceeds 512", c->kv_lora_rank);
    if (c->kv_lora_rank + c->qk_rope > 768)
        return fail(a, WL_ERR_INVALID, "kv_lora_rank + qk_rope = %u exceeds 768", c->kv_lora_rank + c->qk_rope);
    if (c->qk_rope == 0 || c->qk_rope % 4 || c->qk_rope > c->index_head_dim || c->index_head_dim > 256 ||
        c->index_head_dim % 8)
        return fail(a, WL_ERR_INVALID,
                    "need qk_rope a multiple of 4, qk_rope <= index_head_dim <= 256, index_head_dim %% 8 == 0");
    if (c->index_n_heads == 0 || c->index_n_heads * c->index_head_dim > 16384)
        return fail(a, WL_ERR_INVALID, "index_n_heads x index_head_dim must be in [1, 16384]");
    if (c->n_heads == 0 || (c->n_heads > 16 && c->n_heads % 16))
        return fail(a, WL_ERR_INVALID, "n_heads %u: a multiple of 16, or at most 16", c->n_heads);
    if (c->v_head == 0 || c->v_head % 8 || c->qk_nope == 0)
        return fail(a, WL_ERR_INVALID, "v_head must be a positive multiple of 8 and qk_nope positive");
    if (c->index_topk == 0) return fail(a, WL_ERR_INVALID, "index_topk must be positive");
    if (c->n_layers == 0 || c->n_layers > 4096 || c->max_seq == 0)
        return fail(a, WL_ERR_INVALID, "n_layers in [1, 4096] and max_seq > 0 are required");
    return WL_OK;
}

// Appends a job to a launch (at most kMaxJobs per launch; callers add at most four).
void add_job(wl::attn::GemvLaunch& l, uint32_t& n_wg, wl::attn::GemvJob j) {
    if (j.G == 0) {  // ungrouped: row r is W row r, x is shared (GS == 0 marks it)
        j.G = j.N;
        j.GS = 0;
        j.OFF = 0;
        j.XS = 0;
    }
    j.wg0 = n_wg;
    n_wg += wl::attn::gemv_plan(j);
    l.job[l.n_jobs++] = j;
}

wl::attn::GemvJob job(const void* W, const float* x, float* y, uint32_t N, uint32_t K) {
    wl::attn::GemvJob j{};
    j.W = W;
    j.x = x;
    j.y = y;
    j.N = N;
    j.K = K;
    return j;
}

wl_status launched(wl_attn* a, int e, const char* what) {
    if (e != 0) return fail(a, WL_ERR_HIP, "%s launch: %s", what, hipGetErrorString((hipError_t)e));
    return WL_OK;
}

}  // namespace

namespace wl {
namespace attn {

// post_ln -> gate / up (one launch, the norm fused into each job) -> SwiGLU
// fused into the down job's input -> y = add + down . mid (a second launch).
int launch_dense_mlp(const DenseMlp& m, const float* x, const float* add, float* y, float* g, float* u, float* x_norm,
                     float* y_raw, void* stream) {
    GemvLaunch l{};
    uint32_t n = 0;
    auto j = job(m.gate, x, g, m.DI, m.H);
    j.norm_w = m.post_ln;
    j.eps = m.eps;
    j.x_out = x_norm;
    {  // streaming kernel: gate and up rows as one paired job, g = silu(gate x') * up x'
        GemvLaunch lp{};
        uint32_t np = 0;
        auto jp = j;
        jp.W2 = m.up;
        add_job(lp, np, jp);
        GemvLaunch d{};
        uint32_t nd = 0;
        auto jd = job(m.down, g, y, m.H, m.DI);
        jd.add = add;
        jd.y_raw = y_raw;
        add_job(d, nd, jd);
        if (sgemv_fits(lp) && sgemv_fits(d)) {
            int e = launch_gemv(lp, np, stream);
            return e != 0 ? e : launch_gemv(d, nd, stream);
        }
    }
    add_job(l, n, j);
    j = job(m.up, x, u, m.DI, m.H);
    j.norm_w = m.post_ln;
    j.eps = m.eps;
    add_job(l, n, j);
    int e = launch_gemv(l, n, stream);
    if (e != 0) return e;
    GemvLaunch d{};
    n = 0;
    j = job(m.down, g, y, m.H, m.DI);
    j.x2 = u;
    j.add = add;
    j.y_raw = y_raw;
    add_job(d, n, j);
    return launch_gemv(d, n, stream);
}

}  // namespace attn
}  // namespace wl

extern "C" {

wl_status wl_attn_create(const wl_attn_config* cfg, wl_attn** out) {
    if (!out) return WL_ERR_INVALID;
    *out = nullptr;
    wl_attn* a = new wl_attn();
    wl_status st = validate(cfg, a);
    if (st != WL_OK) {
        t_create_err = a->err;
        delete a;
        return st;
    }
    const wl_attn_config& c = *cfg;
    a->cfg = c;
    wl::attn::Shape& s = a->sh;
    s.H = c.hidden;
    s.HN = c.n_heads;
    s.Q = c.q_lora_rank;
    s.L = c.kv_lora_rank;
    s.NP = c.qk_nope;
    s.RP = c.qk_rope;
    s.VD = c.v_head;
    s.IH = c.index_n_heads;
    s.ID = c.index_head_dim;
    s.TOPK = c.index_topk;
    s.DI = c.dense_inter;
    s.eps = c.rms_eps;
    s.theta = c.rope_theta;
    a->layers.resize(c.n_layers);
    const size_t DH = s.NP + s.RP, S = kMaxSplits;
    const size_t f = sizeof(float);
    if ((st = dalloc(a, &a->x_norm, s.H * f)) != WL_OK || (st = dalloc(a, &a->qa_raw, s.Q * f)) != WL_OK ||
        (st = dalloc(a, &a->q_resid, s.Q * f)) != WL_OK || (st = dalloc(a, &a->kv_raw, (s.L + s.RP) * f)) != WL_OK ||
        (st = dalloc(a, &a->ik_raw, s.ID * f)) != WL_OK || (st = dalloc(a, &a->iw, s.IH * f)) != WL_OK ||
        (st = dalloc(a, &a->q, s.HN * DH * f)) != WL_OK || (st = dalloc(a, &a->iq, (size_t)s.IH * s.ID * f)) != WL_OK ||
        (st = dalloc(a, &a->iqr, (size_t)s.IH * s.ID * f)) != WL_OK ||
        (st = dalloc(a, &a->q_abs, (size_t)s.HN * s.L * f)) != WL_OK ||
        (st = dalloc(a, &a->q_rope, (size_t)s.HN * s.RP * f)) != WL_OK || (st = dalloc(a, &a->rope_cs, s.RP * f)) != WL_OK ||
        (st = dalloc(a, &a->isc, (size_t)c.max_seq * f, true)) != WL_OK ||
        (st = dalloc(a, &a->part_m, S * s.HN * f)) != WL_OK || (st = dalloc(a, &a->part_l, S * s.HN * f)) != WL_OK ||
        (st = dalloc(a, &a->part_ctx, S * s.HN * s.L * f)) != WL_OK ||
        (st = dalloc(a, &a->ctx, (size_t)s.HN * s.L * f)) != WL_OK ||
        (st = dalloc(a, &a->attn, (size_t)s.HN * s.VD * f)) != WL_OK ||
        (st = dalloc(a, &a->attn_out, s.H * f)) != WL_OK ||
        (st = dalloc(a, &a->g, (size_t)(s.DI ? s.DI : 8) * f)) != WL_OK ||
        (st = dalloc(a, &a->u, (size_t)(s.DI ? s.DI : 8) * f)) != WL_OK) {
        t_create_err = a->err;
        wl_attn_destroy(a);
        return st;
    }
    for (AttnLayer& L : a->layers) {
        if ((st = dalloc(a, &L.kv_c, (size_t)c.max_seq * s.L * f, true)) != WL_OK ||
            (st = dalloc(a, &L.k_rot, (size_t)c.max_seq * s.RP * f, true)) != WL_OK) {
            t_create_err = a->err;
            wl_attn_destroy(a);
            return st;
        }
    }
    *out = a;
    return WL_OK;
}

void wl_attn_destroy(wl_attn* a) {
    if (!a) return;
    (void)hipDeviceSynchronize();
    for (void* p : a->allocs) (void)hipFree(p);
    delete a;
}

const char* wl_attn_last_error(const wl_attn* a) { return a ? a->err.c_str() : t_create_err.c_str(); }

wl_status wl_attn_set_layer(wl_attn* a, uint32_t layer, const wl_attn_weights* w) {
    if (!a) return WL_ERR_INVALID;
    if (layer >= a->cfg.n_layers) return fail(a, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, a->cfg.n_layers);
    if (!w) return fail(a, WL_ERR_INVALID, "weights are null");
    if (!w->input_ln || !w->q_a_proj || !w->q_a_ln || !w->q_b_proj || !w->kv_a_proj || !w->kv_a_ln || !w->kv_b_proj ||
        !w->o_proj)
        return fail(a, WL_ERR_INVALID, "the eight attention tensors are required");
    const int n_idx = (w->idx_wq_b != nullptr) + (w->idx_wk != nullptr) + (w->idx_k_norm_w != nullptr) +
                      (w->idx_k_norm_b != nullptr) + (w->idx_weights_proj != nullptr);
    if (n_idx != 0 && n_idx != 5)
        return fail(a, WL_ERR_INVALID, "the indexer tensors are all set (owning layer) or all null (shared layer)");
    AttnLayer& L = a->layers[layer];
    L.w = *w;
    L.owner = n_idx == 5;
    if (L.owner && !L.idx_k) {
        wl_status st;
        if ((st = dalloc(a, &L.idx_k, (size_t)a->cfg.max_seq * a->sh.ID * sizeof(float), true)) != WL_OK ||
            (st = dalloc(a, &L.keep, a->cfg.max_seq, true)) != WL_OK ||
            (st = dalloc(a, &L.klist, ((size_t)a->cfg.max_seq + 1) * sizeof(uint32_t), true)) != WL_OK)
            return st;
    }
    L.set = true;
    return WL_OK;
}

wl_status wl_attn_set_dense_mlp(wl_attn* a, uint32_t layer, const uint16_t* d_post_ln, const uint16_t* d_gate,
                                const uint16_t* d_up, const uint16_t* d_down) {
    if (!a) return WL_ERR_INVALID;
    if (layer >= a->cfg.n_layers) return fail(a, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, a->cfg.n_layers);
    if (!a->sh.DI) return fail(a, WL_ERR_INVALID, "dense_inter is 0 in the config");
    if (!d_post_ln || !d_gate || !d_up || !d_down) return fail(a, WL_ERR_INVALID, "the four MLP tensors are required");
    AttnLayer& L = a->layers[layer];
    L.post_ln = d_post_ln;
    L.gate = d_gate;
    L.up = d_up;
    L.down = d_down;
    L.dense = true;
    return WL_OK;
}

wl_status wl_run_attention(wl_attn* a, uint32_t layer, uint32_t pos, float* d_hidden, void* stream) {
    if (!a) return WL_ERR_INVALID;
    if (layer >= a->cfg.n_layers) return fail(a, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, a->cfg.n_layers);
    AttnLayer& L = a->layers[layer];
    if (!L.set) return fail(a, WL_ERR_STATE, "layer %u has no attention weights (wl_attn_set_layer)", layer);
    if (!d_hidden) return fail(a, WL_ERR_INVALID, "hidden is null");
    if ((uintptr_t)d_hidden % 16) return fail(a, WL_ERR_INVALID, "hidden must be 16-byte aligned");
    if (pos >= a->cfg.max_seq) return fail(a, WL_ERR_INVALID, "position %u >= max_seq %u", pos, a->cfg.max_seq);
    const wl::attn::Shape& s = a->sh;
    const uint32_t T = pos + 1, DH = s.NP + s.RP;
    uint8_t* keep = nullptr;
    uint32_t* klist = nullptr;
    if (!L.owner) {
        if (a->share_layer < 0 || a->share_pos != pos)
            return fail(a, WL_ERR_STATE,
                        "layer %u is \"shared\" and no indexer-owning layer published a selection at position %u", layer,
                        pos);
        keep = a->layers[a->share_layer].keep;
        klist = a->layers[a->share_layer].klist;
    } else {
        keep = L.keep;
        klist = L.klist;
    }
    hipStream_t st = (hipStream_t)stream;
    wl_status rs;
    // 1. input norm (fused) -> q_a, kv_a, and the indexer key / head weights
    {
        wl::attn::GemvLaunch l{};
        uint32_t n = 0;
        auto j = job(L.w.q_a_proj, d_hidden, a->qa_raw, s.Q, s.H);
        j.norm_w = L.w.input_ln;
        j.eps = s.eps;
        j.x_out = a->x_norm;
        add_job(l, n, j);
        j = job(L.w.kv_a_proj, d_hidden, a->kv_raw, s.L + s.RP, s.H);
        j.norm_w = L.w.input_ln;
        j.eps = s.eps;
        add_job(l, n, j);
        if (L.owner) {
            j = job(L.w.idx_wk, d_hidden, a->ik_raw, s.ID, s.H);
            j.norm_w = L.w.input_ln;
            j.eps = s.eps;
            add_job(l, n, j);
            j = job(L.w.idx_weights_proj, d_hidden, a->iw, s.IH, s.H);
            j.norm_w = L.w.input_ln;
            j.eps = s.eps;
            j.f32w = 1;
            add_job(l, n, j);
        }
        if ((rs = launched(a, wl::attn::launch_gemv(l, n, st), "attention projections")) != WL_OK) return rs;
    }
    wl::attn::AttnPtrs p{};
    p.kv_c = L.kv_c;
    p.k_rot = L.k_rot;
    p.idx_k = L.idx_k;
    p.kv_a_ln = L.w.kv_a_ln;
    p.kv_b = L.w.kv_b_proj;
    p.idx_k_norm_w = L.w.idx_k_norm_w;
    p.idx_k_norm_b = L.w.idx_k_norm_b;
    p.kv_raw = a->kv_raw;
    p.ik_raw = a->ik_raw;
    p.iw = a->iw;
    p.iw_scale = (float)(1.0 / std::sqrt((double)s.IH));
    p.qk_scale = (float)(1.0 / std::sqrt((double)DH));
    p.ix_scale = (float)(1.0 / std::sqrt((double)s.ID));
    p.q = a->q;
    p.iq = a->iq;
    p.iqr = a->iqr;
    p.q_abs = a->q_abs;
    p.q_rope = a->q_rope;
    p.rope_cs = a->rope_cs;
    p.isc = a->isc;
    p.keep = keep;
    p.klist = klist;
    p.max_seq = a->cfg.max_seq;
    p.part_m = a->part_m;
    p.part_l = a->part_l;
    p.part_ctx = a->part_ctx;
    p.ctx = a->ctx;
    // 2. q_a_layernorm (fused) -> q_b, and the indexer query; in the same
    // launch, the cache rows of pos (kv_c, k_rot, indexer key)
    {
        wl::attn::GemvLaunch l{};
        uint32_t n = 0;
        auto j = job(L.w.q_b_proj, a->qa_raw, a->q, s.HN * DH, s.Q);
        j.norm_w = L.w.q_a_ln;
        j.eps = 1e-6f;  // the LoRA norms take the class default eps (src/glm_loader.cuh LORA_NORM_EPS)
        j.x_out = a->q_resid;
        add_job(l, n, j);
        if (L.owner) {
            j = job(L.w.idx_wq_b, a->qa_raw, a->iq, s.IH * s.ID, s.Q);
            j.norm_w = L.w.q_a_ln;
            j.eps = 1e-6f;
            add_job(l, n, j);
        }
        if ((rs = launched(a, wl::attn::launch_gemv_prep(l, n, s, p, pos, L.owner, st), "query projections")) != WL_OK)
            return rs;
    }
    // 3. absorbed query, RoPE of the queries and (owning layers) the index scores
    if ((rs = launched(a, wl::attn::launch_attn_absorb(s, p, L.owner, T, st), "query absorption")) != WL_OK)
        return rs;
    // 4. the DSA selection (owning layers), published for the shared layers
    if (L.owner) {
        if ((rs = launched(a, wl::attn::launch_index_topk(s, p, T, st), "indexer")) != WL_OK) return rs;
        a->share_layer = (int32_t)layer;
        a->share_pos = pos;
        a->last_owner = (int32_t)layer;
    }
    // 5. attention over keys 0..pos
    const uint32_t S = wl::attn::attn_splits(s, T, kMaxSplits);
    if ((rs = launched(a, wl::attn::launch_attn_core(s, p, T, S, st), "attention")) != WL_OK) return rs;
    // 6. value projection per head, then o_proj + residual
    {
        wl::attn::GemvLaunch l{};
        uint32_t n = 0;
        auto j = job(L.w.kv_b_proj, a->ctx, a->attn, s.HN * s.VD, s.L);
        j.G = s.VD;
        j.GS = s.NP + s.VD;
        j.OFF = s.NP;
        j.XS = s.L;
        add_job(l, n, j);
        if ((rs = launched(a, wl::attn::launch_gemv(l, n, st), "value projection")) != WL_OK) return rs;
    }
    {
        wl::attn::GemvLaunch l{};
        uint32_t n = 0;
        auto j = job(L.w.o_proj, a->attn, d_hidden, s.H, s.HN * s.VD);
        j.add = d_hidden;
        j.y_raw = a->attn_out;
        add_job(l, n, j);
        if ((rs = launched(a, wl::attn::launch_gemv(l, n, st), "o_proj")) != WL_OK) return rs;
    }
    return WL_OK;
}

wl_status wl_run_dense_mlp(wl_attn* a, uint32_t layer, float* d_hidden, void* stream) {
    if (!a) return WL_ERR_INVALID;
    if (layer >= a->cfg.n_layers) return fail(a, WL_ERR_INVALID, "layer %u >= n_layers %u", layer, a->cfg.n_layers);
    AttnLayer& L = a->layers[layer];
    if (!L.dense) return fail(a, WL_ERR_STATE, "layer %u has no dense MLP (wl_attn_set_dense_mlp)", layer);
    if (!d_hidden || (uintptr_t)d_hidden % 16) return fail(a, WL_ERR_INVALID, "hidden must be 16-byte aligned");
    const wl::attn::Shape& s = a->sh;
    const wl::attn::DenseMlp m{L.post_ln, L.gate, L.up, L.down, s.H, s.DI, s.eps};
    return launched(a, wl::attn::launch_dense_mlp(m, d_hidden, d_hidden, d_hidden, a->g, a->u, a->x_norm,
                                                  a->attn_out, stream),
                    "dense MLP");
}

wl_status wl_run_layer(wl_attn* a, wl_ctx* moe, uint32_t layer, uint32_t moe_layer, uint32_t pos, float* d_hidden,
                       void* stream) {
    wl_status rs = wl_run_attention(a, layer, pos, d_hidden, stream);
    if (rs != WL_OK) return rs;
    if (a->layers[layer].dense) return wl_run_dense_mlp(a, layer, d_hidden, stream);
    if (!moe) return fail(a, WL_ERR_INVALID, "layer %u is not dense and no MoE context was given", layer);
    rs = wl::run_moe_in_place(moe, moe_layer, d_hidden, stream);
    if (rs != WL_OK) return fail(a, rs, "MoE layer %u: %s", moe_layer, wl_last_error(moe));
    return WL_OK;
}

wl_status wl_matvec_bf16(const uint16_t* d_W, const float* d_x, float* d_y, uint32_t N, uint32_t K, void* stream) {
    if (!d_W || !d_x || !d_y || N == 0 || K == 0 || K % 8 || K > 16384) return WL_ERR_INVALID;
    if (((uintptr_t)d_W | (uintptr_t)d_x) % 16) return WL_ERR_INVALID;
    wl::attn::GemvLaunch l{};
    uint32_t n = 0;
    add_job(l, n, job(d_W, d_x, d_y, N, K));
    return wl::attn::launch_gemv(l, n, stream) == 0 ? WL_OK : WL_ERR_HIP;
}

wl_status wl_attn_taps(wl_attn* a, wl_attn_taps_out* out) {
    if (!a || !out) return WL_ERR_INVALID;
    out->norm = a->x_norm;
    out->q_resid = a->q_resid;
    out->attn = a->attn;
    out->attn_out = a->attn_out;
    out->index_score = a->isc;
    out->keep = a->last_owner >= 0 ? a->layers[a->last_owner].keep : nullptr;
    return WL_OK;
}

}  // extern "C"
