// windlass_glm.hpp — header-only C++ drop-in for the reference's MoE call
// surface, over the C ABI of windlass_moe.h.
//
// It keeps the spellings of glm::run_moe (src/glm_layer_runner.cuh:352-354)
// and glm::run_moe_batched (:818-820), templated over the caller's own
// Config, LayerWeights, ExpertLayout, ExpertSource, PrefillBufs and stream
// types, so a caller that stops including the reference's definitions and
// includes this header compiles unchanged. (If both are visible, the
// reference's non-template functions win overload resolution and this
// header goes unused.) The fields read are the reference's:
//   Config        n_layers, dense_first, hidden, moe_inter, n_routed_experts,
//                 n_experts_per_tok, n_shared, routed_scaling, norm_topk_prob,
//                 rms_eps (src/glm_loader.cuh:33-69)
//   LayerWeights  router_w, router_bias, post_attn_ln, sh_gate_w, sh_gate_s,
//                 sh_up_w, sh_up_s, sh_down_w, sh_down_s (:259-339)
//   ExpertSource  get(layer, expert), prefetch(layer, ids, n, stream),
//                 get_async(layer, expert, stream) (src/glm_layer_runner.cuh:34-48),
//                 returning reference-layout blocks
//   PrefillBufs   n, hidden (:776-813)
//
// One library context serves the MoE layers [dense_first, n_layers) of each
// Config object (keyed by its address, created on first use); a layer's
// router, bias, norm and MXFP4 shared expert are bound on its first call with
// a given LayerWeights object (that call synchronises the device). Experts
// come through the caller's ExpertSource on every call (the library's source
// path: one host round trip per layer, as the reference's run_moe). A caller
// that keeps its experts resident gets the faster path by binding them once
// with wl_slot_bind (wl_slot_pool_create + wl_expert_to_native fill the
// slots). The dense-MLP layers below
// dense_first are not part of the MoE path: calling run_moe on one aborts.
// Errors abort with the library's message, the reference's error policy
// (GLM_CUDA_OK -> abort, src/glm_loader.cuh:24-26). One host thread, as in
// the reference.
#ifndef WINDLASS_GLM_HPP
#define WINDLASS_GLM_HPP

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <memory>

#include "windlass_moe.h"

namespace windlass_glm {

inline void check(wl_ctx* ctx, wl_status s, const char* what) {
    if (s != WL_OK) {
        std::fprintf(stderr, "%s: status %d: %s\n", what, (int)s, ctx ? wl_last_error(ctx) : "no context");
        std::abort();
    }
}

// The caller's ExpertSource behind wl_expert_source: context layer l is
// model layer first + l.
template <class Src, class Stream>
struct SourceThunk {
    Src* src = nullptr;
    uint32_t first = 0;
    static const uint8_t* get(void* u, uint32_t l, uint32_t e) {
        auto* t = static_cast<SourceThunk*>(u);
        return t->src->get(t->first + l, e);
    }
    static void prefetch(void* u, uint32_t l, const int32_t* ids, uint32_t n, void* s) {
        auto* t = static_cast<SourceThunk*>(u);
        t->src->prefetch(t->first + l, ids, n, (Stream)s);
    }
    static const uint8_t* get_async(void* u, uint32_t l, uint32_t e, void* s) {
        auto* t = static_cast<SourceThunk*>(u);
        return t->src->get_async(t->first + l, e, (Stream)s);
    }
};

// The library context of one Config and what was bound to it.
struct Model {
    wl_ctx* ctx = nullptr;
    uint32_t first = 0, n_moe = 0;
    std::map<uint32_t, const void*> bound;  // context layer -> the LayerWeights it was bound from
    std::shared_ptr<void> thunk;            // the SourceThunk of the last call (outlives it)
    ~Model() { wl_destroy(ctx); }
};

template <class Config>
Model& model_for(const Config& c) {
    static std::map<const void*, std::unique_ptr<Model>> models;
    std::unique_ptr<Model>& m = models[static_cast<const void*>(&c)];
    if (!m) {
        m.reset(new Model());
        m->first = c.dense_first;
        m->n_moe = c.n_layers - c.dense_first;
        wl_moe_config wc{c.hidden, c.moe_inter, c.n_routed_experts, c.n_experts_per_tok, c.n_shared,
                         m->n_moe, c.routed_scaling, c.norm_topk_prob ? 1 : 0, c.rms_eps};
        check(nullptr, wl_create(&wc, &m->ctx), "wl_create");
    }
    return *m;
}

// Context layer of model layer `layer`, with its weights bound from w.
template <class Config, class LayerWeights>
uint32_t bind_layer(Model& m, const Config& c, const LayerWeights& w, uint32_t layer) {
    (void)c;
    if (layer < m.first || layer - m.first >= m.n_moe) {
        std::fprintf(stderr, "windlass_glm: layer %u is not a MoE layer [%u, %u)\n", layer, m.first,
                     m.first + m.n_moe);
        std::abort();
    }
    const uint32_t l = layer - m.first;
    auto it = m.bound.find(l);
    if (it == m.bound.end() || it->second != static_cast<const void*>(&w)) {
        check(m.ctx,
              wl_set_layer_mxfp4(m.ctx, l, w.router_w, w.router_bias, w.post_attn_ln, w.sh_gate_w, w.sh_gate_s,
                                 w.sh_up_w, w.sh_up_s, w.sh_down_w, w.sh_down_s),
              "wl_set_layer_mxfp4");
        m.bound[l] = static_cast<const void*>(&w);
    }
    return l;
}

template <class ExpertSource, class Stream>
void attach_source(Model& m, ExpertSource& src) {
    auto t = std::make_shared<SourceThunk<ExpertSource, Stream>>();
    t->src = &src;
    t->first = m.first;
    const wl_expert_source s{t.get(), &SourceThunk<ExpertSource, Stream>::get,
                             &SourceThunk<ExpertSource, Stream>::prefetch,
                             &SourceThunk<ExpertSource, Stream>::get_async, 0};
    check(m.ctx, wl_set_expert_source(m.ctx, &s), "wl_set_expert_source");
    m.thunk = t;
}

}  // namespace windlass_glm

namespace glm {

// run_moe (src/glm_layer_runner.cuh:352-443): d_out = the MoE block output of
// layer `layer` for the pre-norm hidden state d_hidden (no residual); d_out
// must not alias d_hidden. `lay` is not needed: the library derives the same
// offsets from the config (ExpertLayout::from).
template <class Config, class LayerWeights, class ExpertLayout, class ExpertSource, class Stream>
inline void run_moe(const Config& c, const LayerWeights& w, const ExpertLayout& lay, ExpertSource& src,
                    uint32_t layer, const float* d_hidden, float* d_out, Stream stream) {
    (void)lay;
    windlass_glm::Model& m = windlass_glm::model_for(c);
    const uint32_t l = windlass_glm::bind_layer(m, c, w, layer);
    windlass_glm::attach_source<ExpertSource, Stream>(m, src);
    windlass_glm::check(m.ctx, wl_run_moe(m.ctx, l, d_hidden, d_out, (void*)stream), "wl_run_moe");
}

// run_moe_batched (src/glm_layer_runner.cuh:818-928): b.hidden[i] +=
// moe(b.hidden[i]) for the b.n positions, every unique routed expert fetched
// once through `src`.
template <class Config, class LayerWeights, class ExpertLayout, class ExpertSource, class PrefillBufs,
          class Stream>
inline void run_moe_batched(const Config& c, const LayerWeights& w, const ExpertLayout& lay, ExpertSource& src,
                            uint32_t layer, PrefillBufs& b, Stream stream) {
    (void)lay;
    windlass_glm::Model& m = windlass_glm::model_for(c);
    const uint32_t l = windlass_glm::bind_layer(m, c, w, layer);
    windlass_glm::attach_source<ExpertSource, Stream>(m, src);
    windlass_glm::check(m.ctx, wl_run_moe_batched(m.ctx, l, b.n, b.hidden, b.hidden, b.hidden, (void*)stream),
                        "wl_run_moe_batched");
}

}  // namespace glm

#endif  // WINDLASS_GLM_HPP
