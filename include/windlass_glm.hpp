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
//                 n_experts_per_tok, n_shared, dense_inter, routed_scaling,
//                 norm_topk_prob, rms_eps (src/glm_loader.cuh:33-69)
//   LayerWeights  router_w, router_bias, post_attn_ln, sh_gate_w, sh_gate_s,
//                 sh_up_w, sh_up_s, sh_down_w, sh_down_s, and on the dense
//                 layers mlp_gate, mlp_up, mlp_down (:259-339)
//   ExpertSource  get(layer, expert), prefetch(layer, ids, n, stream),
//                 get_async(layer, expert, stream) (src/glm_layer_runner.cuh:34-48),
//                 returning reference-layout blocks
//   PrefillBufs   n, hidden (:776-813)
//
// One library context serves every layer [0, n_layers) of each Config object
// (keyed by its address, created on first use). Like the reference's run_moe,
// run_moe on a layer below dense_first runs the dense MLP (:373-384), and on
// the others the MoE layer. A layer's weights are bound on its first call
// with a given LayerWeights object (that call synchronises the device).
//
// Experts: by default they come through the caller's ExpertSource on every
// call (the library's source path: one host round trip per layer and a
// conversion of each reference-layout block, as the reference's run_moe
// fetches per call). set_resident(c, true) before the first call makes each
// MoE layer resident on its first call instead: every expert is read once
// from the source into context-owned native blocks (wl_make_resident), and
// the layer then runs with no host round trip. It needs HBM for all experts
// of the layers run (20 MB each at the GLM shape).
//
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

// The caller's ExpertSource behind wl_expert_source (context layer = model
// layer).
template <class Src, class Stream>
struct SourceThunk {
    Src* src = nullptr;
    static const uint8_t* get(void* u, uint32_t l, uint32_t e) { return static_cast<SourceThunk*>(u)->src->get(l, e); }
    static void prefetch(void* u, uint32_t l, const int32_t* ids, uint32_t n, void* s) {
        static_cast<SourceThunk*>(u)->src->prefetch(l, ids, n, (Stream)s);
    }
    static const uint8_t* get_async(void* u, uint32_t l, uint32_t e, void* s) {
        return static_cast<SourceThunk*>(u)->src->get_async(l, e, (Stream)s);
    }
};

// The library context of one Config and what was bound to it.
struct Model {
    wl_ctx* ctx = nullptr;
    uint32_t dense_first = 0, n_layers = 0;
    bool resident = false;
    std::map<uint32_t, const void*> bound;  // layer -> the LayerWeights it was bound from
    std::map<uint32_t, bool> made_resident;
    std::shared_ptr<void> thunk;            // the SourceThunk of the last call (outlives it)
    ~Model() { wl_destroy(ctx); }
};

inline std::map<const void*, std::unique_ptr<Model>>& models() {
    static std::map<const void*, std::unique_ptr<Model>> m;
    return m;
}

template <class Config>
Model& model_for(const Config& c) {
    std::unique_ptr<Model>& m = models()[static_cast<const void*>(&c)];
    if (!m) {
        m.reset(new Model());
        m->dense_first = c.dense_first;
        m->n_layers = c.n_layers;
        wl_moe_config wc{c.hidden, c.moe_inter, c.n_routed_experts, c.n_experts_per_tok, c.n_shared,
                         c.n_layers, c.routed_scaling, c.norm_topk_prob ? 1 : 0, c.rms_eps};
        check(nullptr, wl_create(&wc, &m->ctx), "wl_create");
    }
    return *m;
}

// Opt-in: the MoE layers of this Config become resident on their first call
// (see the header comment). Set it before the first call of a layer.
template <class Config>
void set_resident(const Config& c, bool on) {
    model_for(c).resident = on;
}

// The library context behind this Config (its taps, error checks, schedule).
template <class Config>
wl_ctx* context(const Config& c) {
    return model_for(c).ctx;
}

// Binds layer `layer` from w: the dense MLP below dense_first, else the
// router, bias, norm and MXFP4 shared expert.
template <class Config, class LayerWeights>
void bind_layer(Model& m, const Config& c, const LayerWeights& w, uint32_t layer) {
    if (layer >= m.n_layers) {
        std::fprintf(stderr, "windlass_glm: layer %u >= n_layers %u\n", layer, m.n_layers);
        std::abort();
    }
    auto it = m.bound.find(layer);
    if (it != m.bound.end() && it->second == static_cast<const void*>(&w)) return;
    if (layer < m.dense_first)
        check(m.ctx, wl_set_layer_dense(m.ctx, layer, w.post_attn_ln, w.mlp_gate, w.mlp_up, w.mlp_down, c.dense_inter),
              "wl_set_layer_dense");
    else
        check(m.ctx,
              wl_set_layer_mxfp4(m.ctx, layer, w.router_w, w.router_bias, w.post_attn_ln, w.sh_gate_w, w.sh_gate_s,
                                 w.sh_up_w, w.sh_up_s, w.sh_down_w, w.sh_down_s),
              "wl_set_layer_mxfp4");
    m.bound[layer] = static_cast<const void*>(&w);
}

// Routes the context's expert source to `src`, and in resident mode makes a
// MoE layer resident on its first call.
template <class ExpertSource, class Stream>
void attach_source(Model& m, ExpertSource& src, uint32_t layer, Stream stream) {
    if (layer < m.dense_first) return;
    auto t = std::make_shared<SourceThunk<ExpertSource, Stream>>();
    t->src = &src;
    const wl_expert_source s{t.get(), &SourceThunk<ExpertSource, Stream>::get,
                             &SourceThunk<ExpertSource, Stream>::prefetch,
                             &SourceThunk<ExpertSource, Stream>::get_async, 0};
    check(m.ctx, wl_set_expert_source(m.ctx, &s), "wl_set_expert_source");
    m.thunk = t;
    if (m.resident && !m.made_resident[layer]) {
        check(m.ctx, wl_make_resident(m.ctx, layer, (void*)stream), "wl_make_resident");
        m.made_resident[layer] = true;
    }
}

}  // namespace windlass_glm

namespace glm {

// run_moe (src/glm_layer_runner.cuh:352-443): d_out = the block output of
// layer `layer` for the pre-norm hidden state d_hidden, without the residual:
// the dense MLP below dense_first (:373-384), the MoE layer above. d_out must
// not alias d_hidden. `lay` is not needed: the library derives the same
// offsets from the config (ExpertLayout::from).
template <class Config, class LayerWeights, class ExpertLayout, class ExpertSource, class Stream>
inline void run_moe(const Config& c, const LayerWeights& w, const ExpertLayout& lay, ExpertSource& src,
                    uint32_t layer, const float* d_hidden, float* d_out, Stream stream) {
    (void)lay;
    windlass_glm::Model& m = windlass_glm::model_for(c);
    windlass_glm::bind_layer(m, c, w, layer);
    windlass_glm::attach_source<ExpertSource, Stream>(m, src, layer, stream);
    windlass_glm::check(m.ctx, wl_run_moe(m.ctx, layer, d_hidden, d_out, (void*)stream), "wl_run_moe");
}

// run_moe_batched (src/glm_layer_runner.cuh:818-928): b.hidden[i] +=
// moe(b.hidden[i]) for the b.n positions, every unique routed expert fetched
// once through `src` (a dense layer runs its MLP per position).
template <class Config, class LayerWeights, class ExpertLayout, class ExpertSource, class PrefillBufs,
          class Stream>
inline void run_moe_batched(const Config& c, const LayerWeights& w, const ExpertLayout& lay, ExpertSource& src,
                            uint32_t layer, PrefillBufs& b, Stream stream) {
    (void)lay;
    windlass_glm::Model& m = windlass_glm::model_for(c);
    windlass_glm::bind_layer(m, c, w, layer);
    windlass_glm::attach_source<ExpertSource, Stream>(m, src, layer, stream);
    windlass_glm::check(m.ctx, wl_run_moe_batched(m.ctx, layer, b.n, b.hidden, b.hidden, b.hidden, (void*)stream),
                        "wl_run_moe_batched");
}

}  // namespace glm

#endif  // WINDLASS_GLM_HPP
