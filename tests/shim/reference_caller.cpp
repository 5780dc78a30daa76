// A caller written against the reference's MoE call surface, compiled against
// include/windlass_glm.hpp instead of the reference's CUDA headers, and run
// on the GPU by tests/test_gpu_shim.py and bench.py --workload shim.
//
// The stand-in types carry the fields and member functions the reference
// declares for them (src/glm_loader.cuh:33-69,259-339;
// src/glm_layer_runner.cuh:34-72,776-813). decode_step and prefill are the
// reference's call sites: run_layer's MoE half (:674-675: run_moe into s_acc,
// then residual_add) over every layer from 0, as run_chain loops
// (:1065-1068), and the layer-major prefill's MoE half (:985-999: dense layers
// per position, the others through run_moe_batched).
//
// Usage: reference_caller DIR MODE [BENCH_ITERS]
//   DIR holds cfg.txt and the layers' dense tensors as raw files (written by
//   the test or the bench); routed experts and the MXFP4 shared experts are
//   the library's synthetic blocks (wl_synth_expert, reference layout),
//   served by an ExpertSource over one device pool.
//   MODE: "source" (experts through the source on every call) or "resident"
//   (windlass_glm::set_resident).
//   Without BENCH_ITERS: writes out_decode.bin [n_layers][H] (hidden after
//   each layer), ids_decode.bin [n_layers][K] (-1 on dense layers) and
//   out_prefill.bin [n_layers][T][H]. With BENCH_ITERS: times that many
//   decode steps (every layer once per step) and prints one JSON line with
//   the mean time of a dense and of a MoE layer.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "windlass_glm.hpp"

#define HIP_OK(x)                                                                             \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            std::exit(2);                                                                     \
        }                                                                                     \
    } while (0)

namespace glm {

struct Config {
    uint32_t n_layers, hidden, n_routed_experts, n_experts_per_tok, moe_inter, n_shared, dense_first, kv_lora_rank,
        q_lora_rank, vocab;
    float rms_eps, rope_theta;
    uint32_t n_heads, qk_nope, qk_rope, qk_head, v_head, dense_inter;
    float routed_scaling;
    bool norm_topk_prob;
};

struct LayerWeights {
    uint16_t *input_ln, *post_attn_ln;
    uint16_t* router_w;
    float* router_bias;
    uint8_t *sh_gate_w, *sh_gate_s, *sh_up_w, *sh_up_s, *sh_down_w, *sh_down_s;
    uint16_t *mlp_gate, *mlp_up, *mlp_down;
    float* s_acc;
};

struct ExpertLayout {
    size_t gw_off, gw_len, gs_off, gs_len, uw_off, uw_len, us_off, us_len, dw_off, dw_len, ds_off, ds_len, total;
};

struct ExpertSource {
    virtual uint8_t* get(uint32_t layer, uint32_t expert) = 0;
    virtual void prefetch(uint32_t, const int32_t*, uint32_t, hipStream_t) {}
    virtual uint8_t* get_async(uint32_t layer, uint32_t expert, hipStream_t) { return get(layer, expert); }
    virtual ~ExpertSource() = default;
};

struct PrefillBufs {
    uint32_t n = 0, H = 0, K = 0;
    float* hidden = nullptr;
    float* norm = nullptr;
};

// residual_add (src/glm_primitives.cuh:69-77): out = a + b.
__global__ void residual_add(const float* a, const float* b, float* out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// run_layer's MoE half (src/glm_layer_runner.cuh:674-675) for one layer.
void moe_half(const Config& c, const LayerWeights& w, const ExpertLayout& lay, ExpertSource& src, uint32_t l,
              float* d_hidden, hipStream_t stream) {
    run_moe(c, w, lay, src, l, d_hidden, w.s_acc, stream);
    residual_add<<<(c.hidden + 255) / 256, 256, 0, stream>>>(d_hidden, w.s_acc, d_hidden, c.hidden);
}

// The layer loop of run_chain (:1065-1068), MoE halves only.
void decode_step(const Config& c, const std::vector<LayerWeights>& W, const ExpertLayout& lay, ExpertSource& src,
                 float* d_hidden, hipStream_t stream) {
    for (uint32_t l = 0; l < c.n_layers; l++) moe_half(c, W[l], lay, src, l, d_hidden, stream);
}

// The layer-major prefill's MoE half (:985-999) for one layer.
void prefill_layer(const Config& c, const std::vector<LayerWeights>& W, const ExpertLayout& lay, ExpertSource& src,
                   uint32_t l, PrefillBufs& b, hipStream_t stream) {
    if (l < c.dense_first) {
        for (uint32_t i = 0; i < b.n; i++) {
            float* hid_i = b.hidden + (size_t)i * c.hidden;
            run_moe(c, W[l], lay, src, l, hid_i, W[l].s_acc, stream);
            residual_add<<<(c.hidden + 255) / 256, 256, 0, stream>>>(hid_i, W[l].s_acc, hid_i, c.hidden);
        }
    } else {
        run_moe_batched(c, W[l], lay, src, l, b, stream);
    }
}

}  // namespace glm

// Every routed expert of the MoE layers in one device pool, reference layout.
struct PoolSource : glm::ExpertSource {
    std::vector<uint8_t*> blocks;  // [n_layers * E]
    uint32_t E = 0;
    uint8_t* get(uint32_t layer, uint32_t expert) override { return blocks[(size_t)layer * E + expert]; }
};

static std::vector<uint8_t> read_file(const std::string& path, size_t expect) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) {
        std::fprintf(stderr, "cannot open %s\n", path.c_str());
        std::exit(2);
    }
    std::vector<uint8_t> v(expect);
    const size_t got = std::fread(v.data(), 1, expect, f);
    std::fclose(f);
    if (got != expect) {
        std::fprintf(stderr, "%s: %zu of %zu bytes\n", path.c_str(), got, expect);
        std::exit(2);
    }
    return v;
}

template <class T>
static T* upload(const std::string& path, size_t bytes) {
    std::vector<uint8_t> h = read_file(path, bytes);
    void* d = nullptr;
    HIP_OK(hipMalloc(&d, bytes));
    HIP_OK(hipMemcpy(d, h.data(), bytes, hipMemcpyHostToDevice));
    return (T*)d;
}

static void write_file(const std::string& path, const void* p, size_t bytes) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(p, 1, bytes, f) != bytes) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s DIR source|resident [BENCH_ITERS]\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1], mode = argv[2];
    const int bench = argc > 3 ? std::atoi(argv[3]) : 0;
    // cfg.txt: n_layers dense_first hidden moe_inter E K n_shared dense_inter T seed rms_eps routed_scaling
    glm::Config c{};
    uint32_t T = 0, seed = 0;
    {
        FILE* f = std::fopen((dir + "/cfg.txt").c_str(), "r");
        if (!f || std::fscanf(f, "%u %u %u %u %u %u %u %u %u %u %f %f", &c.n_layers, &c.dense_first, &c.hidden,
                              &c.moe_inter, &c.n_routed_experts, &c.n_experts_per_tok, &c.n_shared, &c.dense_inter,
                              &T, &seed, &c.rms_eps, &c.routed_scaling) != 12) {
            std::fprintf(stderr, "bad %s/cfg.txt\n", dir.c_str());
            return 2;
        }
        std::fclose(f);
    }
    c.norm_topk_prob = true;
    const uint32_t H = c.hidden, E = c.n_routed_experts, K = c.n_experts_per_tok, SI = c.moe_inter * c.n_shared;
    const wl_moe_config wc{H, c.moe_inter, E, K, c.n_shared, c.n_layers, c.routed_scaling, 1, c.rms_eps};
    wl_expert_layout el{}, sl{};
    if (wl_expert_layout_of(&wc, 0, &el) != WL_OK || wl_expert_layout_of(&wc, SI, &sl) != WL_OK) return 2;
    const glm::ExpertLayout lay{el.gw_off, el.gw_len, el.gs_off, el.gs_len, el.uw_off, el.uw_len, el.us_off,
                                el.us_len, el.dw_off, el.dw_len, el.ds_off, el.ds_len, el.total};
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));

    // weights: dense tensors from DIR, experts and MXFP4 shared experts from the generator
    PoolSource src;
    src.E = E;
    src.blocks.assign((size_t)c.n_layers * E, nullptr);
    std::vector<glm::LayerWeights> W(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        glm::LayerWeights& w = W[l];
        std::memset(&w, 0, sizeof(w));
        const std::string p = dir + "/l" + std::to_string(l) + "_";
        w.post_attn_ln = upload<uint16_t>(p + "ln.bin", 2 * (size_t)H);
        HIP_OK(hipMalloc(&w.s_acc, 4 * (size_t)H));
        if (l < c.dense_first) {
            const size_t DI = c.dense_inter;
            w.mlp_gate = upload<uint16_t>(p + "gate.bin", 2 * DI * H);
            w.mlp_up = upload<uint16_t>(p + "up.bin", 2 * DI * H);
            w.mlp_down = upload<uint16_t>(p + "down.bin", 2 * DI * H);
            continue;
        }
        w.router_w = upload<uint16_t>(p + "router.bin", 2 * (size_t)E * H);
        w.router_bias = upload<float>(p + "bias.bin", 4 * (size_t)E);
        uint8_t* sh = nullptr;
        HIP_OK(hipMalloc(&sh, sl.total));
        if (wl_synth_expert(&wc, SI, seed, l, 0xFFFFu, sh, stream) != WL_OK) return 2;
        w.sh_gate_w = sh + sl.gw_off;
        w.sh_gate_s = sh + sl.gs_off;
        w.sh_up_w = sh + sl.uw_off;
        w.sh_up_s = sh + sl.us_off;
        w.sh_down_w = sh + sl.dw_off;
        w.sh_down_s = sh + sl.ds_off;
        uint8_t* pool = nullptr;
        HIP_OK(hipMalloc(&pool, (size_t)E * el.total));
        for (uint32_t e = 0; e < E; e++) {
            src.blocks[(size_t)l * E + e] = pool + (size_t)e * el.total;
            if (wl_synth_expert(&wc, 0, seed, l, e, src.blocks[(size_t)l * E + e], stream) != WL_OK) return 2;
        }
    }
    HIP_OK(hipStreamSynchronize(stream));
    if (mode == "resident") windlass_glm::set_resident(c, true);
    else if (mode != "source") return 2;
    wl_ctx* ctx = windlass_glm::context(c);

    std::vector<float> h0 = [&] {
        std::vector<uint8_t> b = read_file(dir + "/h0.bin", 4 * (size_t)T * H);
        std::vector<float> v((size_t)T * H);
        std::memcpy(v.data(), b.data(), b.size());
        return v;
    }();
    float* d_h = nullptr;
    HIP_OK(hipMalloc(&d_h, 4 * (size_t)T * H));

    if (bench > 0) {
        // decode steps over every layer (a warm-up step binds each layer and,
        // resident, fills it), the hidden state rotating over the T inputs so
        // the routing changes; events at every layer boundary give each
        // layer's time, host round trips of the source path included
        HIP_OK(hipMemcpy(d_h, h0.data(), 4 * (size_t)T * H, hipMemcpyHostToDevice));
        for (int it = 0; it < 2; it++) glm::decode_step(c, W, lay, src, d_h + (size_t)(it % T) * H, stream);
        HIP_OK(hipStreamSynchronize(stream));
        std::vector<hipEvent_t> ev((size_t)bench * (c.n_layers + 1));
        for (hipEvent_t& e : ev) HIP_OK(hipEventCreate(&e));
        const auto t0 = std::chrono::steady_clock::now();
        for (int it = 0; it < bench; it++) {
            float* h = d_h + (size_t)(it % T) * H;
            hipEvent_t* e = &ev[(size_t)it * (c.n_layers + 1)];
            HIP_OK(hipEventRecord(e[0], stream));
            for (uint32_t l = 0; l < c.n_layers; l++) {
                glm::moe_half(c, W[l], lay, src, l, h, stream);
                HIP_OK(hipEventRecord(e[l + 1], stream));
            }
        }
        HIP_OK(hipStreamSynchronize(stream));
        const double wall_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        double us_dense = 0.0, us_moe = 0.0;
        for (int it = 0; it < bench; it++)
            for (uint32_t l = 0; l < c.n_layers; l++) {
                float ms = 0.f;
                const hipEvent_t* e = &ev[(size_t)it * (c.n_layers + 1)];
                HIP_OK(hipEventElapsedTime(&ms, e[l], e[l + 1]));
                (l < c.dense_first ? us_dense : us_moe) += 1000.0 * ms;
            }
        if (wl_check_error(ctx, stream) != WL_OK) {
            std::fprintf(stderr, "device error: %s\n", wl_last_error(ctx));
            return 3;
        }
        const uint32_t n_moe = c.n_layers - c.dense_first;
        std::printf("{\"mode\": \"%s\", \"us_per_moe_layer\": %.3f, \"us_per_dense_layer\": %.3f, "
                    "\"moe_layers\": %u, \"dense_layers\": %u, \"steps\": %d, \"wall_us_per_step\": %.1f}\n",
                    mode.c_str(), n_moe ? us_moe / ((double)bench * n_moe) : 0.0,
                    c.dense_first ? us_dense / ((double)bench * c.dense_first) : 0.0, n_moe, c.dense_first, bench,
                    wall_us / bench);
        return 0;
    }

    // decode: token 0 through every layer, the hidden state after each layer
    std::vector<float> out((size_t)c.n_layers * H);
    std::vector<int32_t> ids((size_t)c.n_layers * K, -1);
    HIP_OK(hipMemcpy(d_h, h0.data(), 4 * (size_t)H, hipMemcpyHostToDevice));
    for (uint32_t l = 0; l < c.n_layers; l++) {
        glm::moe_half(c, W[l], lay, src, l, d_h, stream);
        HIP_OK(hipStreamSynchronize(stream));
        HIP_OK(hipMemcpy(&out[(size_t)l * H], d_h, 4 * (size_t)H, hipMemcpyDeviceToHost));
        if (l >= c.dense_first) {
            wl_taps_out t{};
            if (wl_taps(ctx, &t) != WL_OK) return 2;
            HIP_OK(hipMemcpy(&ids[(size_t)l * K], t.topk_idx, 4 * (size_t)K, hipMemcpyDeviceToHost));
        }
    }
    // the same through decode_step (one call over all layers): the same bits
    HIP_OK(hipMemcpy(d_h, h0.data(), 4 * (size_t)H, hipMemcpyHostToDevice));
    glm::decode_step(c, W, lay, src, d_h, stream);
    std::vector<float> last(H);
    HIP_OK(hipMemcpy(last.data(), d_h, 4 * (size_t)H, hipMemcpyDeviceToHost));
    if (std::memcmp(last.data(), &out[(size_t)(c.n_layers - 1) * H], 4 * (size_t)H) != 0) {
        std::fprintf(stderr, "decode_step differs from the per-layer loop\n");
        return 4;
    }
    // prefill of the T positions, layer-major
    std::vector<float> pout((size_t)c.n_layers * T * H);
    HIP_OK(hipMemcpy(d_h, h0.data(), 4 * (size_t)T * H, hipMemcpyHostToDevice));
    glm::PrefillBufs b;
    b.n = T;
    b.H = H;
    b.K = K;
    b.hidden = d_h;
    for (uint32_t l = 0; l < c.n_layers; l++) {
        glm::prefill_layer(c, W, lay, src, l, b, stream);
        HIP_OK(hipStreamSynchronize(stream));
        HIP_OK(hipMemcpy(&pout[(size_t)l * T * H], d_h, 4 * (size_t)T * H, hipMemcpyDeviceToHost));
    }
    if (wl_check_error(ctx, stream) != WL_OK) {
        std::fprintf(stderr, "device error: %s\n", wl_last_error(ctx));
        return 3;
    }
    write_file(dir + "/out_decode.bin", out.data(), 4 * out.size());
    write_file(dir + "/ids_decode.bin", ids.data(), 4 * ids.size());
    write_file(dir + "/out_prefill.bin", pout.data(), 4 * pout.size());
    std::printf("reference_caller %s: %u layers (%u dense), %u prefill positions: done\n", mode.c_str(), c.n_layers,
                c.dense_first, T);
    return 0;
}
