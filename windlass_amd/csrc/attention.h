// attention.h — structures shared by the attention / dense-MLP kernels
// (attention.hip) and their host code (attn_host.cpp). Not public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wl {
namespace attn {

// One matrix-vector product of a GEMV launch: y[r] = add[r] + W[row(r)] . x(r)
// for r < N, with W bf16 (or f32) rows of K columns (K % 8 == 0), row(r) =
// (r / G) * GS + OFF + r % G and x(r) = x + (r / G) * XS (a grouped product,
// e.g. one x per attention head). Optional input transforms: norm_w != null
// makes x the RMSNorm of x over its K columns (x * (1/sqrt(mean(x^2) + eps))
// * norm_w, norm_w bf16 [K]); x2 != null makes x silu(x) * x2 (SwiGLU).
// x_out (optional, written by the job's first work-group): the transformed x.
// y_raw (optional): W . x without add. W2 (optional, bf16, the shape of W):
// a paired product, y[r] = silu(W[r] . x) * (W2[r] . x) (a SwiGLU's gate and
// up rows in one job; streaming kernel only).
struct GemvJob {
    const void* W;
    const void* W2;
    const float* x;
    const float* x2;
    const uint16_t* norm_w;
    float* x_out;
    float* y;
    const float* add;
    float* y_raw;
    float eps;
    uint32_t N, K;
    uint32_t G, GS, OFF, XS;
    uint32_t f32w;      // W holds f32 values
    uint32_t tpr_log2;  // threads per row: 1 << tpr_log2 (<= 256), each 8 columns per step
    uint32_t wg0;       // first work-group of this job in the launch
    uint32_t rows_wg;   // rows per work-group: kGemvRows x (256 >> tpr_log2)
    uint32_t nwg;       // streaming kernel: work-groups of this job (its rows split evenly over them)
};
constexpr int kMaxJobs = 4;
#ifndef WL_GEMV_ROWS
#define WL_GEMV_ROWS 4
#endif
constexpr uint32_t kGemvRows = WL_GEMV_ROWS;  // rows per thread group
constexpr uint32_t kGemvThreads = 256;
struct GemvLaunch {
    GemvJob job[kMaxJobs];
    uint32_t n_jobs;
};

// Shapes of the attention block (a copy of wl_attn_config's).
struct Shape {
    uint32_t H, HN, Q, L, NP, RP, VD, IH, ID, TOPK, DI;
    float eps, theta;
};

// Per-call pointers of the attention kernels (device memory).
struct AttnPtrs {
    // caches of the layer (rows [0, max_seq))
    float* kv_c;     // [max_seq][L]
    float* k_rot;    // [max_seq][RP]
    float* idx_k;    // [max_seq][ID] (owner layers)
    // weights
    const uint16_t* kv_a_ln;
    const uint16_t* kv_b;        // [HN*(NP+VD)][L]
    const uint16_t* idx_k_norm_w;
    const uint16_t* idx_k_norm_b;
    // scratch
    const float* kv_raw;   // [L + RP] kv_a_proj output
    const float* ik_raw;   // [ID] wk output
    float* iw;             // [IH] weights_proj output, scaled in place by IH^-0.5
    float iw_scale;        // IH^-0.5 (rounded from double)
    float qk_scale;        // (NP + RP)^-0.5
    float ix_scale;        // ID^-0.5
    const float* q;        // [HN][NP+RP] q_b output
    const float* iq;       // [IH][ID] wq_b output
    float* iqr;            // [IH][ID] the indexer query after RoPE
    float* q_abs;          // [HN][L]
    float* q_rope;         // [HN][RP]
    float* rope_cs;        // [RP] cos | sin of the position (written by the prep kernel)
    float* isc;            // [T] index scores
    uint8_t* keep;         // [T] 1: key kept (written by owner layers)
    uint32_t* klist;       // [max_seq + 1]: the kept keys in ascending order, [max_seq] = their count
    uint32_t max_seq;
    uint32_t kps;          // kept keys per split (multiple of 32)
    uint32_t count;        // kept keys: min(T, TOPK)
    uint32_t ident;        // 1: every key kept (klist is 0, 1, ..., T - 1 and is not read)
    uint32_t nsplit;       // splits (slots of part_m / part_l / part_ctx)
    float* part_m;         // [S][HN]
    float* part_l;         // [S][HN]
    float* part_ctx;       // [S][HN][L]
    float* ctx;            // [HN][L]
};

// Runs the jobs of l: on the streaming kernel when every job fits it (a
// paired job must), else on the row-group kernel with n_wg work-groups.
int launch_gemv(const GemvLaunch& l, uint32_t n_wg, void* stream);
// Whether every job of l fits the streaming kernel.
bool sgemv_fits(const GemvLaunch& l);
// A dense SwiGLU MLP layer (the dense branch of run_moe,
// src/glm_layer_runner.cuh:373-384): post_ln [H] bf16, gate / up [DI, H],
// down [H, DI] bf16 row-major.
struct DenseMlp {
    const uint16_t *post_ln, *gate, *up, *down;
    uint32_t H, DI;
    float eps;
};
// y = add + down(silu(gate x') * up x'), x' = RMSNorm(x) with post_ln (add may
// be null; y may alias x and add exactly: each output row reads add[r] before
// it writes y[r], and x is read by the first launch only). g, u: [DI] f32
// scratch; x_norm (optional): x'; y_raw (optional): y without add. Two
// stream-ordered launches; returns the first failing launch's hipError_t.
int launch_dense_mlp(const DenseMlp& m, const float* x, const float* add, float* y, float* g, float* u, float* x_norm,
                     float* y_raw, void* stream);
// A GEMV launch of n_wg work-groups followed by the prep stage's work-groups:
// the KV-cache row of `pos` (kv_a_layernorm of the compressed KV, RoPE of the
// shared rope key) and, on owner layers, the indexer key row (LayerNorm +
// RoPE) and the head weights' scale. Both read only the first GEMV stage.
int launch_gemv_prep(const GemvLaunch& l, uint32_t n_wg, const Shape& s, const AttnPtrs& p, uint32_t pos, bool owner,
                     void* stream);
// q_abs[h] = q_nope[h] . W_kb[h]; RoPE of q_rot (into q_rope) and, on owner
// layers, of the indexer query (into iqr), and the index scores over T keys.
int launch_attn_absorb(const Shape& s, const AttnPtrs& p, bool owner, uint32_t T, void* stream);
// The keep mask of the top-k of the index scores (all kept when T <= TOPK)
// and the list of the kept keys.
int launch_index_topk(const Shape& s, const AttnPtrs& p, uint32_t T, void* stream);
// Scores, softmax and context over the kept keys of klist (T keys at
// position T - 1), in S splits, then the combine into ctx.
uint32_t attn_splits(const Shape& s, uint32_t T, uint32_t max_splits);
size_t attn_split_lds(const Shape& s);
int launch_attn_core(const Shape& s, const AttnPtrs& p, uint32_t T, uint32_t splits, void* stream);

// Work-group count of a GEMV job (sets tpr_log2, rows_wg).
uint32_t gemv_plan(GemvJob& j);
// Dynamic LDS bytes of the index-score work-groups.
size_t index_score_lds(const Shape& s);

}  // namespace attn
}  // namespace wl
