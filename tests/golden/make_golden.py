"""Writes the golden fixtures under tests/golden/ from INDEPENDENT sources.

Run in the build container: python tests/golden/make_golden.py

* mxfp4_hand_fixture.json — the reference's hand-computed MXFP4 known answer
  (tools/glm_mxfp4_numpy.py:44-52), restated as data.
* dequant_tf.npz — MXFP4 dequant of random blocks by transformers'
  integrations.mxfp4._convert_moe_packed_tensors (transformers 5.15.0), an
  implementation independent of the reference and of this repository.
* moe_tf_small.npz — one small GLM MoE layer (RMSNorm + GlmMoeDsaMoE: router,
  routed experts, shared expert) run by transformers' modeling_glm_moe_dsa in
  float32 on this repository's synthetic inputs (oracle/synth.py), with the
  routed MXFP4 experts dequantised by transformers. Stores the expected
  substeps, not the inputs (the inputs are regenerated from the seeds).
* attn_tf_small.npz — two small MLA attention layers with the DSA indexer
  (layer 0 "full", layer 1 "shared": it reuses layer 0's selection) and a
  dense MLP, run by transformers' GlmMoeDsaAttention / GlmMoeDsaMLP in
  float32 (eager) over a 12-position sequence, with weights from
  windlass_amd.synthdata.attention_layer / dense_mlp; stores each
  position's o_proj output, the indexer's selection (as a keep mask over the
  causal keys) and the MLP outputs.

Neither the reference's Python nor this repository's oracle computes any
expected value here.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import synth  # noqa: E402  (inputs only)
from windlass_amd import synthdata  # noqa: E402  (inputs only)

from transformers.integrations.mxfp4 import _convert_moe_packed_tensors  # noqa: E402
from transformers.models.glm_moe_dsa import modeling_glm_moe_dsa as M  # noqa: E402
from transformers.models.glm_moe_dsa.configuration_glm_moe_dsa import GlmMoeDsaConfig  # noqa: E402

SMALL = dict(hidden=256, moe_inter=128, n_routed_experts=32, n_experts_per_tok=4, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
SMALL_SEEDS = [0, 1, 2, 3, 4, 5]


def tf_dequant(w, s):
    # The function takes [experts, rows, blocks, 16] and returns [experts, K, rows]
    # (GPT-OSS stores the transpose); one expert here, transposed back to [N, K].
    n, half = w.shape
    blocks = torch.from_numpy(w.reshape(1, n, half // 16, 16).copy())
    scales = torch.from_numpy(s.reshape(1, n, half // 16).copy())
    out = _convert_moe_packed_tensors(blocks, scales, dtype=torch.float32)
    return out[0].transpose(0, 1).contiguous().numpy()


def hand_fixture():
    # tools/glm_mxfp4_numpy.py:44-52: 16 bytes, one scale byte 128 (x2.0)
    w = [0x21, 0x43, 0x65, 0x87, 0xA9, 0xCB, 0xED, 0x0F] + [0x00] * 8
    expected = [1.0, 2.0, 3.0, 4.0, 6.0, 8.0, 12.0, -0.0, -1.0, -2.0, -3.0, -4.0, -6.0, -8.0, -12.0, 0.0] + [0.0] * 16
    return {"source": "tools/glm_mxfp4_numpy.py:44-52", "w": w, "s": [128], "expected": expected,
            "negative_zero_index": 7}


def dequant_fixture():
    rng = np.random.default_rng(20261201)
    N, K = 16, 256
    w = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    s = rng.integers(118, 135, size=(N, K // 32), dtype=np.uint8)
    s[0, :4] = [1, 127, 200, 254]  # far corners of the finite E8M0 range
    return {"w": w, "s": s, "expected": tf_dequant(w, s)}


def moe_small(seed):
    c = SMALL
    H, I, E, K = c["hidden"], c["moe_inter"], c["n_routed_experts"], c["n_experts_per_tok"]
    SI = I * c["n_shared"]
    cfg = GlmMoeDsaConfig(hidden_size=H, moe_intermediate_size=I, n_routed_experts=E,
                          num_experts_per_tok=K, n_shared_experts=c["n_shared"],
                          routed_scaling_factor=c["routed_scaling"], n_group=1, topk_group=1,
                          norm_topk_prob=True, num_hidden_layers=4, hidden_act="silu",
                          rms_norm_eps=c["rms_eps"])
    moe = M.GlmMoeDsaMoE(cfg).float().eval()
    norm = M.GlmMoeDsaRMSNorm(H, eps=c["rms_eps"]).float().eval()
    dense = synth.dense_layer(H, E, SI, seed, 0)
    with torch.no_grad():
        moe.gate.weight.copy_(torch.from_numpy(synth.bf16_to_f32(dense["router_w"])))
        moe.gate.e_score_correction_bias.copy_(torch.from_numpy(dense["bias"]))
        for e in range(E):
            gw, gs, uw, us, dw, ds = synth.expert_block(H, I, seed, 0, e)
            moe.experts.gate_up_proj[e].copy_(torch.from_numpy(np.concatenate([tf_dequant(gw, gs), tf_dequant(uw, us)])))
            moe.experts.down_proj[e].copy_(torch.from_numpy(tf_dequant(dw, ds)))
        moe.shared_experts.gate_proj.weight.copy_(torch.from_numpy(synth.bf16_to_f32(dense["sh_gate"])))
        moe.shared_experts.up_proj.weight.copy_(torch.from_numpy(synth.bf16_to_f32(dense["sh_up"])))
        moe.shared_experts.down_proj.weight.copy_(torch.from_numpy(synth.bf16_to_f32(dense["sh_down"])))
        norm.weight.fill_(1.0)
        h = torch.from_numpy(synth.hidden_state(H, seed)).reshape(1, H)
        xn = norm(h)
        logits, topw, topi = moe.gate(xn)
        shared = moe.shared_experts(xn)
        out = moe(xn)
        scores = torch.sigmoid(logits) + moe.gate.e_score_correction_bias
        srt = torch.sort(scores[0], descending=True).values
    ids = topi[0].numpy().astype(np.int32)
    order = np.argsort(ids)
    return {"norm": xn[0].numpy(), "logits": logits[0].numpy(), "topk_idx_sorted": ids[order],
            "topk_w_by_sorted_id": topw[0].numpy()[order].astype(np.float32),
            "shared": shared[0].numpy(), "out": out[0].numpy(),
            "margin": np.float32(srt[K - 1] - srt[K])}


ATT = dict(hidden=256, n_heads=4, q_lora_rank=64, kv_lora_rank=32, qk_nope=16, qk_rope=16, v_head=24,
           index_n_heads=4, index_head_dim=32, index_topk=6, dense_inter=384, rms_eps=1e-5, rope_theta=10000.0)
ATT_SEQ, ATT_SEED = 12, 7


def attn_small():
    a = ATT
    H, S = a["hidden"], ATT_SEQ
    cfg = GlmMoeDsaConfig(hidden_size=H, num_attention_heads=a["n_heads"], num_key_value_heads=a["n_heads"],
                          q_lora_rank=a["q_lora_rank"], kv_lora_rank=a["kv_lora_rank"],
                          qk_nope_head_dim=a["qk_nope"], qk_rope_head_dim=a["qk_rope"], v_head_dim=a["v_head"],
                          index_n_heads=a["index_n_heads"], index_head_dim=a["index_head_dim"],
                          index_topk=a["index_topk"], intermediate_size=a["dense_inter"], num_hidden_layers=2,
                          first_k_dense_replace=1, indexer_types=["full", "shared"], rms_norm_eps=a["rms_eps"],
                          rope_parameters={"rope_type": "default", "rope_theta": a["rope_theta"]},
                          hidden_act="silu", attention_bias=False)
    cfg._attn_implementation = "eager"
    rot = M.GlmMoeDsaRotaryEmbedding(cfg)
    pos = torch.arange(S).reshape(1, S)
    out = {}
    prev = None
    for layer in range(2):
        w = synthdata.as_f32(synthdata.attention_layer(a, ATT_SEED, layer, owner=(layer == 0)))
        att = M.GlmMoeDsaAttention(cfg, layer).float().eval()
        norm = M.GlmMoeDsaRMSNorm(H, eps=a["rms_eps"]).float().eval()
        t = lambda k: torch.from_numpy(w[k])
        with torch.no_grad():
            norm.weight.copy_(t("input_ln"))
            att.q_a_proj.weight.copy_(t("q_a_proj"))
            att.q_a_layernorm.weight.copy_(t("q_a_ln"))
            att.q_b_proj.weight.copy_(t("q_b_proj"))
            att.kv_a_proj_with_mqa.weight.copy_(t("kv_a_proj"))
            att.kv_a_layernorm.weight.copy_(t("kv_a_ln"))
            att.kv_b_proj.weight.copy_(t("kv_b_proj"))
            att.o_proj.weight.copy_(t("o_proj"))
            if layer == 0:
                att.indexer.wq_b.weight.copy_(t("idx_wq_b"))
                att.indexer.wk.weight.copy_(t("idx_wk"))
                att.indexer.k_norm.weight.copy_(t("idx_k_norm_w"))
                att.indexer.k_norm.bias.copy_(t("idx_k_norm_b"))
                att.indexer.weights_proj.weight.copy_(t("idx_weights_proj"))
            hs = torch.from_numpy(np.stack([synth.hidden_state(H, ATT_SEED * 100 + layer, p) for p in range(S)]))
            x = norm(hs.reshape(1, S, H))
            cos, sin = rot(x, pos)
            o, _, topk = att(x, (cos, sin), None, None, pos, prev_topk_indices=prev)
        if layer == 0:
            prev = topk
            keep = np.zeros((S, S), bool)  # keep[q, k]: key k (causal, k <= q) selected for query q
            for q in range(S):
                for k in topk[0, q].numpy():
                    if 0 <= k <= q:
                        keep[q, k] = True
            out["keep"] = keep
        out[f"attn_out{layer}"] = o[0].numpy()
    mw = synthdata.as_f32(synthdata.dense_mlp(H, a["dense_inter"], ATT_SEED, 0))
    mlp = M.GlmMoeDsaMLP(cfg, intermediate_size=a["dense_inter"]).float().eval()
    pn = M.GlmMoeDsaRMSNorm(H, eps=a["rms_eps"]).float().eval()
    with torch.no_grad():
        mlp.gate_proj.weight.copy_(torch.from_numpy(mw["gate"]))
        mlp.up_proj.weight.copy_(torch.from_numpy(mw["up"]))
        mlp.down_proj.weight.copy_(torch.from_numpy(mw["down"]))
        pn.weight.copy_(torch.from_numpy(mw["post_ln"]))
        hs = torch.from_numpy(np.stack([synth.hidden_state(H, ATT_SEED * 100 + 9, p) for p in range(4)]))
        out["mlp_out"] = mlp(pn(hs)).numpy()
    out["config"] = np.array(json.dumps(ATT))
    out["seq"] = np.array(ATT_SEQ)
    out["seed"] = np.array(ATT_SEED)
    return out


def main():
    with open(os.path.join(HERE, "mxfp4_hand_fixture.json"), "w") as f:
        json.dump(hand_fixture(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "dequant_tf.npz"), **dequant_fixture())
    arrs = {}
    for seed in SMALL_SEEDS:
        for k, v in moe_small(seed).items():
            arrs[f"s{seed}_{k}"] = v
    arrs["config"] = np.array(json.dumps(SMALL))
    arrs["seeds"] = np.array(SMALL_SEEDS)
    np.savez_compressed(os.path.join(HERE, "moe_tf_small.npz"), **arrs)
    np.savez_compressed(os.path.join(HERE, "attn_tf_small.npz"), **attn_small())
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
