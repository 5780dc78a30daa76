"""Synthetic dense inputs of the benchmark configs (host side, numpy).

The routed MXFP4 experts are generated on the device (wl_synth_expert). The
small dense tensors are drawn here with numpy's default_rng seeded by
(seed, layer, tag) and rounded to bf16 (round-to-nearest-even) where the
config says bf16:

  router weight [E,H] bf16 ~ N(0, 0.02)      tag 1
  e_score_correction_bias [E] f32 ~ N(0, 0.01) tag 2
  shared gate [SI,H], up [SI,H], down [H,SI] bf16 ~ N(0, 0.02)   tags 3, 4, 5
  hidden state [H] bf16 ~ N(0, 1), widened to f32   tag 6 (layer slot = step)
  post-attention norm weight [H] bf16            tag 7

Attention and dense-MLP weights of a decoder layer (attention_layer,
dense_mlp): bf16 (the indexer's weights_proj f32) ~ N(0, 1/fan_in) so that
projections keep unit scale, norm weights 1 + N(0, 0.1), tags 20-34.

The oracle restates the same recipe independently (oracle/synth.py);
tests/test_oracle.py checks that both give identical arrays.
"""
import numpy as np

TAG_ROUTER, TAG_BIAS, TAG_SH_GATE, TAG_SH_UP, TAG_SH_DOWN, TAG_HIDDEN, TAG_LN = 1, 2, 3, 4, 5, 6, 7


def f32_to_bf16(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def _rng(seed, layer, tag):
    return np.random.default_rng(np.random.SeedSequence([seed, layer, tag]))


def normal_bf16(seed, layer, tag, shape, std):
    x = _rng(seed, layer, tag).standard_normal(size=shape, dtype=np.float32) * np.float32(std)
    return f32_to_bf16(x).reshape(shape)


def router_only(H, E, seed, layer):
    """The router weight and bias of dense_layer (same draws)."""
    router_w = normal_bf16(seed, layer, TAG_ROUTER, (E, H), 0.02)
    bias = (_rng(seed, layer, TAG_BIAS).standard_normal(size=E, dtype=np.float32)
            * np.float32(0.01)).astype(np.float32)
    return {"router_w": router_w, "bias": bias}


def dense_layer(H, E, SI, seed, layer):
    r = router_only(H, E, seed, layer)
    router_w, bias = r["router_w"], r["bias"]
    sg = normal_bf16(seed, layer, TAG_SH_GATE, (SI, H), 0.02)
    su = normal_bf16(seed, layer, TAG_SH_UP, (SI, H), 0.02)
    sd = normal_bf16(seed, layer, TAG_SH_DOWN, (H, SI), 0.02)
    return {"router_w": router_w, "bias": bias, "sh_gate": sg, "sh_up": su, "sh_down": sd,
            "shared_block": np.concatenate([sg.reshape(-1), su.reshape(-1), sd.reshape(-1)])}


def hidden_state(H, seed, step=0):
    return bf16_to_f32(normal_bf16(seed, step, TAG_HIDDEN, (H,), 1.0))


def zipf_bias_offset(E, seed, s=1.1, amplitude=0.05):
    """Zipf(s)-shaped popularity offset for the router bias (configs 3 and 4):
    the expert of popularity rank r (a seeded permutation) gets amplitude*r^-s."""
    perm = np.random.default_rng(np.random.SeedSequence([seed, 0xF00D])).permutation(E)
    off = np.empty(E, dtype=np.float32)
    off[perm] = (np.float32(amplitude) * (np.arange(1, E + 1, dtype=np.float64) ** -s)).astype(np.float32)
    return off


def _w_bf16(seed, layer, tag, shape, fan_in, scale=1.0):
    return normal_bf16(seed, layer, tag, shape, scale / np.sqrt(fan_in))


def _norm_w(seed, layer, tag, n):
    x = np.float32(1.0) + _rng(seed, layer, tag).standard_normal(size=n, dtype=np.float32) * np.float32(0.1)
    return f32_to_bf16(x)


def attention_layer(a, seed, layer, owner=True):
    """Synthetic weights of one MLA attention block with the DSA indexer
    (owner: the layer has its own indexer). `a` holds hidden, n_heads,
    q_lora_rank, kv_lora_rank, qk_nope, qk_rope, v_head, index_n_heads,
    index_head_dim. bf16 arrays are uint16 bits in the checkpoint's
    [out, in] row-major layout."""
    H, HN, Q, L = a["hidden"], a["n_heads"], a["q_lora_rank"], a["kv_lora_rank"]
    NP, RP, VD = a["qk_nope"], a["qk_rope"], a["v_head"]
    IH, ID = a["index_n_heads"], a["index_head_dim"]
    w = {"input_ln": _norm_w(seed, layer, 20, H),
         "q_a_proj": _w_bf16(seed, layer, 21, (Q, H), H),
         "q_a_ln": _norm_w(seed, layer, 22, Q),
         "q_b_proj": _w_bf16(seed, layer, 23, (HN * (NP + RP), Q), Q),
         "kv_a_proj": _w_bf16(seed, layer, 24, (L + RP, H), H),
         "kv_a_ln": _norm_w(seed, layer, 25, L),
         "kv_b_proj": _w_bf16(seed, layer, 26, (HN * (NP + VD), L), L),
         "o_proj": _w_bf16(seed, layer, 27, (H, HN * VD), HN * VD, 0.5)}
    if owner:
        w.update({"idx_wq_b": _w_bf16(seed, layer, 28, (IH * ID, Q), Q),
                  "idx_wk": _w_bf16(seed, layer, 29, (ID, H), H),
                  "idx_k_norm_w": _norm_w(seed, layer, 30, ID),
                  "idx_k_norm_b": normal_bf16(seed, layer, 31, (ID,), 0.1),
                  "idx_weights_proj": (_rng(seed, layer, 32).standard_normal(size=(IH, H), dtype=np.float32)
                                       * np.float32(1.0 / np.sqrt(H))).astype(np.float32)})
    return w


def dense_mlp(H, DI, seed, layer):
    """Synthetic weights of a dense SwiGLU MLP layer: post_ln [H], gate / up
    [DI, H], down [H, DI] (bf16 bits)."""
    return {"post_ln": _norm_w(seed, layer, 33, H),
            "gate": _w_bf16(seed, layer, 34, (DI, H), H),
            "up": _w_bf16(seed, layer, 35, (DI, H), H),
            "down": _w_bf16(seed, layer, 36, (H, DI), DI)}


def as_f32(w):
    """The same weights widened to f32 (bf16 bits -> values), for the oracle."""
    return {k: (bf16_to_f32(v) if v.dtype == np.uint16 else v) for k, v in w.items()}
