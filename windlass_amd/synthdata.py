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
