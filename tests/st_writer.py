"""Safetensors checkpoints for the loader tests, written from the synthetic
generator under the reference's tensor names (src/glm_loader.cuh:597-611;
tools/repack_experts_glm.py:46-53). The file writer is
windlass_amd.checkpoint's, itself checked against the `safetensors` library
in tests/test_loader.py."""
import numpy as np

from oracle import synth
from windlass_amd import synthdata
from windlass_amd.checkpoint import write_checkpoint, write_safetensors  # noqa: F401 (re-exported)
from windlass_amd.model import SHARED_KEY


def ln_weight(H, seed, layer):
    """A post-attention norm weight near 1 (bf16 bits)."""
    x = 1.0 + 0.1 * np.random.default_rng([seed, layer, 7]).standard_normal(H).astype(np.float32)
    return synthdata.f32_to_bf16(x)


def _expert_tensors(P, parts, H, I):
    """The six tensors of one MXFP4 expert (parts in ExpertLayout order)."""
    out = []
    for j, proj in enumerate(["gate_proj", "up_proj", "down_proj"]):
        rows, cols = (I, H) if j < 2 else (H, I)
        w, s = parts[2 * j], parts[2 * j + 1]
        out.append((f"{P}{proj}.weight", "U8", (rows, cols // 2), w.tobytes()))
        out.append((f"{P}{proj}.weight_scale", "U8", (rows, cols // 32), s.tobytes()))
    return out


def moe_layer_tensors(cfg, seed, ckpt_layer, synth_layer, shared_mxfp4=False, experts=None, bias_offset=None):
    """The MoE tensors of checkpoint layer `ckpt_layer`, holding the synthetic
    layer `synth_layer` of `seed`: the same bytes DeviceModel binds for that
    layer (routed experts `experts`, default all; norm weight ln_weight)."""
    H, I, E = cfg["hidden"], cfg["moe_inter"], cfg["n_routed_experts"]
    SI = I * cfg.get("n_shared", 1)
    d = synthdata.dense_layer(H, E, SI, seed, synth_layer)
    bias = d["bias"] if bias_offset is None else (d["bias"] + bias_offset).astype(np.float32)
    P = f"model.layers.{ckpt_layer}."
    ts = [(P + "post_attention_layernorm.weight", "BF16", (H,), ln_weight(H, seed, synth_layer).tobytes()),
          (P + "mlp.gate.weight", "BF16", (E, H), d["router_w"].tobytes()),
          (P + "mlp.gate.e_score_correction_bias", "F32", (E,), bias.tobytes())]
    if shared_mxfp4:
        ts += _expert_tensors(P + "mlp.shared_experts.", synth.expert_block(H, SI, seed, synth_layer, SHARED_KEY), H, SI)
    else:
        ts += [(P + "mlp.shared_experts.gate_proj.weight", "BF16", (SI, H), d["sh_gate"].tobytes()),
               (P + "mlp.shared_experts.up_proj.weight", "BF16", (SI, H), d["sh_up"].tobytes()),
               (P + "mlp.shared_experts.down_proj.weight", "BF16", (H, SI), d["sh_down"].tobytes())]
    for e in (range(E) if experts is None else experts):
        ts += _expert_tensors(f"{P}mlp.experts.{e}.", synth.expert_block(H, I, seed, synth_layer, e), H, I)
    return ts
