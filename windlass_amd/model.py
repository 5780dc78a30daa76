"""A resident synthetic MoE model built through the C ABI: every routed
expert of every layer in one context-owned HBM slot pool (written on the device
in the native layout by wl_synth_expert_native), dense tensors from
windlass_amd.synthdata uploaded once.
Used by the benchmark and the GPU tests."""
import numpy as np

from . import hip, moe, synthdata


class DeviceModel:
    def __init__(self, cfg, seed, n_layers=1, ln_weights=None, bias_offset=None):
        self.c = dict(cfg)
        self.seed = seed
        self.L = n_layers
        H, I, E = cfg["hidden"], cfg["moe_inter"], cfg["n_routed_experts"]
        self.SI = I * cfg.get("n_shared", 1)
        self.cfg = moe.make_config(hidden=H, moe_inter=I, n_routed_experts=E,
                                   n_experts_per_tok=cfg["n_experts_per_tok"],
                                   n_shared=cfg.get("n_shared", 1), n_layers=n_layers,
                                   routed_scaling=cfg.get("routed_scaling", 2.5),
                                   norm_topk_prob=cfg.get("norm_topk_prob", True),
                                   rms_eps=cfg.get("rms_eps", 1e-5))
        self.ctx = moe.Context(self.cfg)
        self.ctx.slot_pool_create(n_layers * E)
        self.dense, self.bufs = [], []
        for l in range(n_layers):
            for e in range(E):
                p = self.ctx.slot_pool_ptr(l * E + e)
                moe.synth_expert_native(self.cfg, seed, l, e, p)  # = wl_expert_to_native(synth block)
                self.ctx.slot_bind(l, e, p)
            d = synthdata.dense_layer(H, E, self.SI, seed, l)
            if bias_offset is not None:
                d["bias"] = (d["bias"] + bias_offset).astype(np.float32)
            self.dense.append(d)
            rw = hip.DeviceBuffer.from_array(d["router_w"])
            bb = hip.DeviceBuffer.from_array(d["bias"])
            sb = hip.DeviceBuffer.from_array(d["shared_block"])
            lw = hip.DeviceBuffer.from_array(ln_weights[l]) if ln_weights is not None else None
            self.bufs.append((rw, bb, sb, lw))
            self.ctx.set_layer(l, rw.ptr, bb.ptr, lw.ptr if lw else None, sb.ptr)
        hip.synchronize()

    def close(self):
        self.ctx.close()
        self.bufs = []


def make_io(H):
    return hip.DeviceBuffer(4 * H), hip.DeviceBuffer(4 * H)
