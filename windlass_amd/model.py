"""Synthetic MoE models built through the C ABI, used by the benchmark and the
GPU tests.

DeviceModel: every routed expert of every layer resident in one context-owned
HBM slot pool (written on the device in the native layout by
wl_synth_expert_native).

CachedModel: the same layers with their experts behind the HBM expert cache:
a pinned host pool of `n_host` native blocks is the backing store, and
(layer, expert) reads host block (layer * E + expert) mod n_host, whose bytes
are the synthetic expert (hb // E, hb % E) — so `expert_source_key` maps every
(layer, expert) to the synthetic key the oracle regenerates.

Dense tensors come from windlass_amd.synthdata and are uploaded once. With
shared_alias, every layer uses layer 0's shared expert (it is not behind the
cache, so aliasing it changes nothing the cache does and saves generating one
75 MB expert per layer)."""
import ctypes

import numpy as np

from . import hip, moe, synthdata


# Synthetic MXFP4 shared experts use the routed generator under this expert
# index (no routed expert has it).
SHARED_KEY = 0xFFFF


class _Layers:
    def __init__(self, cfg, seed, n_layers, ln_weights=None, bias_offset=None, shared_alias=False,
                 shared_mxfp4=False):
        self.c = dict(cfg)
        self.seed = seed
        self.L = n_layers
        H, I, E = cfg["hidden"], cfg["moe_inter"], cfg["n_routed_experts"]
        self.E = E
        self.SI = I * cfg.get("n_shared", 1)
        self.cfg = moe.make_config(hidden=H, moe_inter=I, n_routed_experts=E,
                                   n_experts_per_tok=cfg["n_experts_per_tok"],
                                   n_shared=cfg.get("n_shared", 1), n_layers=n_layers,
                                   routed_scaling=cfg.get("routed_scaling", 2.5),
                                   norm_topk_prob=cfg.get("norm_topk_prob", True),
                                   rms_eps=cfg.get("rms_eps", 1e-5))
        self.ctx = moe.Context(self.cfg)
        self._ln_weights = ln_weights
        self._bias_offset = bias_offset
        self._shared_alias = shared_alias
        self.shared_mxfp4 = shared_mxfp4
        self.dense, self.bufs = [], []

    def _bind_dense(self):
        H, E = self.c["hidden"], self.E
        shared0 = None
        for l in range(self.L):
            if self._shared_alias and l > 0:
                d = dict(synthdata.router_only(H, E, self.seed, l))
                d.update({k: self.dense[0][k] for k in ("sh_gate", "sh_up", "sh_down", "shared_block")})
            else:
                d = synthdata.dense_layer(H, E, self.SI, self.seed, l)
            if self._bias_offset is not None:
                d["bias"] = (d["bias"] + self._bias_offset).astype(np.float32)
            self.dense.append(d)
            rw = hip.DeviceBuffer.from_array(d["router_w"])
            bb = hip.DeviceBuffer.from_array(d["bias"])
            if shared0 is None or not self._shared_alias:
                if self.shared_mxfp4:  # a reference-layout MXFP4 block, inter = SI
                    shared0 = hip.DeviceBuffer(moe.expert_layout(self.cfg, self.SI).total)
                    moe.synth_expert(self.cfg, self.seed, self.shared_key(l)[0], SHARED_KEY, shared0.ptr, inter=self.SI)
                    hip.synchronize()
                else:
                    shared0 = hip.DeviceBuffer.from_array(d["shared_block"])
            sb = shared0
            lw = hip.DeviceBuffer.from_array(self._ln_weights[l]) if self._ln_weights is not None else None
            self.bufs.append((rw, bb, sb, lw))
            self.ctx.set_layer(l, rw.ptr, bb.ptr, lw.ptr if lw else None, sb.ptr,
                               moe.SHARED_MXFP4 if self.shared_mxfp4 else moe.SHARED_BF16)

    def expert_source_key(self, layer, expert):
        return layer, expert

    def shared_key(self, layer):
        """(layer, expert) key of layer's synthetic MXFP4 shared expert."""
        return (0 if self._shared_alias else layer), SHARED_KEY

    def close(self):
        self.ctx.close()
        self.bufs = []


class DeviceModel(_Layers):
    """expert_key(layer, expert) -> (layer', expert') chooses which synthetic
    expert fills each slot (default: its own)."""

    def __init__(self, cfg, seed, n_layers=1, ln_weights=None, bias_offset=None, expert_key=None,
                 shared_alias=False, shared_mxfp4=False):
        super().__init__(cfg, seed, n_layers, ln_weights, bias_offset, shared_alias, shared_mxfp4)
        self._key = expert_key or (lambda l, e: (l, e))
        E = self.E
        self.ctx.slot_pool_create(n_layers * E)
        for l in range(n_layers):
            for e in range(E):
                p = self.ctx.slot_pool_ptr(l * E + e)
                kl, ke = self._key(l, e)
                moe.synth_expert_native(self.cfg, seed, kl, ke, p)  # = wl_expert_to_native(synth block)
                self.ctx.slot_bind(l, e, p)
        self._bind_dense()
        hip.synchronize()

    def expert_source_key(self, layer, expert):
        return self._key(layer, expert)


class AliasedModel(_Layers):
    """Every (layer, expert) resident, bound to one of `n_blocks` device blocks:
    (layer, expert) -> block (layer * E + expert) mod n_blocks, which holds the
    synthetic expert (b // E, b % E). This is CachedModel's host mapping, so the
    two compute the same layers: a resident counterpart for cache runs whose
    distinct experts would not fit in HBM (75 GLM layers)."""

    def __init__(self, cfg, seed, n_layers, n_blocks, ln_weights=None, bias_offset=None, shared_alias=False,
                 shared_mxfp4=False):
        super().__init__(cfg, seed, n_layers, ln_weights, bias_offset, shared_alias, shared_mxfp4)
        self.n_blocks = n_blocks
        E = self.E
        self.ctx.slot_pool_create(n_blocks)
        for b in range(n_blocks):
            kl, ke = divmod(b, E)
            moe.synth_expert_native(self.cfg, seed, kl, ke, self.ctx.slot_pool_ptr(b))
        for l in range(n_layers):
            for e in range(E):
                self.ctx.slot_bind(l, e, self.ctx.slot_pool_ptr((l * E + e) % n_blocks))
        self._bind_dense()
        hip.synchronize()

    def expert_source_key(self, layer, expert):
        return divmod((layer * self.E + expert) % self.n_blocks, self.E)


class CachedModel(_Layers):
    def __init__(self, cfg, seed, n_layers, capacity, n_host, ln_weights=None, bias_offset=None,
                 shared_alias=False, shared_mxfp4=False):
        super().__init__(cfg, seed, n_layers, ln_weights, bias_offset, shared_alias, shared_mxfp4)
        self.n_host = n_host
        self.nb = moe.native_block_bytes(self.cfg)
        self.host = hip.HostBuffer(n_host * self.nb)
        tmp = hip.DeviceBuffer(self.nb)
        for hb in range(n_host):
            kl, ke = divmod(hb, self.E)
            moe.synth_expert_native(self.cfg, seed, kl, ke, tmp.ptr)
            hip.copy_d2h_ptr(self.host.ptr + hb * self.nb, tmp.ptr, self.nb)
        tmp.free()
        base, nb, E, nh = self.host.ptr, self.nb, self.E, n_host
        self.ctx.cache_create(capacity, lambda l, e: base + ((l * E + e) % nh) * nb)
        self._bind_dense()
        hip.synchronize()

    def host_block_index(self, layer, expert):
        return (layer * self.E + expert) % self.n_host

    def expert_source_key(self, layer, expert):
        return divmod(self.host_block_index(layer, expert), self.E)

    def close(self):
        super().close()
        self.host.free()


class SourceModel(_Layers):
    """The layers of a DeviceModel `dm` in a second context with no expert
    bound: every expert comes through a wl_expert_source. native=True: the
    source hands out dm's own slot blocks; native=False: reference-layout
    blocks of the same synthetic experts (a pool written by wl_synth_expert),
    which the library converts. with_prefetch / with_async drop the optional
    callbacks when False. `missing` lists (layer, expert) keys the source has
    no block for. Every call is logged in self.calls."""

    def __init__(self, dm, native=True, with_prefetch=True, with_async=True, missing=()):
        super().__init__(dm.c, dm.seed, dm.L, dm._ln_weights, dm._bias_offset, dm._shared_alias, dm.shared_mxfp4)
        E = self.E
        self.calls = []
        self.missing = set(missing)
        if native:
            self.blocks = {(l, e): dm.ctx.slot_pool_ptr(l * E + e) for l in range(dm.L) for e in range(E)}
            self.pool = None
        else:
            lay = moe.expert_layout(self.cfg)
            self.pool = hip.DeviceBuffer(dm.L * E * lay.total)
            self.blocks = {}
            for l in range(dm.L):
                for e in range(E):
                    p = self.pool.ptr + (l * E + e) * lay.total
                    kl, ke = dm.expert_source_key(l, e)
                    moe.synth_expert(self.cfg, dm.seed, kl, ke, p)
                    self.blocks[(l, e)] = p
        self._bind_dense()

        def block(layer, expert):
            return 0 if (layer, expert) in self.missing else self.blocks[(layer, expert)]

        def get(layer, expert):
            self.calls.append(("get", layer, expert))
            return block(layer, expert)

        def prefetch(layer, ids, stream):
            self.calls.append(("prefetch", layer, tuple(ids)))

        def get_async(layer, expert, stream):
            self.calls.append(("get_async", layer, expert))
            return block(layer, expert)

        self.ctx.set_expert_source(get, prefetch if with_prefetch else None, get_async if with_async else None,
                                   native=native)
        hip.synchronize()

    def close(self):
        super().close()
        if self.pool is not None:
            self.pool.free()


class FileModel(_Layers):
    """The layers with their experts behind the HBM cache over packed expert
    files: directory/layer_{first_layer + l}.bin holds E reference-layout
    records, record e being the synthetic expert (l, e) (the caller writes
    the files)."""

    def __init__(self, cfg, seed, n_layers, capacity, directory, first_layer=0, io_threads=4, ln_weights=None,
                 bias_offset=None, shared_alias=False, shared_mxfp4=False, direct=False):
        super().__init__(cfg, seed, n_layers, ln_weights, bias_offset, shared_alias, shared_mxfp4)
        self.ctx.cache_create_files(capacity, directory, first_layer, io_threads, direct=direct)
        self._bind_dense()
        hip.synchronize()


def make_io(H):
    return hip.DeviceBuffer(4 * H), hip.DeviceBuffer(4 * H)


class AttnModel:
    """Decoder-layer attention (and dense MLPs) with synthetic weights
    (synthdata.attention_layer / dense_mlp) uploaded once: `owners[l]` says
    whether layer l has its own indexer; layers in `dense` get a dense MLP."""

    def __init__(self, a, seed, n_layers, owners, dense=(), max_seq=4096):
        self.a = dict(a)
        self.cfg = moe.make_attn_config(hidden=a["hidden"], n_heads=a["n_heads"], q_lora_rank=a["q_lora_rank"],
                                        kv_lora_rank=a["kv_lora_rank"], qk_nope=a["qk_nope"], qk_rope=a["qk_rope"],
                                        v_head=a["v_head"], index_n_heads=a["index_n_heads"],
                                        index_head_dim=a["index_head_dim"], index_topk=a["index_topk"],
                                        dense_inter=a.get("dense_inter", 0), n_layers=n_layers, max_seq=max_seq,
                                        rms_eps=a.get("rms_eps", 1e-5), rope_theta=a.get("rope_theta", 10000.0))
        self.attn = moe.Attention(self.cfg)
        self.weights, self.mlp, self.bufs = [], {}, []
        for l in range(n_layers):
            w = synthdata.attention_layer(a, seed, l, owner=owners[l])
            self.weights.append(w)
            ptrs = {}
            for k, v in w.items():
                b = hip.DeviceBuffer.from_array(v)
                self.bufs.append(b)
                ptrs[k] = b.ptr
            self.attn.set_layer(l, ptrs)
            if l in dense:
                m = synthdata.dense_mlp(a["hidden"], a["dense_inter"], seed, l)
                self.mlp[l] = m
                bs = [hip.DeviceBuffer.from_array(m[k]) for k in ("post_ln", "gate", "up", "down")]
                self.bufs += bs
                self.attn.set_dense_mlp(l, *[b.ptr for b in bs])
        hip.synchronize()

    def close(self):
        self.attn.close()
        self.bufs = []
