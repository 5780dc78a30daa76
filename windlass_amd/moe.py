"""ctypes binding of include/windlass_moe.h.

The MoE path itself is the native library libwindlass_moe.so (gfx950 HIP
kernels behind a C ABI). This module only marshals arguments; it has no compute
of its own and no fallback: if the library is missing, loading fails loudly.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("WINDLASS_MOE_LIB") or os.path.join(HERE, "libwindlass_moe.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "windlass_moe.h")

WL_OK = 0
STATUS = {0: "WL_OK", 1: "WL_ERR_INVALID", 2: "WL_ERR_HIP", 3: "WL_ERR_OOM", 4: "WL_ERR_NOT_RESIDENT",
          5: "WL_ERR_STATE", 6: "WL_ERR_DEVICE", 7: "WL_ERR_IO", 8: "WL_ERR_NOT_FOUND", 9: "WL_ERR_FORMAT"}
SHARED_BF16, SHARED_MXFP4 = 0, 1
SCHED_FUSED, SCHED_PHASED = 0, 1
MAX_TOPK = 32


class NativeLibraryMissing(ImportError):
    pass


class WindlassError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


class MoeConfig(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_uint32), ("moe_inter", ctypes.c_uint32),
                ("n_routed_experts", ctypes.c_uint32), ("n_experts_per_tok", ctypes.c_uint32),
                ("n_shared", ctypes.c_uint32), ("n_layers", ctypes.c_uint32),
                ("routed_scaling", ctypes.c_float), ("norm_topk_prob", ctypes.c_int32),
                ("rms_eps", ctypes.c_float)]


class ExpertLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in
                ["gw_off", "gw_len", "gs_off", "gs_len", "uw_off", "uw_len", "us_off", "us_len",
                 "dw_off", "dw_len", "ds_off", "ds_len", "total"]]


class CacheStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ["hits", "misses", "evictions", "spec_requests", "spec_copies",
                                               "spec_hits", "bytes_h2d"]] + \
               [("used", ctypes.c_uint32), ("capacity", ctypes.c_uint32), ("bypassed", ctypes.c_uint64)]


POLICY = {"lru": 0, "lfu": 1, "slru": 2, "2q": 3, "tinylfu": 4, "belady": 5, "belady_bypass": 6}


class CachePolicy(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("protected_frac", ctypes.c_float), ("ghost", ctypes.c_uint32)]


def make_policy(name="lru", protected_frac=0.5, ghost=0):
    return CachePolicy(POLICY[name], protected_frac, ghost)


# const uint8_t* host_block(void* user, uint32_t layer, uint32_t expert)
HOST_BLOCK_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32)


# wl_expert_source callbacks (the C form of glm::ExpertSource)
SRC_GET_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32)
SRC_PREFETCH_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_int32),
                                   ctypes.c_uint32, ctypes.c_void_p)
SRC_GET_ASYNC_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                    ctypes.c_void_p)


class ExpertSourceC(ctypes.Structure):
    _fields_ = [("user", ctypes.c_void_p), ("get", SRC_GET_FN), ("prefetch", SRC_PREFETCH_FN),
                ("get_async", SRC_GET_ASYNC_FN), ("native", ctypes.c_int32)]


class StTensor(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_char * 16), ("ndim", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 8),
                ("nbytes", ctypes.c_uint64), ("file_offset", ctypes.c_uint64), ("shard", ctypes.c_uint32)]


class AttnConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ["hidden", "n_heads", "q_lora_rank", "kv_lora_rank", "qk_nope", "qk_rope", "v_head", "index_n_heads",
                 "index_head_dim", "index_topk", "dense_inter", "n_layers", "max_seq"]] + \
               [("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


ATTN_WEIGHTS = ["input_ln", "q_a_proj", "q_a_ln", "q_b_proj", "kv_a_proj", "kv_a_ln", "kv_b_proj", "o_proj",
                "idx_wq_b", "idx_wk", "idx_k_norm_w", "idx_k_norm_b", "idx_weights_proj"]


class AttnWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ATTN_WEIGHTS]


class AttnTaps(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ["norm", "q_resid", "attn", "attn_out", "index_score", "keep"]]


class Taps(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ["norm", "logits", "topk_idx", "topk_w", "mid", "shared"]]


_lib = None


def load():
    """Loads libwindlass_moe.so (raises NativeLibraryMissing if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -m windlass_amd.build` (there is no fallback path)")
    lib = ctypes.CDLL(LIB_PATH)
    vp, u32, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int32
    sig = {
        "wl_expert_layout_of": [ctypes.POINTER(MoeConfig), u32, ctypes.POINTER(ExpertLayout)],
        "wl_create": [ctypes.POINTER(MoeConfig), ctypes.POINTER(vp)],
        "wl_set_layer": [vp, u32, vp, vp, vp, vp, i32],
        "wl_set_layer_mxfp4": [vp, u32, vp, vp, vp, vp, vp, vp, vp, vp, vp],
        "wl_set_layer_dense": [vp, u32, vp, vp, vp, vp, u32],
        "wl_make_resident": [vp, u32, vp],
        "wl_slot_bind": [vp, u32, u32, vp],
        "wl_slot_unbind": [vp, u32, u32],
        "wl_slot_pool_create": [vp, u32],
        "wl_slot_pool_ptr": [vp, u32, ctypes.POINTER(vp)],
        "wl_run_moe": [vp, u32, vp, vp, vp],
        "wl_run_moe_residual": [vp, u32, vp, vp, vp, vp],
        "wl_run_chain": [vp, u32, u32, vp, vp, vp],
        "wl_run_moe_batched": [vp, u32, u32, vp, vp, vp, vp],
        "wl_run_moe_batched_noalloc": [vp, u32, u32, vp, vp, vp, vp],
        "wl_batched_counts": [vp, ctypes.POINTER(u32)],
        "wl_batched_routing": [vp, u32, ctypes.POINTER(u32), vp, vp, vp],
        "wl_taps": [vp, ctypes.POINTER(Taps)],
        "wl_check_error": [vp, vp],
        "wl_set_schedule": [vp, i32],
        "wl_set_taps": [vp, i32],
        "wl_synth_expert": [ctypes.POINTER(MoeConfig), u32, u32, u32, u32, vp, vp],
        "wl_synth_expert_native": [ctypes.POINTER(MoeConfig), u32, u32, u32, vp, vp],
        "wl_expert_to_native": [ctypes.POINTER(MoeConfig), vp, vp, vp],
        "wl_dequant_matvec_mxfp4": [vp, vp, vp, vp, u32, u32, vp],
        "wl_expert_ffn": [vp, vp, vp, vp, vp, vp],
        "wl_cache_create": [vp, u32, HOST_BLOCK_FN, vp],
        "wl_cache_create_files": [vp, u32, ctypes.c_char_p, u32, u32],
        "wl_cache_create_files_ex": [vp, u32, ctypes.c_char_p, u32, u32, u32],
        "wl_set_expert_source": [vp, ctypes.POINTER(ExpertSourceC)],
        "wl_cache_set_speculation": [vp, i32],
        "wl_cache_get_stats": [vp, ctypes.POINTER(CacheStats)],
        "wl_cache_reset_stats": [vp],
        "wl_cache_prefetch": [vp, u32, ctypes.POINTER(i32), u32, vp],
        "wl_cache_get": [vp, u32, u32, vp, ctypes.POINTER(vp)],
        "wl_lru_replay": [u32, ctypes.POINTER(u32), u32, u32, ctypes.POINTER(ctypes.c_uint8),
                          ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                          ctypes.POINTER(ctypes.c_uint64)],
        "wl_policy_replay": [ctypes.POINTER(CachePolicy), u32, ctypes.POINTER(u32), u32, u32, ctypes.POINTER(u32), u32,
                             ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_uint64),
                             ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
        "wl_cache_set_policy": [vp, ctypes.POINTER(CachePolicy)],
        "wl_cache_pin": [vp, u32, u32, i32],
        "wl_st_open": [ctypes.c_char_p, i32, ctypes.POINTER(vp)],
        "wl_st_info": [vp, ctypes.c_char_p, ctypes.POINTER(StTensor)],
        "wl_st_read": [vp, ctypes.c_char_p, vp, ctypes.c_size_t],
        "wl_st_pack_layer": [vp, ctypes.POINTER(MoeConfig), u32, ctypes.c_char_p],
        "wl_load_layer": [vp, vp, u32, u32],
        "wl_load_experts": [vp, vp, u32, u32, ctypes.POINTER(u32), u32, u32, vp],
        "wl_attn_create": [ctypes.POINTER(AttnConfig), ctypes.POINTER(vp)],
        "wl_attn_set_layer": [vp, u32, ctypes.POINTER(AttnWeights)],
        "wl_attn_set_dense_mlp": [vp, u32, vp, vp, vp, vp],
        "wl_run_attention": [vp, u32, u32, vp, vp],
        "wl_run_dense_mlp": [vp, u32, vp, vp],
        "wl_run_layer": [vp, vp, u32, u32, u32, vp, vp],
        "wl_attn_taps": [vp, ctypes.POINTER(AttnTaps)],
        "wl_matvec_bf16": [vp, vp, vp, u32, u32, vp],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.wl_native_block_bytes.argtypes = [ctypes.POINTER(MoeConfig)]
    lib.wl_native_block_bytes.restype = ctypes.c_size_t
    lib.wl_destroy.argtypes = [vp]
    lib.wl_destroy.restype = None
    lib.wl_last_error.argtypes = [vp]
    lib.wl_last_error.restype = ctypes.c_char_p
    lib.wl_attn_destroy.argtypes = [vp]
    lib.wl_attn_destroy.restype = None
    lib.wl_attn_last_error.argtypes = [vp]
    lib.wl_attn_last_error.restype = ctypes.c_char_p
    lib.wl_st_close.argtypes = [vp]
    lib.wl_st_close.restype = None
    lib.wl_st_last_error.argtypes = [vp]
    lib.wl_st_last_error.restype = ctypes.c_char_p
    lib.wl_st_count.argtypes = [vp]
    lib.wl_st_count.restype = u32
    lib.wl_st_name.argtypes = [vp, u32]
    lib.wl_st_name.restype = ctypes.c_char_p
    _lib = lib
    return lib


def header_functions(path=HEADER):
    """Names of every function declared in the public header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wl_[a-z0-9_]+)\s*\(", text)))


def make_config(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
                n_layers=1, routed_scaling=2.5, norm_topk_prob=True, rms_eps=1e-5):
    return MoeConfig(hidden, moe_inter, n_routed_experts, n_experts_per_tok, n_shared, n_layers,
                     routed_scaling, 1 if norm_topk_prob else 0, rms_eps)


def expert_layout(cfg, inter=0):
    lay = ExpertLayout()
    rc = load().wl_expert_layout_of(ctypes.byref(cfg), inter, ctypes.byref(lay))
    if rc != WL_OK:
        raise WindlassError(rc, "wl_expert_layout_of")
    return lay


def synth_expert(cfg, seed, layer, expert, d_block, stream=0, inter=0):
    rc = load().wl_synth_expert(ctypes.byref(cfg), inter, seed, layer, expert, d_block, stream)
    if rc != WL_OK:
        raise WindlassError(rc, "wl_synth_expert")


def synth_expert_native(cfg, seed, layer, expert, d_native, stream=0):
    rc = load().wl_synth_expert_native(ctypes.byref(cfg), seed, layer, expert, d_native, stream)
    if rc != WL_OK:
        raise WindlassError(rc, "wl_synth_expert_native")


def expert_to_native(cfg, d_ref, d_native, stream=0):
    rc = load().wl_expert_to_native(ctypes.byref(cfg), d_ref, d_native, stream)
    if rc != WL_OK:
        raise WindlassError(rc, "wl_expert_to_native")


def native_block_bytes(cfg):
    return int(load().wl_native_block_bytes(ctypes.byref(cfg)))


def lru_replay(capacity, keys, batch):
    """The cache's LRU bookkeeping over a key sequence (no device use):
    returns (per-key 1 hit / 0 miss / 2 skipped duplicate, hits, misses, evictions)."""
    import numpy as np
    k = np.ascontiguousarray(keys, dtype=np.uint32)
    out = np.zeros(len(k), dtype=np.uint8)
    h, m, e = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    rc = load().wl_lru_replay(capacity, k.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), len(k), batch,
                              out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), ctypes.byref(h), ctypes.byref(m),
                              ctypes.byref(e))
    if rc != WL_OK:
        raise WindlassError(rc, "wl_lru_replay")
    return out, h.value, m.value, e.value


def policy_replay(policy, capacity, keys, batch, pinned=()):
    """The cache's bookkeeping under `policy` (a CachePolicy or a name) over a
    key sequence (no device use): (per-key 1 hit / 0 retained miss / 3 miss
    not retained / 2 skipped duplicate, hits, misses, evictions)."""
    import numpy as np
    pol = make_policy(policy) if isinstance(policy, str) else policy
    k = np.ascontiguousarray(keys, dtype=np.uint32)
    pn = np.ascontiguousarray(list(pinned), dtype=np.uint32)
    out = np.zeros(len(k), dtype=np.uint8)
    h, m, e = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    P32 = ctypes.POINTER(ctypes.c_uint32)
    rc = load().wl_policy_replay(ctypes.byref(pol), capacity, k.ctypes.data_as(P32), len(k), batch,
                                 pn.ctypes.data_as(P32), len(pn), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                                 ctypes.byref(h), ctypes.byref(m), ctypes.byref(e))
    if rc != WL_OK:
        raise WindlassError(rc, "wl_policy_replay")
    return out, h.value, m.value, e.value


def matvec_bf16(d_W, d_x, d_y, N, K, stream=0):
    rc = load().wl_matvec_bf16(d_W, d_x, d_y, N, K, stream)
    if rc != WL_OK:
        raise WindlassError(rc, "wl_matvec_bf16")


def dequant_matvec_mxfp4(d_W, d_S, d_x, d_y, N, K, stream=0):
    rc = load().wl_dequant_matvec_mxfp4(d_W, d_S, d_x, d_y, N, K, stream)
    if rc != WL_OK:
        raise WindlassError(rc, "wl_dequant_matvec_mxfp4")


class SafeTensors:
    """An open safetensors checkpoint (wl_st_*): a directory with
    model.safetensors.index.json or model.safetensors, or one .safetensors
    file. Host-only."""

    def __init__(self, path, allow_missing_shards=False):
        self.lib = load()
        h = ctypes.c_void_p()
        rc = self.lib.wl_st_open(os.fsencode(path), 1 if allow_missing_shards else 0, ctypes.byref(h))
        if rc != WL_OK:
            raise WindlassError(rc, f"wl_st_open: {self.lib.wl_st_last_error(None).decode()}")
        self.h = h.value

    def _ck(self, rc, what):
        if rc != WL_OK:
            raise WindlassError(rc, f"{what}: {self.lib.wl_st_last_error(self.h).decode()}")

    def names(self):
        return [self.lib.wl_st_name(self.h, i).decode() for i in range(self.lib.wl_st_count(self.h))]

    def info(self, name):
        """dict(dtype, shape, nbytes, file_offset, shard), or None if absent."""
        t = StTensor()
        rc = self.lib.wl_st_info(self.h, name.encode(), ctypes.byref(t))
        if rc == 8:  # WL_ERR_NOT_FOUND
            return None
        self._ck(rc, "wl_st_info")
        return {"dtype": t.dtype.decode(), "shape": tuple(t.shape[i] for i in range(t.ndim)), "nbytes": t.nbytes,
                "file_offset": t.file_offset, "shard": t.shard}

    def read(self, name, capacity=None):
        """The tensor's raw bytes (numpy uint8)."""
        import numpy as np
        t = self.info(name)
        n = t["nbytes"] if t else 0
        buf = np.empty(max(n, 1) if capacity is None else capacity, np.uint8)
        self._ck(self.lib.wl_st_read(self.h, name.encode(), buf.ctypes.data, buf.nbytes), f"wl_st_read({name})")
        return buf[:n]

    def pack_layer(self, cfg, ckpt_layer, path):
        self._ck(self.lib.wl_st_pack_layer(self.h, ctypes.byref(cfg), ckpt_layer, os.fsencode(path)),
                 "wl_st_pack_layer")

    def close(self):
        if self.h:
            self.lib.wl_st_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def make_attn_config(hidden=6144, n_heads=64, q_lora_rank=2048, kv_lora_rank=512, qk_nope=192, qk_rope=64,
                     v_head=256, index_n_heads=32, index_head_dim=128, index_topk=2048, dense_inter=12288,
                     n_layers=1, max_seq=4096, rms_eps=1e-5, rope_theta=1e6):
    return AttnConfig(hidden, n_heads, q_lora_rank, kv_lora_rank, qk_nope, qk_rope, v_head, index_n_heads,
                      index_head_dim, index_topk, dense_inter, n_layers, max_seq, rms_eps, rope_theta)


class Attention:
    """One wl_attn: the attention (and dense MLP) side of decoder layers."""

    def __init__(self, cfg):
        self.lib = load()
        self.cfg = cfg
        h = ctypes.c_void_p()
        rc = self.lib.wl_attn_create(ctypes.byref(cfg), ctypes.byref(h))
        if rc != WL_OK:
            raise WindlassError(rc, f"wl_attn_create: {self.lib.wl_attn_last_error(None).decode()}")
        self.h = h.value

    def _ck(self, rc, what):
        if rc != WL_OK:
            raise WindlassError(rc, f"{what}: {self.lib.wl_attn_last_error(self.h).decode()}")

    def set_layer(self, layer, ptrs):
        """ptrs: dict of ATTN_WEIGHTS names -> device pointers (idx_* absent on a shared layer)."""
        w = AttnWeights(*[ptrs.get(n) for n in ATTN_WEIGHTS])
        self._ck(self.lib.wl_attn_set_layer(self.h, layer, ctypes.byref(w)), "wl_attn_set_layer")

    def set_dense_mlp(self, layer, post_ln, gate, up, down):
        self._ck(self.lib.wl_attn_set_dense_mlp(self.h, layer, post_ln, gate, up, down), "wl_attn_set_dense_mlp")

    def run_attention(self, layer, pos, d_hidden, stream=0):
        self._ck(self.lib.wl_run_attention(self.h, layer, pos, d_hidden, stream), "wl_run_attention")

    def run_dense_mlp(self, layer, d_hidden, stream=0):
        self._ck(self.lib.wl_run_dense_mlp(self.h, layer, d_hidden, stream), "wl_run_dense_mlp")

    def run_layer(self, moe_ctx, layer, moe_layer, pos, d_hidden, stream=0):
        self._ck(self.lib.wl_run_layer(self.h, moe_ctx.h if moe_ctx else None, layer, moe_layer, pos, d_hidden,
                                       stream), "wl_run_layer")

    def taps(self):
        t = AttnTaps()
        self._ck(self.lib.wl_attn_taps(self.h, ctypes.byref(t)), "wl_attn_taps")
        return {n: getattr(t, n) for n, _ in AttnTaps._fields_}

    def close(self):
        if self.h:
            self.lib.wl_attn_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    """One wl_ctx: the MoE layers of a model on the current device."""

    def __init__(self, cfg):
        self.lib = load()
        self.cfg = cfg
        h = ctypes.c_void_p()
        rc = self.lib.wl_create(ctypes.byref(cfg), ctypes.byref(h))
        if rc != WL_OK:
            raise WindlassError(rc, "wl_create")
        self.h = h.value

    def _ck(self, rc, what):
        if rc != WL_OK:
            raise WindlassError(rc, f"{what}: {self.lib.wl_last_error(self.h).decode()}")

    def close(self):
        if self.h:
            self.lib.wl_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_layer(self, layer, router_w, bias, ln_w, shared, shared_dtype=SHARED_BF16):
        self._ck(self.lib.wl_set_layer(self.h, layer, router_w, bias, ln_w, shared, shared_dtype),
                 "wl_set_layer")

    def set_layer_mxfp4(self, layer, router_w, bias, ln_w, gw, gs, uw, us, dw, ds):
        self._ck(self.lib.wl_set_layer_mxfp4(self.h, layer, router_w, bias, ln_w, gw, gs, uw, us, dw, ds),
                 "wl_set_layer_mxfp4")

    def set_layer_dense(self, layer, post_ln, gate, up, down, dense_inter):
        self._ck(self.lib.wl_set_layer_dense(self.h, layer, post_ln, gate, up, down, dense_inter),
                 "wl_set_layer_dense")

    def make_resident(self, layer, stream=0):
        self._ck(self.lib.wl_make_resident(self.h, layer, stream), "wl_make_resident")

    def load_layer(self, st, ckpt_layer, layer):
        self._ck(self.lib.wl_load_layer(self.h, st.h, ckpt_layer, layer), "wl_load_layer")

    def load_experts(self, st, ckpt_layer, layer, experts=None, n=None, first_slot=0, stream=0):
        if experts is None:
            arr, cnt = None, n
        else:
            arr = (ctypes.c_uint32 * len(experts))(*[int(e) for e in experts])
            cnt = len(experts)
        self._ck(self.lib.wl_load_experts(self.h, st.h, ckpt_layer, layer, arr, cnt, first_slot, stream),
                 "wl_load_experts")

    def slot_bind(self, layer, expert, d_block):
        self._ck(self.lib.wl_slot_bind(self.h, layer, expert, d_block), "wl_slot_bind")

    def slot_unbind(self, layer, expert):
        self._ck(self.lib.wl_slot_unbind(self.h, layer, expert), "wl_slot_unbind")

    def slot_pool_create(self, n_slots):
        self._ck(self.lib.wl_slot_pool_create(self.h, n_slots), "wl_slot_pool_create")

    def slot_pool_ptr(self, slot):
        p = ctypes.c_void_p()
        self._ck(self.lib.wl_slot_pool_ptr(self.h, slot, ctypes.byref(p)), "wl_slot_pool_ptr")
        return p.value

    def run_moe(self, layer, d_hidden, d_out, stream=0):
        self._ck(self.lib.wl_run_moe(self.h, layer, d_hidden, d_out, stream), "wl_run_moe")

    def run_moe_residual(self, layer, d_hidden, d_resid, d_out, stream=0):
        self._ck(self.lib.wl_run_moe_residual(self.h, layer, d_hidden, d_resid, d_out, stream),
                 "wl_run_moe_residual")

    def run_moe_batched(self, layer, n_tokens, d_hidden, d_resid, d_out, stream=0):
        self._ck(self.lib.wl_run_moe_batched(self.h, layer, n_tokens, d_hidden, d_resid, d_out, stream),
                 "wl_run_moe_batched")

    def run_moe_batched_noalloc(self, layer, n_tokens, d_hidden, d_resid, d_out, stream=0):
        self._ck(self.lib.wl_run_moe_batched_noalloc(self.h, layer, n_tokens, d_hidden, d_resid, d_out, stream),
                 "wl_run_moe_batched_noalloc")

    def batched_counts(self):
        import numpy as np
        out = np.zeros(self.cfg.n_routed_experts, dtype=np.uint32)
        self._ck(self.lib.wl_batched_counts(self.h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))),
                 "wl_batched_counts")
        return out

    def batched_routing(self, max_tokens):
        """(logits [T, E], ids [T, K], weights [T, K]) of the last batched chunk."""
        import numpy as np
        E, K = self.cfg.n_routed_experts, self.cfg.n_experts_per_tok
        n = ctypes.c_uint32(0)
        lg = np.zeros((max_tokens, E), np.float32)
        ids = np.zeros((max_tokens, K), np.int32)
        w = np.zeros((max_tokens, K), np.float32)
        self._ck(self.lib.wl_batched_routing(self.h, max_tokens, ctypes.byref(n), lg.ctypes.data,
                                             ids.ctypes.data, w.ctypes.data), "wl_batched_routing")
        T = n.value
        return lg[:T], ids[:T], w[:T]

    def run_chain(self, first_layer, n_layers, d_h, d_tmp, stream=0):
        self._ck(self.lib.wl_run_chain(self.h, first_layer, n_layers, d_h, d_tmp, stream), "wl_run_chain")

    def taps(self):
        t = Taps()
        self._ck(self.lib.wl_taps(self.h, ctypes.byref(t)), "wl_taps")
        return {n: getattr(t, n) for n, _ in Taps._fields_}

    def check_error(self, stream=0):
        self._ck(self.lib.wl_check_error(self.h, stream), "wl_check_error")

    def expert_ffn(self, d_block, d_x, d_y, d_y_bf16=None, stream=0):
        self._ck(self.lib.wl_expert_ffn(self.h, d_block, d_x, d_y, d_y_bf16, stream), "wl_expert_ffn")

    def set_schedule(self, sched):
        self._ck(self.lib.wl_set_schedule(self.h, sched), "wl_set_schedule")

    def set_taps(self, enable):
        self._ck(self.lib.wl_set_taps(self.h, 1 if enable else 0), "wl_set_taps")

    # ---- expert source ----------------------------------------------------
    def set_expert_source(self, get, prefetch=None, get_async=None, native=True):
        """get(layer, expert) -> device address (int, 0 = none); prefetch(layer,
        ids, stream); get_async(layer, expert, stream) -> device address.
        None detaches the source when get is None."""
        if get is None:
            self._src = None
            self._ck(self.lib.wl_set_expert_source(self.h, None), "wl_set_expert_source")
            return
        g = SRC_GET_FN(lambda user, layer, expert: get(layer, expert) or None)
        p = SRC_PREFETCH_FN(lambda user, layer, ids, n, stream: prefetch(layer, [ids[i] for i in range(n)], stream)) \
            if prefetch else ctypes.cast(None, SRC_PREFETCH_FN)
        a = SRC_GET_ASYNC_FN(lambda user, layer, expert, stream: get_async(layer, expert, stream) or None) \
            if get_async else ctypes.cast(None, SRC_GET_ASYNC_FN)
        self._src = ExpertSourceC(None, g, p, a, 1 if native else 0)
        self._ck(self.lib.wl_set_expert_source(self.h, ctypes.byref(self._src)), "wl_set_expert_source")

    # ---- HBM expert cache -------------------------------------------------
    def cache_create(self, capacity, host_block):
        """host_block(layer, expert) -> address of a pinned native block (int)."""
        self._host_block_cb = HOST_BLOCK_FN(lambda user, layer, expert: host_block(layer, expert))
        self._ck(self.lib.wl_cache_create(self.h, capacity, self._host_block_cb, None), "wl_cache_create")

    def cache_create_files(self, capacity, directory, first_layer=0, io_threads=4, direct=False):
        self._ck(self.lib.wl_cache_create_files_ex(self.h, capacity, os.fsencode(directory), first_layer, io_threads,
                                                   1 if direct else 0), "wl_cache_create_files")

    def cache_set_speculation(self, enable):
        self._ck(self.lib.wl_cache_set_speculation(self.h, 1 if enable else 0), "wl_cache_set_speculation")

    def cache_stats(self):
        st = CacheStats()
        self._ck(self.lib.wl_cache_get_stats(self.h, ctypes.byref(st)), "wl_cache_get_stats")
        return {n: getattr(st, n) for n, _ in CacheStats._fields_}

    def cache_set_policy(self, name="lru", protected_frac=0.5, ghost=0):
        pol = make_policy(name, protected_frac, ghost)
        self._ck(self.lib.wl_cache_set_policy(self.h, ctypes.byref(pol)), "wl_cache_set_policy")

    def cache_pin(self, layer, expert, pinned=True):
        self._ck(self.lib.wl_cache_pin(self.h, layer, expert, 1 if pinned else 0), "wl_cache_pin")

    def cache_reset_stats(self):
        self._ck(self.lib.wl_cache_reset_stats(self.h), "wl_cache_reset_stats")

    def cache_prefetch(self, layer, experts, stream=0):
        arr = (ctypes.c_int32 * len(experts))(*[int(e) for e in experts])
        self._ck(self.lib.wl_cache_prefetch(self.h, layer, arr, len(experts), stream), "wl_cache_prefetch")

    def cache_get(self, layer, expert, stream=0):
        p = ctypes.c_void_p()
        self._ck(self.lib.wl_cache_get(self.h, layer, expert, stream, ctypes.byref(p)), "wl_cache_get")
        return p.value
