"""CPU restatement (numpy, fp32) of windlass's MoE layer — the parity oracle.

TEST INFRASTRUCTURE ONLY. Imported by tests/, by bench.py's cpu_baseline leg
and by __graft_entry__.smoke(), as the checker; the product path (the HIP
library) never imports or calls it.

Each function cites the reference line it restates. The reference's numpy
files are not imported: this is a fresh restatement pinned by (a) the
reference's hand fixture (tools/glm_mxfp4_numpy.py:44-52), (b) transformers'
independent MXFP4 dequant and GLM router (tests/golden/make_golden.py), (c) an
fp64 brute force in oracle/moe_oracle.c, and (d) closed-form checks in
tests/test_oracle.py.
"""
import numpy as np

from . import synth

# E2M1 code -> value; index = 4-bit code, sign in bit 3
# (tools/glm_mxfp4_numpy.py:14-15; src/glm_kernels.cuh:48-51).
E2M1 = np.array([0., .5, 1., 1.5, 2., 3., 4., 6., -0., -.5, -1., -1.5, -2., -3., -4., -6.],
                dtype=np.float32)


def dequant(w, s):
    """MXFP4 [N, K/2] packed nibbles (low nibble = even column) with [N, K/32]
    E8M0 scales -> fp32 [N, K] (tools/glm_mxfp4_numpy.py:17-26).

    The scale is 2^(s-127) computed exactly with ldexp. The reference writes
    np.exp2(float32(s) - 127), which equals ldexp everywhere except s = 254,
    where numpy's float32 exp2 is 1 ulp high (checked in tests/test_oracle.py);
    the reference's CUDA kernel (exp2f) and transformers (ldexp) are exact
    there, so the oracle follows them. s = 255 (E8M0 NaN) yields NaN, as the
    reference kernel does (src/glm_kernels.cuh:53-61)."""
    assert w.dtype == np.uint8 and s.dtype == np.uint8
    n, half = w.shape
    k = half * 2
    assert s.shape == (n, k // 32)
    out = np.empty((n, k), dtype=np.float32)
    out[:, 0::2] = E2M1[w & 0xF]
    out[:, 1::2] = E2M1[w >> 4]
    sc = np.ldexp(np.float32(1.0), s.astype(np.int32) - 127).astype(np.float32)
    sc[s == 255] = np.nan
    with np.errstate(over="ignore", invalid="ignore"):
        out *= np.repeat(sc, 32, axis=1)
    return out


def rms_norm(x, w, eps):
    """w * (x * (1/sqrt(mean(x^2) + eps))) in fp32 (tools/ref_glm_chain.py:63-80)."""
    x = x.astype(np.float32)
    w = np.ones_like(x) if w is None else w.astype(np.float32)
    return w * (x * (np.float32(1.0) / np.sqrt((x * x).mean(-1, keepdims=True) + np.float32(eps))))


def silu(x):
    """x / (1 + exp(-x)) (tools/ref_glm_chain.py:123-124). exp(-x) overflows
    to inf for x < -88, which gives the correct limit -0."""
    with np.errstate(over="ignore"):
        return x / (np.float32(1.0) + np.exp(-x))


def route(x_norm, gate_w, bias, top_k, routed_scaling, norm_topk_prob):
    """GlmMoeDsaTopkRouter at n_group == topk_group == 1 (tools/ref_glm_chain.py:
    127-149): fp32 logits, sigmoid, choice = score + bias (f32), top-k of choice,
    weight = unbiased score, / (sum + 1e-20), x routed_scaling.

    The reference takes np.argpartition, whose order is unspecified; this
    restatement returns the slots in descending biased score with ties to the
    lowest index, the order of the reference's device kernel
    (src/glm_layer_runner.cuh:318-330). Only the SET and the id-aligned weights
    carry meaning.
    """
    assert bias.dtype == np.float32
    logits = x_norm.astype(np.float32) @ gate_w.astype(np.float32).T
    scores = np.float32(1.0) / (np.float32(1.0) + np.exp(-logits))
    choice = scores + bias.astype(np.float32)
    order = np.lexsort((np.arange(choice.shape[-1]), -choice))
    idx = order[:top_k]
    w = scores[idx].copy()
    if norm_topk_prob:
        w /= (w.sum() + np.float32(1e-20))
    w *= np.float32(routed_scaling)
    return logits, idx.astype(np.int32), w.astype(np.float32), choice


def expert_slot(xn, G, U, D):
    """One routed expert on one position, without the routing weight
    (tools/ref_glm_chain.py:679-685)."""
    g = xn @ G.T
    u = xn @ U.T
    return (silu(g) * u) @ D.T


def swiglu_mid(xn, G, U):
    return silu(xn @ G.T) * (xn @ U.T)


def moe_finish(wt, slot_outs, shared):
    """y = 0; y += w_k e_k (slot order); y = y + shared (tools/ref_glm_chain.py:
    688-711, MoE branch, without the residual)."""
    y = np.zeros(shared.shape[0], np.float32)
    for a, so in zip(wt, slot_outs):
        y += a * so
    return y + shared


class ExpertSource:
    """Dequantised experts of the synthetic model, rebuilt on demand from the
    counter-based generator (the oracle's counterpart of read_expert +
    dequant_expert, tools/ref_glm_chain.py:419-434,667-676)."""

    def __init__(self, H, I, seed, cache=64):
        self.H, self.I, self.seed = H, I, seed
        self._cache = {}
        self._order = []
        self._cap = cache

    def get(self, layer, expert):
        key = (layer, expert)
        if key not in self._cache:
            gw, gs, uw, us, dw, ds = synth.expert_block(self.H, self.I, self.seed, layer, expert)
            self._cache[key] = (dequant(gw, gs), dequant(uw, us), dequant(dw, ds))
            self._order.append(key)
            if len(self._order) > self._cap:
                self._cache.pop(self._order.pop(0))
        return self._cache[key]


def shared_matrices(dense, H, SI):
    """The bf16 shared expert widened to fp32 (dequant_or_raw on a tensor with
    no _scale, tools/ref_glm_chain.py:234-238)."""
    return (synth.bf16_to_f32(dense["sh_gate"]).reshape(SI, H),
            synth.bf16_to_f32(dense["sh_up"]).reshape(SI, H),
            synth.bf16_to_f32(dense["sh_down"]).reshape(H, SI))


def moe_layer(h, dense, experts, layer, cfg, ln_w=None, shared_f32=None):
    """One MoE layer at one position: moe_prepare + expert_slot + moe_finish
    (tools/ref_glm_chain.py:646-711), returning every substep the reference's
    SubstepHook exposes (src/test_glm_chain.cu:434-441). `out` excludes the
    residual, like run_moe's d_out."""
    H, E, K = cfg["hidden"], cfg["n_routed_experts"], cfg["n_experts_per_tok"]
    SI = cfg["moe_inter"] * cfg.get("n_shared", 1)
    xn = rms_norm(h, ln_w, cfg.get("rms_eps", 1e-5))
    router_w = synth.bf16_to_f32(dense["router_w"]).reshape(E, H)
    logits, idx, wt, choice = route(xn, router_w, dense["bias"], K, cfg.get("routed_scaling", 2.5),
                                    cfg.get("norm_topk_prob", True))
    mids, slot_outs = [], []
    for e in idx:
        G, U, D = experts.get(layer, int(e))
        mid = swiglu_mid(xn, G, U)
        mids.append(mid)
        slot_outs.append(mid @ D.T)
    if shared_f32 is None:
        shared_f32 = shared_matrices(dense, H, SI)
    SG, SU, SD = shared_f32
    shared = (silu(xn @ SG.T) * (xn @ SU.T)) @ SD.T
    out = moe_finish(wt, slot_outs, shared)
    return {"norm": xn, "logits": logits, "choice": choice, "topk_idx": idx, "topk_w": wt,
            "mid": np.stack(mids), "slot_outs": np.stack(slot_outs), "shared": shared, "out": out}


def topk_margin(choice, k):
    """Gap between the k-th and (k+1)-th largest biased scores: a routing flip
    needs a logit error larger than this."""
    s = np.sort(choice)[::-1]
    return float(s[k - 1] - s[k]) if s.shape[0] > k else float("inf")


def rel_to_scale(ref, got):
    """max|ref - got| / max|ref| (src/test_glm_chain.cu:297-316)."""
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    return float(np.max(np.abs(ref - got)) / (np.max(np.abs(ref)) + 1e-300))


def align_weights(ref_idx, ref_w, got_idx, got_w):
    """got_w reordered to ref_idx's slot order (src/test_glm_chain.cu:747-754)."""
    pos = {int(e): i for i, e in enumerate(got_idx)}
    return np.array([got_w[pos[int(e)]] for e in ref_idx], dtype=np.float32)
