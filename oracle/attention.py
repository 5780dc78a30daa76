"""CPU restatement of the caller side of a decoder layer — parity oracle:
input_layernorm -> MLA attention with the DSA indexer -> o_proj -> first
residual, and the dense MLP of layers below dense_first.

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker, and by bench.py's
cpu_baseline leg). The product path never imports it.

Restates tools/ref_glm_chain.py (the reference's numpy decoder layer):
  rms_norm            :63-80   (eps 1e-5 for the layer norms, 1e-6 for the
                                q_a / kv_a LoRA norms: LORA_NORM_EPS)
  rope_tables         :83-94   (inv_freq in float64, cos/sin rounded to f32)
  rope_interleave     :97-106  (adjacent input pairs -> halves layout)
  layer_norm          :109-120 (the indexer's k_norm: LayerNorm with bias)
  indexer_keys        :465-479 (RoPE on the LEADING qk_rope of the key)
  indexer_scores      :482-501 (relu between q.k and the head weighting;
                                scales D^-0.5 and n_heads^-0.5)
  indexer_topk        :504-515
  index_drop_mask     :518-532
  attn_block          :556-643 (materialised per-head K/V, like transformers)
  dense MLP           :700-701 (moe_finish's dense branch)
The decode form caches exactly positions 0..pos, so causality is structural.
"""
import numpy as np

LORA_NORM_EPS = 1e-6
INDEXER_LN_EPS = 1e-6


def rms_norm(x, w, eps):
    x = x.astype(np.float32)
    return w.astype(np.float32) * (x * (np.float32(1.0) / np.sqrt((x * x).mean(-1, keepdims=True) + np.float32(eps))))


def rope_tables(max_pos, rot, theta):
    inv = 1.0 / (theta ** (np.arange(0, rot, 2, dtype=np.float64) / rot))
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_interleave(x, cos, sin):
    a, b = x[..., 0::2], x[..., 1::2]
    return np.concatenate([a * cos - b * sin, b * cos + a * sin], axis=-1)


def layer_norm(x, w, b, eps):
    x = x.astype(np.float32)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + np.float32(eps)) * w.astype(np.float32) + b.astype(np.float32)


def silu(x):
    with np.errstate(over="ignore"):
        return x / (np.float32(1.0) + np.exp(-x))


def indexer_keys(x, W, cfg, pos, cos, sin):
    R = cfg["qk_rope"]
    k = x.astype(np.float32) @ W["idx_wk"].T
    k = layer_norm(k, W["idx_k_norm_w"], W["idx_k_norm_b"], INDEXER_LN_EPS)
    return np.concatenate([rope_interleave(k[..., :R], cos[pos], sin[pos]), k[..., R:]], -1)


def indexer_scores(q_resid, x, K_ix, W, cfg, pos, cos, sin):
    IH, ID, R = cfg["index_n_heads"], cfg["index_head_dim"], cfg["qk_rope"]
    q = (q_resid.astype(np.float32) @ W["idx_wq_b"].T).reshape(IH, ID)
    q = np.concatenate([rope_interleave(q[:, :R], cos[pos], sin[pos]), q[:, R:]], -1)
    s = np.maximum((q @ K_ix.T) * np.float32(ID ** -0.5), np.float32(0.0))
    w = (W["idx_weights_proj"] @ x.astype(np.float32)) * np.float32(IH ** -0.5)
    return q, w, (w[:, None] * s).sum(0, dtype=np.float32)


def indexer_topk(index_score, index_topk):
    k = min(index_topk, index_score.shape[0])
    return np.argsort(-index_score, kind="stable")[:k].astype(np.int32)


def index_drop_mask(sel, T):
    drop = np.ones(T, bool)
    sel = np.asarray(sel)
    drop[sel[(sel >= 0) & (sel < T)]] = False
    return drop


class LayerCache:
    """Per-layer decode cache: materialised K [T, HN, DH], V [T, HN, VD] and
    the indexer keys [T, ID] (f32)."""

    def __init__(self):
        self.k, self.v, self.ik = [], [], []


class IndexShare:
    """prev_topk_indices threaded through the layers of one token
    (tools/ref_glm_chain.py:444-462): a full layer publishes its raw
    selection, a shared layer consumes it unchanged and raises if empty."""

    def __init__(self):
        self.indices = None


def attn_block(h, W, cfg, pos, cos, sin, cache, owner, share, taps=None):
    """input_layernorm .. o_proj + first residual for ONE position.
    Returns the new hidden state; taps (a dict) receives the substeps."""
    HN, NP, RP, VD, L = cfg["n_heads"], cfg["qk_nope"], cfg["qk_rope"], cfg["v_head"], cfg["kv_lora_rank"]
    DH = NP + RP
    tap = (lambda k, v: taps.__setitem__(k, np.asarray(v))) if taps is not None else (lambda k, v: None)
    x = rms_norm(h, W["input_ln"], cfg["rms_eps"])
    tap("norm", x)
    q_resid = rms_norm(x @ W["q_a_proj"].T, W["q_a_ln"], LORA_NORM_EPS)
    tap("q_resid", q_resid)
    q = (q_resid @ W["q_b_proj"].T).reshape(HN, DH)
    q_pass, q_rot = q[:, :NP], q[:, NP:]
    ckv = x @ W["kv_a_proj"].T
    kc, k_rot = ckv[:L], ckv[L:]
    kc = rms_norm(kc, W["kv_a_ln"], LORA_NORM_EPS)
    tap("kv_c", kc)
    kv = (kc @ W["kv_b_proj"].T).reshape(HN, NP + VD)
    k_pass, v = kv[:, :NP], kv[:, NP:]
    if owner:
        cache.ik.append(indexer_keys(x, W, cfg, pos, cos, sin))
        q_ix, w_ix, isc = indexer_scores(q_resid, x, np.stack(cache.ik), W, cfg, pos, cos, sin)
        sel = indexer_topk(isc, cfg["index_topk"])
        tap("index_q", q_ix)
        tap("index_w", w_ix)
        tap("index_score", isc)
        tap("index_sel", sel)
        share.indices = sel
    elif share.indices is None:
        raise RuntimeError("shared layer with no published indexer selection")
    else:
        sel = share.indices
    q_rot = rope_interleave(q_rot, cos[pos], sin[pos])
    k_rot = rope_interleave(k_rot, cos[pos], sin[pos])
    tap("k_rot", k_rot)
    k = np.concatenate([k_pass, np.broadcast_to(k_rot, (HN, RP))], -1)
    q = np.concatenate([q_pass, q_rot], -1)
    cache.k.append(k)
    cache.v.append(v)
    K = np.stack(cache.k)
    V = np.stack(cache.v)
    s = np.einsum("hd,thd->ht", q, K).astype(np.float32) * np.float32(DH ** -0.5)
    drop = index_drop_mask(sel, K.shape[0])
    if drop.any():
        s = np.where(drop, -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = np.einsum("ht,thd->hd", p, V).reshape(HN * VD).astype(np.float32)
    tap("attn", o)
    attn_out = o @ W["o_proj"].T
    tap("attn_out", attn_out)
    return (h + attn_out).astype(np.float32)


def dense_mlp(h, W, cfg, taps=None):
    """post_attention_layernorm -> SwiGLU MLP -> second residual."""
    xn = rms_norm(h, W["post_ln"], cfg["rms_eps"])
    y = (silu(xn @ W["gate"].T) * (xn @ W["up"].T)) @ W["down"].T
    if taps is not None:
        taps["mlp_norm"] = xn
        taps["mlp_out"] = y
    return (h + y).astype(np.float32)


def prefill_rows(Hs, W, cfg, cos, sin, owner):
    """Everything position p's own input decides, for every row of Hs [T, H]
    at positions 0..T-1, vectorised (tools/ref_glm_chain.py:749-786 does the
    same for its long cross-checks): the norm, q_resid, the rotated query, K,
    V and the indexer key. attn_at then runs one position against the rows
    before it. Equal to attn_block stepped position by position
    (tests/test_attention_oracle.py)."""
    HN, NP, RP, VD, L = cfg["n_heads"], cfg["qk_nope"], cfg["qk_rope"], cfg["v_head"], cfg["kv_lora_rank"]
    T = Hs.shape[0]
    pos = np.arange(T)
    x = rms_norm(Hs, W["input_ln"], cfg["rms_eps"])
    q_resid = rms_norm(x @ W["q_a_proj"].T, W["q_a_ln"], LORA_NORM_EPS)
    q = (q_resid @ W["q_b_proj"].T).reshape(T, HN, NP + RP)
    ckv = x @ W["kv_a_proj"].T
    kc = rms_norm(ckv[:, :L], W["kv_a_ln"], LORA_NORM_EPS)
    kv = (kc @ W["kv_b_proj"].T).reshape(T, HN, NP + VD)
    c, s = cos[pos][:, None, :], sin[pos][:, None, :]
    q_rot = rope_interleave(q[:, :, NP:], c, s)
    k_rot = rope_interleave(ckv[:, L:], cos[pos], sin[pos])
    rows = {"x": x, "q_resid": q_resid, "q": np.concatenate([q[:, :, :NP], q_rot], -1),
            "K": np.concatenate([kv[:, :, :NP], np.broadcast_to(k_rot[:, None, :], (T, HN, RP))], -1),
            "V": kv[:, :, NP:]}
    if owner:
        rows["ik"] = np.stack([indexer_keys(x[p], W, cfg, p, cos, sin) for p in range(T)])
    return rows


def index_select_at(p, rows, W, cfg, cos, sin):
    """(index scores over keys 0..p, selection) of an owning layer at p."""
    _, _, isc = indexer_scores(rows["q_resid"][p], rows["x"][p], rows["ik"][:p + 1], W, cfg, p, cos, sin)
    return isc, indexer_topk(isc, cfg["index_topk"])


def attn_at(p, rows, W, cfg, sel):
    """The attention context (before o_proj) and o_proj output of position p
    over keys 0..p, keys outside `sel` dropped."""
    HN, NP, RP, VD = cfg["n_heads"], cfg["qk_nope"], cfg["qk_rope"], cfg["v_head"]
    K, V = rows["K"][:p + 1], rows["V"][:p + 1]
    s = np.einsum("hd,thd->ht", rows["q"][p], K).astype(np.float32) * np.float32((NP + RP) ** -0.5)
    drop = index_drop_mask(sel, p + 1)
    if drop.any():
        s = np.where(drop, -np.inf, s)
    e = np.exp(s - s.max(-1, keepdims=True))
    e /= e.sum(-1, keepdims=True)
    o = np.einsum("ht,thd->hd", e, V).reshape(HN * VD).astype(np.float32)
    return o, o @ W["o_proj"].T
