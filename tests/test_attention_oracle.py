"""The attention / dense-MLP oracle (oracle/attention.py) against transformers'
GlmMoeDsaAttention and GlmMoeDsaMLP (tests/golden/attn_tf_small.npz, written
by tests/golden/make_golden.py), position by position in decode form, with
planted mistakes that the fixture must catch (CPU)."""
import json
import os

import numpy as np
import pytest

from oracle import attention as A
from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import synthdata

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "attn_tf_small.npz"))
CFG = json.loads(str(FIX["config"]))
S, SEED = int(FIX["seq"]), int(FIX["seed"])
TOL = 1e-5


def run_oracle():
    """Both layers over the sequence, one position at a time: layer 0 owns
    the indexer and publishes, layer 1 consumes. Returns attn_out[layer][p],
    the selection keep masks of layer 0, and the MLP outputs."""
    H = CFG["hidden"]
    W = [synthdata.as_f32(synthdata.attention_layer(CFG, SEED, l, owner=(l == 0))) for l in range(2)]
    cos, sin = A.rope_tables(S, CFG["qk_rope"], CFG["rope_theta"])
    caches = [A.LayerCache(), A.LayerCache()]
    outs = [[], []]
    keep = np.zeros((S, S), bool)
    for p in range(S):
        share = A.IndexShare()
        for l in range(2):
            h = synth.hidden_state(H, SEED * 100 + l, p)
            taps = {}
            A.attn_block(h, W[l], CFG, p, cos, sin, caches[l], l == 0, share, taps)
            outs[l].append(taps["attn_out"])
            if l == 0:
                keep[p, taps["index_sel"]] = True
    mw = synthdata.as_f32(synthdata.dense_mlp(H, CFG["dense_inter"], SEED, 0))
    mlp = [A.dense_mlp(synth.hidden_state(H, SEED * 100 + 9, p), mw, CFG) - synth.hidden_state(H, SEED * 100 + 9, p)
           for p in range(4)]
    return [np.stack(o) for o in outs], keep, np.stack(mlp)


def mismatch(outs, keep, mlp):
    """Worst rel_to_scale over every checked output, and whether the
    selections agree."""
    worst = 0.0
    for l in range(2):
        for p in range(S):
            worst = max(worst, O.rel_to_scale(FIX[f"attn_out{l}"][p], outs[l][p]))
    for p in range(4):
        worst = max(worst, O.rel_to_scale(FIX["mlp_out"][p], mlp[p]))
    return worst, bool(np.array_equal(keep, FIX["keep"]))


def test_oracle_matches_transformers():
    worst, same_sel = mismatch(*run_oracle())
    assert same_sel
    assert worst < TOL, worst
    # the selection is sparse from position index_topk on: the mask is live
    assert FIX["keep"][-1].sum() == CFG["index_topk"] < S


def _rms_as_layer_norm(x, w, b, eps):
    return A.rms_norm(x, w, eps)


PLANTED = {
    # the indexer's k_norm as RMSNorm (no mean, no bias)
    "k_norm_rms": ("layer_norm", _rms_as_layer_norm),
    # RoPE on the pass part instead of the rope part of the indexer key
    "index_rope_tail": ("indexer_keys", lambda x, W, cfg, pos, cos, sin: np.concatenate(
        [(x.astype(np.float32) @ W["idx_wk"].T)[..., :cfg["index_head_dim"] - cfg["qk_rope"]],
         A.rope_interleave(A.layer_norm(x.astype(np.float32) @ W["idx_wk"].T, W["idx_k_norm_w"], W["idx_k_norm_b"],
                                        A.INDEXER_LN_EPS)[..., cfg["index_head_dim"] - cfg["qk_rope"]:],
                           cos[pos], sin[pos])], -1)),
    # every key kept (the drop mask ignored)
    "no_mask": ("index_drop_mask", lambda sel, T: np.zeros(T, bool)),
    # the half-split RoPE of DeepSeek-V3 instead of the interleaved one
    "rope_halves": ("rope_interleave", lambda x, cos, sin: np.concatenate(
        [x[..., :x.shape[-1] // 2] * cos - x[..., x.shape[-1] // 2:] * sin,
         x[..., x.shape[-1] // 2:] * cos + x[..., :x.shape[-1] // 2] * sin], -1)),
    # the selection by the lowest scores
    "topk_lowest": ("indexer_topk", lambda s, k: np.argsort(s, kind="stable")[:min(k, s.shape[0])].astype(np.int32)),
}


@pytest.mark.parametrize("name", sorted(PLANTED))
def test_planted_mistakes_are_caught(monkeypatch, name):
    attr, fn = PLANTED[name]
    monkeypatch.setattr(A, attr, fn)
    worst, same_sel = mismatch(*run_oracle())
    assert worst > 100 * TOL or not same_sel, (name, worst)


def test_lora_eps_matters(monkeypatch):
    """q_a / kv_a norms take eps 1e-6, not the layer's 1e-5: with inputs of
    small scale the difference shows."""
    x = np.full(64, 1e-3, np.float32)
    w = np.ones(64, np.float32)
    a, b = A.rms_norm(x, w, A.LORA_NORM_EPS), A.rms_norm(x, w, 1e-5)
    assert abs(a[0] - 1.0 / np.sqrt(1.0 + 1.0)) < 1e-6  # 1e-6 / (1e-3)^2 = 1: rsqrt(2) per element
    assert abs(b[0] - a[0]) > 0.1


def test_vectorised_rows_equal_the_step_function():
    """prefill_rows + index_select_at + attn_at (used by the long GPU tests)
    give attn_block's outputs position by position."""
    H = CFG["hidden"]
    cos, sin = A.rope_tables(S, CFG["qk_rope"], CFG["rope_theta"])
    W0 = synthdata.as_f32(synthdata.attention_layer(CFG, SEED, 0, owner=True))
    Hs = np.stack([synth.hidden_state(H, SEED * 100, p) for p in range(S)])
    rows = A.prefill_rows(Hs, W0, CFG, cos, sin, True)
    cache = A.LayerCache()
    for p in range(S):
        taps = {}
        A.attn_block(Hs[p], W0, CFG, p, cos, sin, cache, True, A.IndexShare(), taps)
        isc, sel = A.index_select_at(p, rows, W0, CFG, cos, sin)
        assert O.rel_to_scale(taps["index_score"], isc) < 1e-6
        assert np.array_equal(np.sort(taps["index_sel"]), np.sort(sel))
        o, out = A.attn_at(p, rows, W0, CFG, sel)
        assert O.rel_to_scale(taps["attn"], o) < 1e-6
        assert O.rel_to_scale(taps["attn_out"], out) < 1e-6
