"""The caller side of a decoder layer on the GPU (run with -m gpu): MLA
attention with the DSA indexer (run_attention, src/glm_layer_runner.cuh:
525-661), the dense MLP (:373-384) and run_layer (:668-675).

Checked against transformers' GlmMoeDsaAttention / GlmMoeDsaMLP
(tests/golden/attn_tf_small.npz) and against the oracle (oracle/attention.py)
at the fixture's shape, at the GLM shape (with a small index_topk, and with
GLM's own 2048 over 2,112 positions) and over 2,500- and 8,400-position
sequences whose DSA selection drops most keys. Bars: f32 outputs within 1e-5
rel_to_scale; the selection equal to the oracle's, except where two index
scores at the top-k boundary are within 1e-5 of each other (then the oracle
is run with the GPU's selection, as the reference's --force-oracle-topk
does)."""
import json
import os

import numpy as np
import pytest

from oracle import attention as A
from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import hip as H_
from windlass_amd import moe, synthdata
from windlass_amd.model import AttnModel, DeviceModel

pytestmark = pytest.mark.gpu
TOL = 1e-5
HERE = os.path.dirname(os.path.abspath(__file__))
FIX = np.load(os.path.join(HERE, "golden", "attn_tf_small.npz"))
FCFG = json.loads(str(FIX["config"]))
GLM_ATTN = dict(hidden=6144, n_heads=64, q_lora_rank=2048, kv_lora_rank=512, qk_nope=192, qk_rope=64, v_head=256,
                index_n_heads=32, index_head_dim=128, index_topk=24, dense_inter=12288, rms_eps=1e-5,
                rope_theta=1e6)


def _step(am, layer, pos, h):
    """run_attention on h at pos: (new hidden, taps as host arrays)."""
    d = H_.DeviceBuffer.from_array(h.astype(np.float32))
    am.attn.run_attention(layer, pos, d.ptr)
    H_.synchronize()
    tp = am.attn.taps()
    a = am.a
    T = pos + 1
    out = {"h": d.download(np.float32),
           "norm": H_.download_ptr(tp["norm"], np.float32, a["hidden"]),
           "q_resid": H_.download_ptr(tp["q_resid"], np.float32, a["q_lora_rank"]),
           "attn": H_.download_ptr(tp["attn"], np.float32, a["n_heads"] * a["v_head"]),
           "attn_out": H_.download_ptr(tp["attn_out"], np.float32, a["hidden"]),
           "isc": H_.download_ptr(tp["index_score"], np.float32, T)}
    if tp["keep"]:
        out["keep"] = H_.download_ptr(tp["keep"], np.uint8, T).astype(bool)
    return out


def test_fixture_shape_vs_transformers_and_oracle(gpu):
    S, seed = int(FIX["seq"]), int(FIX["seed"])
    H = FCFG["hidden"]
    am = AttnModel(FCFG, seed, 2, owners=[True, False], dense=[0], max_seq=64)
    W = [synthdata.as_f32(w) for w in am.weights]
    cos, sin = A.rope_tables(S, FCFG["qk_rope"], FCFG["rope_theta"])
    caches = [A.LayerCache(), A.LayerCache()]
    worst = 0.0
    for p in range(S):
        share = A.IndexShare()
        for l in range(2):
            h = synth.hidden_state(H, seed * 100 + l, p)
            got = _step(am, l, p, h)
            taps = {}
            A.attn_block(h, W[l], FCFG, p, cos, sin, caches[l], l == 0, share, taps)
            for k in ("norm", "q_resid", "attn", "attn_out"):
                r = O.rel_to_scale(taps[k], got[k])
                worst = max(worst, r)
                assert r < TOL, (l, p, k, r)
            assert O.rel_to_scale(FIX[f"attn_out{l}"][p], got["attn_out"]) < TOL, (l, p)
            assert O.rel_to_scale(h + FIX[f"attn_out{l}"][p], got["h"]) < TOL, (l, p)
            if l == 0:
                assert np.array_equal(got["keep"], FIX["keep"][p, :p + 1]), p
                assert O.rel_to_scale(taps["index_score"], got["isc"]) < TOL, p
    mw = W and synthdata.as_f32(am.mlp[0])
    for p in range(4):
        h = synth.hidden_state(H, seed * 100 + 9, p)
        d = H_.DeviceBuffer.from_array(h)
        am.attn.run_dense_mlp(0, d.ptr)
        got = d.download(np.float32) - h
        assert O.rel_to_scale(FIX["mlp_out"][p], got) < TOL, p
        assert O.rel_to_scale(A.dense_mlp(h, mw, FCFG) - h, got) < TOL, p
    print(f"fixture shape: worst vs oracle {worst:.2e}", flush=True)
    am.close()


def _check_positions(am, W, a, Hs, checks, owner_rows, label):
    """Steps layer 0 (owner) and layer 1 (shared) through every position of
    Hs [T, H] (both layers get the same input) and compares the checked
    positions with the vectorised oracle."""
    T = Hs.shape[0]
    cos, sin = A.rope_tables(T, a["qk_rope"], a["rope_theta"])
    rows = [A.prefill_rows(Hs, W[0], a, cos, sin, True), A.prefill_rows(Hs, W[1], a, cos, sin, False)]
    worst, forced = 0.0, 0
    for p in range(T):
        g0 = _step(am, 0, p, Hs[p]) if p in checks else None
        if g0 is None:
            d = H_.DeviceBuffer.from_array(Hs[p])
            am.attn.run_attention(0, p, d.ptr)
        g1 = _step(am, 1, p, Hs[p]) if p in checks else None
        if g1 is None:
            d = H_.DeviceBuffer.from_array(Hs[p])
            am.attn.run_attention(1, p, d.ptr)
            continue
        isc, sel = A.index_select_at(p, rows[0], W[0], a, cos, sin)
        assert O.rel_to_scale(isc, g0["isc"]) < TOL, (label, p)
        want = ~A.index_drop_mask(sel, p + 1)
        if not np.array_equal(want, g0["keep"]):
            # only a near-tie at the boundary may differ: the k-th and (k+1)-th scores within 1e-5
            srt = np.sort(isc)[::-1]
            k = min(a["index_topk"], p + 1)
            assert k < p + 1 and abs(srt[k - 1] - srt[k]) <= 1e-5 * np.abs(isc).max(), (label, p)
            sel = np.nonzero(g0["keep"])[0]
            forced += 1
        assert int(g0["keep"].sum()) == min(a["index_topk"], p + 1)
        for l, g in ((0, g0), (1, g1)):
            o, out = A.attn_at(p, rows[l], W[l], a, sel)
            for ref, k in ((o, "attn"), (out, "attn_out")):
                r = O.rel_to_scale(ref, g[k])
                worst = max(worst, r)
                assert r < TOL, (label, l, p, k, r)
    print(f"{label}: {len(checks)} positions checked of {T}, worst {worst:.2e}, forced selections {forced}", flush=True)


def test_glm_shape(gpu):
    a = GLM_ATTN
    am = AttnModel(a, 21, 2, owners=[True, False], max_seq=64)
    W = [synthdata.as_f32(w) for w in am.weights]
    T = 40
    Hs = np.stack([synth.hidden_state(a["hidden"], 2100, p) for p in range(T)]).astype(np.float32)
    _check_positions(am, W, a, Hs, {0, 1, 23, 24, 25, 39}, None, "GLM shape")
    am.close()


def test_glm_shape_at_glm_selection_size(gpu):
    """GLM dimensions (hidden 6144, 64 heads, q_lora 2048, kv_lora 512,
    32 indexer heads of 128) with GLM's own index_topk of 2048 over 2,112
    positions: every key kept up to position 2047, then the radix select
    dropping 1, 2, 3 and 64 keys (positions 2048-2050 and the last)."""
    a = dict(GLM_ATTN, index_topk=2048)
    T = 2112
    am = AttnModel(a, 25, 2, owners=[True, False], max_seq=T)
    W = [synthdata.as_f32(w) for w in am.weights]
    Hs = np.stack([synth.hidden_state(a["hidden"], 2500, p) for p in range(T)]).astype(np.float32)
    _check_positions(am, W, a, Hs, {1000, 2046, 2047, 2048, 2049, 2050, T - 1}, None, "GLM at index_topk 2048")
    am.close()


def test_long_sequence_sparse_selection(gpu):
    """2,500 positions with index_topk 100: many key splits, and the
    radix-select top-k dropping all but 100 keys."""
    a = dict(FCFG, index_topk=100)
    am = AttnModel(a, 22, 2, owners=[True, False], max_seq=2560)
    W = [synthdata.as_f32(w) for w in am.weights]
    T = 2500
    Hs = np.stack([synth.hidden_state(a["hidden"], 2200, p) for p in range(T)]).astype(np.float32)
    _check_positions(am, W, a, Hs, {31, 32, 99, 100, 101, 1000, 2047, 2048, 2499}, None, "long sequence")
    am.close()


def test_very_long_sequence_topk_from_memory(gpu):
    """8,400 positions: past 8,192 keys the top-k kernel's threads hold more
    scores than it keeps in registers and read them from memory on every
    radix pass; positions on both sides of that switch are checked."""
    a = dict(FCFG, index_topk=100)
    T = 8400
    am = AttnModel(a, 24, 2, owners=[True, False], max_seq=T)
    W = [synthdata.as_f32(w) for w in am.weights]
    Hs = np.stack([synth.hidden_state(a["hidden"], 2400, p) for p in range(T)]).astype(np.float32)
    _check_positions(am, W, a, Hs, {8000, 8191, 8192, 8399}, None, "very long sequence")
    am.close()


def test_run_layer_composes(gpu):
    """wl_run_layer == run_attention then the MoE layer + residual (or the
    dense MLP), bit for bit."""
    a = dict(FCFG)
    mcfg = dict(hidden=a["hidden"], moe_inter=128, n_routed_experts=32, n_experts_per_tok=4, n_shared=1,
                routed_scaling=2.5, rms_eps=1e-5)
    am = AttnModel(a, 23, 2, owners=[True, False], dense=[0], max_seq=16)
    dm = DeviceModel(mcfg, seed=23, n_layers=1)
    H = a["hidden"]
    for p in range(3):
        h = synth.hidden_state(H, 2300, p)
        d1 = H_.DeviceBuffer.from_array(h)
        am.attn.run_layer(None, 0, 0, p, d1.ptr)  # dense layer 0
        am.attn.run_layer(dm.ctx, 1, 0, p, d1.ptr)  # MoE layer 1
        H_.synchronize()
        got = d1.download(np.float32)
        d2 = H_.DeviceBuffer.from_array(h)
        am.attn.run_attention(0, p, d2.ptr)
        am.attn.run_dense_mlp(0, d2.ptr)
        am.attn.run_attention(1, p, d2.ptr)
        out = H_.DeviceBuffer(4 * H)
        dm.ctx.run_moe_residual(0, d2.ptr, d2.ptr, out.ptr)
        H_.synchronize()
        assert np.array_equal(got.view(np.uint32), out.download(np.float32).view(np.uint32)), p
    dm.close()
    am.close()


def test_errors(gpu):
    a = dict(FCFG)
    am = AttnModel(a, 24, 2, owners=[True, False], max_seq=8)
    d = H_.DeviceBuffer(4 * a["hidden"] + 64)

    def status(fn, *args):
        with pytest.raises(moe.WindlassError) as ei:
            fn(*args)
        return ei.value.status

    assert status(am.attn.run_attention, 1, 0, d.ptr) == 5    # shared layer, nothing published: WL_ERR_STATE
    am.attn.run_attention(0, 0, d.ptr)
    am.attn.run_attention(1, 0, d.ptr)                         # published at 0: runs
    assert status(am.attn.run_attention, 1, 1, d.ptr) == 5    # published at 0, asked at 1
    assert status(am.attn.run_attention, 0, 8, d.ptr) == 1    # pos >= max_seq
    assert status(am.attn.run_attention, 0, 1, d.ptr + 4) == 1  # misaligned hidden
    assert status(am.attn.run_attention, 2, 0, d.ptr) == 1    # no such layer
    assert status(am.attn.run_dense_mlp, 0, d.ptr) == 5       # no MLP bound
    am.close()
    with pytest.raises(moe.WindlassError):
        moe.Attention(moe.make_attn_config(n_heads=24))


@pytest.mark.parametrize("N,K", [(48, 256), (2048, 6144), (6144, 16384), (100, 24), (16384, 2048), (1, 8), (7, 520),
                                 (3000, 1032), (65536, 64)])
def test_matvec_bf16(gpu, N, K):
    """wl_matvec_bf16 against an fp64 product of the same bf16 weights and f32
    input, within 1e-5 term-relative (the reference's matvec test bar,
    src/test_glm_mxfp4.cu:186-191, applied to bf16)."""
    rng = np.random.default_rng(N + K)
    W = synthdata.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    x = rng.standard_normal(K).astype(np.float32)
    dW, dx, dy = H_.DeviceBuffer.from_array(W), H_.DeviceBuffer.from_array(x), H_.DeviceBuffer(4 * N)
    moe.matvec_bf16(dW.ptr, dx.ptr, dy.ptr, N, K)
    H_.synchronize()
    y = dy.download(np.float32)
    Wf = synthdata.bf16_to_f32(W).astype(np.float64)
    ref = Wf @ x.astype(np.float64)
    scale = np.abs(Wf) @ np.abs(x.astype(np.float64))
    assert np.max(np.abs(y - ref) / scale) < 1e-5
