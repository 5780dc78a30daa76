"""The oracle pinned against the reference's known answers, an independent
implementation (transformers 5.15.0) and closed forms. CPU only."""
import json
import os

import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import native, synth

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def test_hand_fixture_exact():
    # tools/glm_mxfp4_numpy.py:44-52 — written out by hand, incl. the -0.0 at column 7
    fx = json.load(open(os.path.join(GOLD, "mxfp4_hand_fixture.json")))
    w = np.array([fx["w"]], dtype=np.uint8)
    s = np.array([fx["s"]], dtype=np.uint8)
    d = O.dequant(w, s)[0]
    exp = np.array(fx["expected"], dtype=np.float32)
    assert np.array_equal(d, exp)
    assert np.signbit(d[fx["negative_zero_index"]])


def test_hand_fixture_catches_planted_mistakes():
    fx = json.load(open(os.path.join(GOLD, "mxfp4_hand_fixture.json")))
    w = np.array([fx["w"]], dtype=np.uint8)
    s = np.array([fx["s"]], dtype=np.uint8)
    exp = np.array(fx["expected"], dtype=np.float32)

    def hi_even(w, s):  # nibble order flipped (a plausible mistake)
        out = np.empty((w.shape[0], w.shape[1] * 2), np.float32)
        out[:, 0::2] = O.E2M1[w >> 4]
        out[:, 1::2] = O.E2M1[w & 0xF]
        return out * np.repeat(np.exp2(s.astype(np.float32) - 127), 32, axis=1)

    def scale_inverted(w, s):
        out = O.dequant(w, s)
        return out / np.repeat(np.exp2(s.astype(np.float32) - 127), 32, axis=1) ** 2

    assert not np.array_equal(hi_even(w, s)[0], exp)
    assert not np.array_equal(scale_inverted(w, s)[0], exp)


def test_dequant_matches_transformers():
    fx = np.load(os.path.join(GOLD, "dequant_tf.npz"))
    assert np.array_equal(O.dequant(fx["w"], fx["s"]), fx["expected"])


def test_scale_closed_form_and_numpy_exp2_quirk():
    # 2^(s-127) exactly for every finite E8M0 byte; numpy's float32 exp2 (the
    # reference's formula) agrees everywhere but s = 254
    s = np.arange(0, 255, dtype=np.uint8).reshape(-1, 1)
    w = np.full((255, 16), 0x22, np.uint8)  # every value 1.0
    d = O.dequant(w, s)
    exact = np.array([np.ldexp(np.float32(1), k - 127) for k in range(255)], np.float32)
    assert np.array_equal(d[:, 0], exact)
    np_exp2 = np.exp2(s[:, 0].astype(np.float32) - np.float32(127.0))
    assert [int(k) for k in np.nonzero(np_exp2 != exact)[0]] == [254]
    assert np.isnan(O.dequant(w[:1], np.array([[255]], np.uint8))).all()


def test_generators_agree():
    # numpy restatement vs the C restatement of the device generator
    for seed, layer, expert in [(0, 0, 0), (7, 3, 11), (123, 23, 255)]:
        k = synth.synth_key(seed, layer, expert)
        assert k == native.synth_key(seed, layer, expert)
        for r in range(6):
            assert np.array_equal(synth.region_bytes(k, r, 8192), native.synth_region(k, r, 8192))


def test_generator_distribution():
    gw, gs, *_ = synth.expert_block(6144, 2048, 0, 0, 0)
    nib = np.concatenate([(gw & 0xF).ravel(), (gw >> 4).ravel()])
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.95 * nib.size / 16 and counts.max() < 1.05 * nib.size / 16
    assert gs.min() == 118 and gs.max() == 126
    sc = np.bincount(gs.ravel() - 118, minlength=9)
    assert sc.min() > 0.95 * gs.size / 9


@pytest.mark.parametrize("seed", [0x915, 0x1])
@pytest.mark.parametrize("shape", [(2048, 6144), (6144, 2048)])
def test_dequant_matvec_fp32_vs_fp64(seed, shape):
    # numpy fp32 (dequant + BLAS) vs fp64 brute force, term-relative bar 1e-5
    # (src/test_glm_mxfp4.cu:95-105,186-191)
    N, K = shape
    rng = np.random.default_rng(seed)
    W = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    S = rng.integers(118, 127, size=(N, K // 32), dtype=np.uint8)
    x = rng.uniform(-1, 1, size=K).astype(np.float32)
    y32 = O.dequant(W, S) @ x
    y64, absacc = native.dequant_matvec_f64(W, S, x)
    term_rel = np.max(np.abs(y32 - y64) / absacc)
    assert term_rel < 1e-6


def test_rms_norm_closed_form():
    x = np.full(64, 3.0, np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    y = O.rms_norm(x, w, 1e-5)
    np.testing.assert_allclose(y, w * (3.0 / np.sqrt(9.0 + 1e-5)), rtol=1e-6)


def test_route_brute_force_and_ties():
    rng = np.random.default_rng(5)
    E, H, K = 24, 16, 5
    W = rng.standard_normal((E, H)).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    bias = np.zeros(E, np.float32)
    logits, idx, w, choice = O.route(x, W, bias, K, 2.5, True)
    # brute force: repeated strict-> argmax, ties to the lowest index
    c = choice.astype(np.float64).copy()
    picked = []
    for _ in range(K):
        b = int(np.argmax(c))  # numpy argmax returns the first maximum
        picked.append(b)
        c[b] = -np.inf
    assert list(idx) == picked
    s = 1 / (1 + np.exp(-logits.astype(np.float64)))
    ref_w = s[picked] / s[picked].sum() * 2.5
    np.testing.assert_allclose(w, ref_w, rtol=2e-6)
    assert abs(w.sum() - 2.5) < 1e-5
    # exact ties: equal choices resolve to the lower index
    logits_t = np.zeros(E, np.float32)
    _, idx_t, _, _ = O.route(np.zeros(H, np.float32), np.zeros((E, H), np.float32), bias, K, 2.5, True)
    assert list(idx_t) == list(range(K))


def test_route_negative_controls():
    rng = np.random.default_rng(9)
    E, H, K = 64, 32, 8
    W = rng.standard_normal((E, H)).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    # real-checkpoint-like bias: ~34 +- 0.138 (tools/dump_glm_oracle.py:123-127)
    bias = (34.0 + 0.138 * rng.standard_normal(E)).astype(np.float32)
    _, idx, w, _ = O.route(x, W, bias, K, 2.5, True)
    # bias cast to bf16 collapses the selection
    b16 = synth.bf16_to_f32(synth.f32_to_bf16(bias))
    _, idx16, _, _ = O.route(x, W, b16, K, 2.5, True)
    assert set(idx16) != set(idx)
    # routed_scaling 1.0 is caught by the weights
    _, _, w1, _ = O.route(x, W, bias, K, 1.0, True)
    assert O.rel_to_scale(w, w1) > 0.5
    # weight gathered from the biased score is caught by the weights
    logits = x @ W.T
    s = 1 / (1 + np.exp(-logits))
    wb = (s + bias)[idx]
    wb = wb / wb.sum() * 2.5
    assert O.rel_to_scale(w, wb.astype(np.float32)) > 1e-3


def _small_cfg():
    fx = np.load(os.path.join(GOLD, "moe_tf_small.npz"))
    return fx, json.loads(str(fx["config"]))


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5])
def test_moe_layer_matches_transformers(seed):
    fx, c = _small_cfg()
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    dense = synth.dense_layer(H, E, I, seed, 0)
    h = synth.hidden_state(H, seed)
    r = O.moe_layer(h, dense, O.ExpertSource(H, I, seed), 0, c)
    p = f"s{seed}_"
    assert O.rel_to_scale(fx[p + "norm"], r["norm"]) < 1e-6
    assert O.rel_to_scale(fx[p + "logits"], r["logits"]) < 1e-6
    assert np.array_equal(np.sort(r["topk_idx"]), fx[p + "topk_idx_sorted"])
    got_w = O.align_weights(fx[p + "topk_idx_sorted"], None, r["topk_idx"], r["topk_w"])
    assert O.rel_to_scale(fx[p + "topk_w_by_sorted_id"], got_w) < 1e-6
    assert O.rel_to_scale(fx[p + "shared"], r["shared"]) < 1e-6
    assert O.rel_to_scale(fx[p + "out"], r["out"]) < 1e-5


def test_moe_layer_negative_controls():
    # the layer gate (1e-5 rel_to_scale) fails on each planted mistake
    fx, c = _small_cfg()
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    seed = 0
    dense = synth.dense_layer(H, E, I, seed, 0)
    h = synth.hidden_state(H, seed)
    ref = fx["s0_out"]
    bad = dict(c, routed_scaling=1.0)
    assert O.rel_to_scale(ref, O.moe_layer(h, dense, O.ExpertSource(H, I, seed), 0, bad)["out"]) > 1e-2

    class Swapped(O.ExpertSource):
        def get(self, layer, expert):
            G, U, D = super().get(layer, expert)
            return G[:, ::-1].copy(), U, D  # column order scrambled

    assert O.rel_to_scale(ref, O.moe_layer(h, dense, Swapped(H, I, seed), 0, c)["out"]) > 1e-2


def test_product_and_oracle_input_recipes_agree():
    # the product's input generator and the oracle's restatement of it
    from windlass_amd import synthdata
    a = synthdata.dense_layer(256, 32, 128, 5, 2)
    b = synth.dense_layer(256, 32, 128, 5, 2)
    for k in a:
        assert np.array_equal(a[k], b[k]), k
    assert np.array_equal(synthdata.hidden_state(256, 3, 1), synth.hidden_state(256, 3, 1))
    assert np.array_equal(synthdata.zipf_bias_offset(64, 4), synth.zipf_bias_offset(64, 4))


@pytest.mark.parametrize("shape", [(256, 128), (384, 256), (6144, 2048)])
def test_native_layout_is_a_reordering(shape):
    """The native layout restatement moves every weight byte exactly once and
    puts every real scale byte of a lane's row where the kernel reads it."""
    from oracle import native_layout
    H, I = shape
    parts = synth.expert_block(H, I, 5, 1, 7)
    nat = native_layout.to_native(parts, H, I)
    gu, gus, dn, dns, bgus, bdns = native_layout.native_sizes(H, I)
    assert nat.size == gu + gus + dn + dns + bgus + bdns
    assert np.array_equal(np.sort(nat[:gu]), np.sort(np.concatenate([parts[0].ravel(), parts[2].ravel()])))
    assert np.array_equal(np.sort(nat[gu + gus:gu + gus + dn]), np.sort(parts[4].ravel()))
    # lane (n=3, g=2) of tile 1, k tile 1: gate row 11, bytes [64 + 32, +16)
    nkt = H // 128
    chunk = nat[(1 * nkt + 1) * 1024:(1 * nkt + 2) * 1024].reshape(64, 16)
    assert np.array_equal(chunk[2 * 16 + 3], parts[0][11, 96:112])
    # its scale: byte 1 of lane 35's chunk in tile 1's first scale chunk = gate_s[11, 4*1 + 2]
    sc = nat[gu + 1 * ((nkt + 15) // 16) * 1024:][:1024].reshape(64, 16)
    assert sc[35, 1] == parts[1][11, 6]
    # the batched kernels' copy of the same scales: group 0, wave 1 (tile 1 =
    # 8 * slice 0 + 1), step 0, lane 35, byte 2 * 0 + 1 (k tile 1)
    base = gu + gus + dn + dns
    word = nat[base + ((0 * 8 + 1) * -(-H // 256) + 0) * 512:][:512].reshape(64, 8)
    assert word[35, 1] == parts[1][11, 6]
    # and every scale byte of each region appears in it as often as the
    # kernels read it: each real gate/up scale once, each real down scale once
    bg = nat[base:base + bgus]
    assert np.array_equal(np.sort(bg[bg != 0]), np.sort(np.concatenate([parts[1].ravel(), parts[3].ravel()])[
        np.concatenate([parts[1].ravel(), parts[3].ravel()]) != 0]))
    bd = nat[base + bgus:base + bgus + bdns]
    assert np.array_equal(np.sort(bd[bd != 0]), np.sort(parts[5].ravel()[parts[5].ravel() != 0]))
    # down: row block 0, wave 2 (row pairs 4, 5), step 0, lane (n=3, g=3): byte
    # 2 * 1 + 1 = slice 1, pair 5: down row 32 * 5 + 3 + 16 = 179, block 2 * 1 + 1
    word = nat[base + bgus + ((0 * 8 + 2) * -(-I // 256) + 0) * 512:][:512].reshape(64, 8)
    assert word[3 * 16 + 3, 3] == parts[5][179, 3]
