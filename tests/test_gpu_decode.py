"""Parity of the HIP decode path with the oracle (GPU; run with -m gpu).

Bars: expert ids bit-exact as a set; f32 outputs within 1e-5 rel_to_scale
(max|d|/max|ref|, src/test_glm_chain.cu:297-316) of the numpy oracle; MXFP4
matvecs within 1e-5 term-relative of the fp64 brute force
(src/test_glm_mxfp4.cu:186-191)."""
import json
import os

import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import native, synth
from windlass_amd import hip as H_, moe
from windlass_amd.model import DeviceModel, make_io

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
TOL = 1e-5
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)
SEEDS8 = [0x915, 0x1, 0x42, 0xABC, 0xDEAD, 0xF00D, 0x2718, 0x1618]


def _taps(dm, hip):
    t = dm.ctx.taps()
    c = dm.c
    H, E, K, I = c["hidden"], c["n_routed_experts"], c["n_experts_per_tok"], c["moe_inter"]
    return {"norm": hip.download_ptr(t["norm"], np.float32, H),
            "logits": hip.download_ptr(t["logits"], np.float32, E),
            "topk_idx": hip.download_ptr(t["topk_idx"], np.int32, K),
            "topk_w": hip.download_ptr(t["topk_w"], np.float32, K),
            "mid": hip.download_ptr(t["mid"], np.float32, K * I).reshape(K, I),
            "shared": hip.download_ptr(t["shared"], np.float32, H)}


def _check_layer(ref, got, out, tag):
    assert O.rel_to_scale(ref["norm"], got["norm"]) < TOL, tag
    assert O.rel_to_scale(ref["logits"], got["logits"]) < TOL, tag
    assert np.array_equal(np.sort(ref["topk_idx"]), np.sort(got["topk_idx"])), (tag, ref["topk_idx"], got["topk_idx"])
    # the device emits slots in descending biased score, ties to the lowest id
    assert np.array_equal(ref["topk_idx"], got["topk_idx"]), tag
    assert O.rel_to_scale(ref["topk_w"], O.align_weights(ref["topk_idx"], None, got["topk_idx"], got["topk_w"])) < TOL
    assert O.rel_to_scale(ref["mid"], got["mid"]) < TOL, tag
    assert O.rel_to_scale(ref["shared"], got["shared"]) < TOL, tag
    r = O.rel_to_scale(ref["out"], out)
    assert r < TOL, (tag, r)
    return r


@pytest.mark.parametrize("shape", [(2048, 6144), (6144, 2048)])
def test_dequant_matvec_eight_seeds(gpu, shape):
    """The reference's unit test (src/test_glm_mxfp4.cu:138-191): 8 seeds, bytes
    uniform, E8M0 in [120,134], x ~ U(-1,1); worst term-relative < 1e-5."""
    hip = gpu
    N, K = shape
    worst = 0.0
    for seed in SEEDS8:
        rng = np.random.default_rng(seed)
        W = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
        S = rng.integers(120, 135, size=(N, K // 32), dtype=np.uint8)
        x = rng.uniform(-1, 1, size=K).astype(np.float32)
        dW, dS, dx = (hip.DeviceBuffer.from_array(a) for a in (W, S, x))
        dy = hip.DeviceBuffer(4 * N)
        moe.dequant_matvec_mxfp4(dW.ptr, dS.ptr, dx.ptr, dy.ptr, N, K)
        hip.synchronize()
        y = dy.download(np.float32)
        y64, absacc = native.dequant_matvec_f64(W, S, x)
        worst = max(worst, float(np.max(np.abs(y - y64) / absacc)))
    print(f"dequant_matvec {N}x{K}: worst term_rel over 8 seeds {worst:.3e}", flush=True)
    assert worst < 1e-5


def test_expert_ffn_config0(gpu):
    """Config 0: one MXFP4 expert SwiGLU FFN at bs=1, 8 seeds; f32 output within
    1e-5 rel_to_scale of the oracle, bf16 output = RNE of the f32 output."""
    hip = gpu
    H, I = 6144, 2048
    cfg = moe.make_config(hidden=H, moe_inter=I)
    ctx = moe.Context(cfg)
    lay = moe.expert_layout(cfg)
    blk = hip.DeviceBuffer(lay.total)
    dx, dy = make_io(H)
    dyb = hip.DeviceBuffer(2 * H)
    worst = 0.0
    for i, seed in enumerate(SEEDS8):
        moe.synth_expert(cfg, seed, 0, 0, blk.ptr)
        x = synth.hidden_state(H, seed)
        dx.upload(x)
        ctx.expert_ffn(blk.ptr, dx.ptr, dy.ptr, dyb.ptr)
        ctx.check_error()
        y = dy.download(np.float32)
        yb = dyb.download(np.uint16)
        G, U, D = O.ExpertSource(H, I, seed).get(0, 0)
        ref = O.expert_slot(x, G, U, D)
        r = O.rel_to_scale(ref, y)
        worst = max(worst, r)
        assert np.array_equal(yb, synth.f32_to_bf16(y))
    print(f"config0 expert ffn: worst rel_to_scale over 8 seeds {worst:.3e}", flush=True)
    assert worst < TOL


@pytest.fixture(scope="module")
def glm_model(gpu):
    return DeviceModel(GLM, seed=1, n_layers=1)


@pytest.mark.parametrize("step", [0, 1, 2])
def test_layer_config1(gpu, glm_model, step):
    """Config 1: one full GLM MoE decode layer at the BASELINE shape."""
    hip = gpu
    dm = glm_model
    H = GLM["hidden"]
    h = synth.hidden_state(H, 100 + step)
    dh, dout = make_io(H)
    dh.upload(h)
    dm.ctx.run_moe(0, dh.ptr, dout.ptr)
    dm.ctx.check_error()
    out = dout.download(np.float32)
    got = _taps(dm, hip)
    ref = O.moe_layer(h, dm.dense[0], O.ExpertSource(H, GLM["moe_inter"], dm.seed), 0, GLM)
    margin = O.topk_margin(ref["choice"], GLM["n_experts_per_tok"])
    r = _check_layer(ref, got, out, f"step{step}")
    print(f"config1 step{step}: out rel_to_scale {r:.3e}, top-8 margin {margin:.3e}, ids {sorted(got['topk_idx'])}",
          flush=True)


def test_layer_config1_with_norm_weight(gpu):
    """The GLM-shape kernel with a post-attention norm weight (a separate
    kernel argument of its own) under both schedules."""
    hip = gpu
    H = GLM["hidden"]
    ln = [(1.0 + synth.bf16_to_f32(synth.normal_bf16(5, 0, synth.TAG_LN, (H,), 0.25))).astype(np.float32)]
    ln = [synth.f32_to_bf16(ln[0])]
    dm = DeviceModel(GLM, seed=2, n_layers=1, ln_weights=ln)
    h = synth.hidden_state(H, 321)
    ref = O.moe_layer(h, dm.dense[0], O.ExpertSource(H, GLM["moe_inter"], 2), 0, GLM,
                      ln_w=synth.bf16_to_f32(ln[0]))
    for sched in [moe.SCHED_FUSED, moe.SCHED_PHASED]:
        dm.ctx.set_schedule(sched)
        dh, dout = make_io(H)
        dh.upload(h)
        dm.ctx.run_moe(0, dh.ptr, dout.ptr)
        dm.ctx.check_error()
        r = _check_layer(ref, _taps(dm, hip), dout.download(np.float32), f"ln sched{sched}")
        print(f"config1 with norm weight, schedule {sched}: out rel_to_scale {r:.3e}", flush=True)
    dm.ctx.close()


def test_schedules_identical_and_stable(gpu, glm_model):
    hip = gpu
    dm = glm_model
    H = GLM["hidden"]
    dh, dout = make_io(H)
    dh.upload(synth.hidden_state(H, 7))
    outs = []
    for sched in [moe.SCHED_FUSED, moe.SCHED_PHASED, moe.SCHED_FUSED]:
        dm.ctx.set_schedule(sched)
        for _ in range(5):
            dm.ctx.run_moe(0, dh.ptr, dout.ptr)
        dm.ctx.check_error()
        outs.append(dout.download(np.float32))
    dm.ctx.set_schedule(moe.SCHED_FUSED)
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_two_level_combine(gpu, glm_model):
    """WL_DECODE_XL2=1: the partials are summed per XCD through that XCD's L2
    first (plain stores, non-temporal loads), then over the 8 XCDs. Checked
    against the oracle under both schedules (which must agree bit for bit)
    and against the default one-level combine (a different summation order:
    within the bar, not bit-equal)."""
    hip = gpu
    H = GLM["hidden"]
    os.environ["WL_DECODE_XL2"] = "1"
    try:
        dm = DeviceModel(GLM, seed=1, n_layers=1)
    finally:
        del os.environ["WL_DECODE_XL2"]
    try:
        for step in range(3):
            h = synth.hidden_state(H, 100 + step)
            ref = O.moe_layer(h, dm.dense[0], O.ExpertSource(H, GLM["moe_inter"], dm.seed), 0, GLM)
            outs = []
            for sched in [moe.SCHED_FUSED, moe.SCHED_PHASED]:
                dm.ctx.set_schedule(sched)
                dh, dout = make_io(H)
                dh.upload(h)
                dm.ctx.run_moe(0, dh.ptr, dout.ptr)
                dm.ctx.check_error()
                outs.append(dout.download(np.float32))
                r = _check_layer(ref, _taps(dm, hip), outs[-1], f"xl2 step{step} sched{sched}")
            assert np.array_equal(outs[0], outs[1]), step
            dh, dout = make_io(H)
            dh.upload(h)
            glm_model.ctx.run_moe(0, dh.ptr, dout.ptr)
            glm_model.ctx.check_error()
            one = dout.download(np.float32)
            d = O.rel_to_scale(one, outs[0])
            assert d < TOL, d
            print(f"two-level combine step {step}: out rel_to_scale {r:.3e}, vs one-level {d:.3e}", flush=True)
    finally:
        dm.close()


def _small():
    fx = np.load(os.path.join(GOLD, "moe_tf_small.npz"))
    return fx, json.loads(str(fx["config"])), [int(s) for s in fx["seeds"]]


def test_small_layer_vs_transformers_fixture(gpu):
    """The HIP layer against transformers' GlmMoeDsaMoE outputs (committed
    fixture), independently of this repository's oracle."""
    hip = gpu
    fx, c, seeds = _small()
    H = c["hidden"]
    for seed in seeds:
        dm = DeviceModel(c, seed=seed, n_layers=1)
        dh, dout = make_io(H)
        dh.upload(synth.hidden_state(H, seed))
        dm.ctx.run_moe(0, dh.ptr, dout.ptr)
        dm.ctx.check_error()
        out = dout.download(np.float32)
        got = _taps(dm, hip)
        p = f"s{seed}_"
        assert np.array_equal(np.sort(got["topk_idx"]), fx[p + "topk_idx_sorted"]), seed
        assert O.rel_to_scale(fx[p + "logits"], got["logits"]) < TOL
        assert O.rel_to_scale(fx[p + "topk_w_by_sorted_id"],
                              O.align_weights(fx[p + "topk_idx_sorted"], None, got["topk_idx"], got["topk_w"])) < TOL
        assert O.rel_to_scale(fx[p + "shared"], got["shared"]) < TOL
        assert O.rel_to_scale(fx[p + "out"], out) < TOL, seed
        dm.ctx.close()


@pytest.mark.parametrize("shape", [
    dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1),
    dict(hidden=1024, moe_inter=384, n_routed_experts=64, n_experts_per_tok=1, n_shared=2),
    dict(hidden=768, moe_inter=128, n_routed_experts=16, n_experts_per_tok=16, n_shared=1),
])
def test_generic_shapes(gpu, shape):
    hip = gpu
    c = dict(shape, routed_scaling=2.5, rms_eps=1e-5)
    H = c["hidden"]
    ln = [synth.normal_bf16(3, 0, synth.TAG_LN, (H,), 0.5)]
    dm = DeviceModel(c, seed=3, n_layers=1, ln_weights=ln)
    for sched in [moe.SCHED_FUSED, moe.SCHED_PHASED]:
        dm.ctx.set_schedule(sched)
        h = synth.hidden_state(H, 11)
        dh, dout = make_io(H)
        dh.upload(h)
        dm.ctx.run_moe(0, dh.ptr, dout.ptr)
        dm.ctx.check_error()
        out = dout.download(np.float32)
        got = _taps(dm, hip)
        ref = O.moe_layer(h, dm.dense[0], O.ExpertSource(H, c["moe_inter"], 3), 0, c,
                          ln_w=synth.bf16_to_f32(ln[0]))
        _check_layer(ref, got, out, str(shape))
    dm.ctx.close()


def test_partial_tags_over_consecutive_calls(gpu):
    """The combine takes a partial word as this call's only when its 2-bit
    tag matches, and the tag repeats every third call: eight back-to-back
    calls with a different hidden state each (both schedules, the shared tap
    on and off, two layers), nothing synchronised between them, each output
    against the oracle. A stale word accepted as fresh would carry another
    call's input."""
    c = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
    H, I = c["hidden"], c["moe_inter"]
    dm = DeviceModel(c, seed=5, n_layers=2)
    src = O.ExpertSource(H, I, 5)
    n = 8
    hs = [synth.hidden_state(H, 300 + i) for i in range(n)]
    dhs, douts = [], []
    for i in range(n):
        dh, dout = make_io(H)
        dh.upload(hs[i])
        dhs.append(dh)
        douts.append(dout)
    for i in range(n):
        dm.ctx.set_schedule(moe.SCHED_PHASED if i % 3 == 1 else moe.SCHED_FUSED)
        dm.ctx.set_taps(i % 2 == 0)
        dm.ctx.run_moe(i % 2, dhs[i].ptr, douts[i].ptr)
    dm.ctx.check_error()
    for i in range(n):
        ref = O.moe_layer(hs[i], dm.dense[i % 2], src, i % 2, c)["out"]
        r = O.rel_to_scale(ref, douts[i].download(np.float32))
        assert r < TOL, (i, r)
    dm.ctx.set_schedule(moe.SCHED_FUSED)
    dm.ctx.close()


def test_chain_residual(gpu):
    """h <- h + moe(h) over 3 layers, 2 steps (the MoE half of run_chain)."""
    hip = gpu
    fx, c, _ = _small()
    H, I = c["hidden"], c["moe_inter"]
    dm = DeviceModel(c, seed=9, n_layers=3)
    src = O.ExpertSource(H, I, 9)
    dh, dtmp = make_io(H)
    h = synth.hidden_state(H, 21)
    dh.upload(h)
    ref = h.copy()
    for step in range(2):
        dm.ctx.run_chain(0, 3, dh.ptr, dtmp.ptr)
        for l in range(3):
            ref = ref + O.moe_layer(ref, dm.dense[l], src, l, c)["out"]
    dm.ctx.check_error()
    got = dh.download(np.float32)
    assert O.rel_to_scale(ref, got) < TOL
    dm.ctx.close()


def test_not_resident_is_an_error_then_recovers(gpu):
    fx, c, _ = _small()
    H = c["hidden"]
    dm = DeviceModel(c, seed=1, n_layers=1)
    dm.ctx.slot_unbind(0, 5)
    dh, dout = make_io(H)
    with pytest.raises(moe.WindlassError) as ei:
        dm.ctx.run_moe(0, dh.ptr, dout.ptr)
    assert ei.value.status == 4
    T = 3
    do_b = H_.DeviceBuffer(4 * T * H)
    with pytest.raises(moe.WindlassError) as ei:
        dm.ctx.run_moe_batched(0, T, dh.ptr, None, do_b.ptr)
    assert ei.value.status == 4
    # the refusals leave the context usable: bind the expert again and both
    # schedules and the batched layer match the oracle
    dm.ctx.slot_bind(0, 5, dm.ctx.slot_pool_ptr(5))
    src = O.ExpertSource(H, c["moe_inter"], 1)
    hs = np.stack([synth.hidden_state(H, 410 + t) for t in range(T)]).astype(np.float32)
    refs = [O.moe_layer(hs[t], dm.dense[0], src, 0, c)["out"] for t in range(T)]
    for sched in (moe.SCHED_FUSED, moe.SCHED_PHASED):
        dm.ctx.set_schedule(sched)
        for t in range(T):
            dh.upload(hs[t])
            dm.ctx.run_moe(0, dh.ptr, dout.ptr)
            dm.ctx.check_error()
            assert O.rel_to_scale(refs[t], dout.download(np.float32)) < TOL, (sched, t)
    dm.ctx.set_schedule(moe.SCHED_FUSED)
    dhb = H_.DeviceBuffer.from_array(hs)
    dm.ctx.run_moe_batched(0, T, dhb.ptr, None, do_b.ptr)
    dm.ctx.check_error()
    outs = do_b.download(np.float32).reshape(T, H)
    for t in range(T):
        assert O.rel_to_scale(refs[t], outs[t]) < TOL, t
    dm.ctx.close()


@pytest.mark.parametrize("shape", [(256, 128), (384, 256), (6144, 2048), (2176, 2176)])
def test_native_layout(gpu, shape):
    """wl_synth_expert_native == wl_expert_to_native(wl_synth_expert block) ==
    the numpy restatement of the native layout (oracle/native_layout.py).
    (2176, 2176): 17 k tiles (a last group of one), 68 down row pairs (a last
    scale group of four) and 34 slices (a second slice group of two)."""
    from oracle import native_layout
    hip = gpu
    H, I = shape
    cfg = moe.make_config(hidden=H, moe_inter=I)
    lay = moe.expert_layout(cfg)
    nbytes = moe.native_block_bytes(cfg)
    assert nbytes == sum(native_layout.native_sizes(H, I))
    ref = hip.DeviceBuffer(lay.total)
    nat1, nat2 = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    moe.synth_expert(cfg, 5, 1, 7, ref.ptr)
    moe.expert_to_native(cfg, ref.ptr, nat1.ptr)
    moe.synth_expert_native(cfg, 5, 1, 7, nat2.ptr)
    hip.synchronize()
    a, b = nat1.download(np.uint8), nat2.download(np.uint8)
    assert np.array_equal(a, b)
    want = native_layout.to_native(synth.expert_block(H, I, 5, 1, 7), H, I)
    assert np.array_equal(a, want)
