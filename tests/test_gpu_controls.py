"""Negative controls re-run against the HIP path (GPU; run with -m gpu).

The parity gate (ids as a set, outputs within 1e-5 rel_to_scale) is only
evidence if it fails on the plausible mistakes: each test below runs the HIP
layer once, checks it against the correct oracle, then against the oracle
with one mistake planted (on the CPU, never in the product) and asserts that
the gate separates them by orders of magnitude. The mistakes are the MoE
controls of the reference (docs/RESULTS.md:42-54; tools/check_ref_vs_oracle.py:
473-485,506-519; tools/dump_glm_oracle.py:123-136): nibble order flipped,
routed_scaling_factor 1.0, weights gathered from the biased score, the
correction bias cast to bf16; plus an E8M0 exponent bias off by one and a
dropped shared expert (a small term here: caught with less margin)."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd.model import DeviceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
C = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
         routed_scaling=2.5, rms_eps=1e-5)
SEED = 4


class _Flipped(O.ExpertSource):
    """High nibble = even column (the reference layout is low nibble first)."""

    def get(self, layer, expert):
        key = ("flip", layer, expert)
        if key not in self._cache:
            gw, gs, uw, us, dw, ds = synth.expert_block(self.H, self.I, self.seed, layer, expert)
            swap = lambda w: ((w >> 4) | (w << 4)).astype(np.uint8)
            self._cache[key] = (O.dequant(swap(gw), gs), O.dequant(swap(uw), us), O.dequant(swap(dw), ds))
        return self._cache[key]


class _ScaleOffByOne(O.ExpertSource):
    """E8M0 read as 2^(s-126) instead of 2^(s-127)."""

    def get(self, layer, expert):
        G, U, D = super().get(layer, expert)
        return G * 2, U * 2, D * 2


def _run(bias_offset=None):
    H = C["hidden"]
    dm = DeviceModel(C, seed=SEED, n_layers=1, bias_offset=bias_offset)
    h = synth.hidden_state(H, 77)
    dh, dout = make_io(H)
    dh.upload(h)
    dm.ctx.run_moe(0, dh.ptr, dout.ptr)
    dm.ctx.check_error()
    out = dout.download(np.float32)
    from windlass_amd import hip
    idx = hip.download_ptr(dm.ctx.taps()["topk_idx"], np.int32, C["n_experts_per_tok"])
    dense = dm.dense[0]
    dm.ctx.close()
    return h, dense, out, idx


def test_gate_separates_planted_mistakes(gpu):
    H, I = C["hidden"], C["moe_inter"]
    h, dense, out, idx = _run()
    src = O.ExpertSource(H, I, SEED)
    ref = O.moe_layer(h, dense, src, 0, C)
    good = O.rel_to_scale(ref["out"], out)
    assert good < TOL
    assert np.array_equal(np.sort(ref["topk_idx"]), np.sort(idx))
    bad = {
        "nibble order flipped": O.moe_layer(h, dense, _Flipped(H, I, SEED), 0, C)["out"],
        "routed_scaling 1.0": O.moe_layer(h, dense, src, 0, dict(C, routed_scaling=1.0))["out"],
        "E8M0 bias off by one": O.moe_layer(h, dense, _ScaleOffByOne(H, I, SEED), 0, C)["out"],
    }
    # weights gathered from the biased score (the selection itself is right)
    s = 1.0 / (1.0 + np.exp(-ref["logits"].astype(np.float64)))
    wb = (s + dense["bias"])[ref["topk_idx"]]
    wb = (wb / wb.sum() * C["routed_scaling"]).astype(np.float32)
    bad["weights from the biased score"] = O.moe_finish(wb, ref["slot_outs"], ref["shared"])
    for name, b in bad.items():
        r = O.rel_to_scale(b, out)
        assert r > 1e3 * good and r > 1e-3, (name, r, good)
    # The synthetic shared expert (weights N(0, 0.02)) is a small term: left
    # out, the output moves by about 2.5e-5 of its scale (measured on the
    # oracle). The gate still fails on it; the shared-output tap is compared
    # on its own in test_gpu_decode.py.
    r = O.rel_to_scale(ref["out"] - ref["shared"], out)
    assert r > 2 * TOL and r > 10 * good, ("shared expert dropped", r, good)


def test_bias_cast_to_bf16_changes_the_selection(gpu):
    """With a checkpoint-like correction bias (about 34 +- 0.138,
    tools/dump_glm_oracle.py:123-127) a bf16 bias collapses the selection: the
    HIP ids match the f32-bias oracle and not the bf16-bias one."""
    H, I, E = C["hidden"], C["moe_inter"], C["n_routed_experts"]
    rng = np.random.default_rng(12)
    offset = (34.0 + 0.138 * rng.standard_normal(E)).astype(np.float32)
    h, dense, out, idx = _run(bias_offset=offset)
    src = O.ExpertSource(H, I, SEED)
    ref = O.moe_layer(h, dense, src, 0, C)
    assert np.array_equal(np.sort(ref["topk_idx"]), np.sort(idx))
    assert O.rel_to_scale(ref["out"], out) < TOL
    d16 = dict(dense, bias=synth.bf16_to_f32(synth.f32_to_bf16(dense["bias"])))
    bad = O.moe_layer(h, d16, src, 0, C)
    assert set(bad["topk_idx"].tolist()) != set(idx.tolist())
    assert O.rel_to_scale(bad["out"], out) > 1e-2


def test_decode_layer_refuses_graph_capture(gpu):
    """A MoE decode launch carries a new call epoch and partial tag from the
    host, so a replayed capture could read an earlier call's logits or
    partials as its own: under capture wl_run_moe, wl_run_moe_residual and
    wl_run_chain return WL_ERR_STATE, enqueue nothing, and the context works
    normally afterwards."""
    from windlass_amd import hip as H_, moe
    c = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
    H = c["hidden"]
    dm = DeviceModel(c, seed=3, n_layers=2)
    try:
        h = synth.hidden_state(H, 44)
        dh, dout = make_io(H)
        dh.upload(h)
        st = H_.Stream()
        for call in ("run_moe", "run_moe_residual", "run_chain"):
            g = H_.Graph(st)
            g.begin()
            with pytest.raises(moe.WindlassError) as ei:
                if call == "run_moe":
                    dm.ctx.run_moe(0, dh.ptr, dout.ptr, st.handle)
                elif call == "run_moe_residual":
                    dm.ctx.run_moe_residual(0, dh.ptr, dh.ptr, dout.ptr, st.handle)
                else:
                    dm.ctx.run_chain(0, 2, dout.ptr, dh.ptr, st.handle)
            g.end()
            g.destroy()
            assert ei.value.status == 5, call  # WL_ERR_STATE
        dh.upload(h)
        dm.ctx.run_moe(0, dh.ptr, dout.ptr, st.handle)
        dm.ctx.check_error(st.handle)
        ref = O.moe_layer(h, dm.dense[0], O.ExpertSource(H, c["moe_inter"], 3), 0, c)
        assert O.rel_to_scale(ref["out"], dout.download(np.float32)) < 1e-5
    finally:
        dm.close()
