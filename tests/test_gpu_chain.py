"""Config 2 at full size (GPU; run with -m gpu): 24 resident GLM MoE layers
(6144 MXFP4 expert blocks, 123 GB of HBM) chained through wl_run_chain,
h <- h + moe(h) per layer (the MoE half of run_chain's layer loop, reference
src/glm_layer_runner.cuh:1065-1068).

The oracle is too slow to run 24 full layers per check, so the chain is pinned
at its two ends: the first layer from the seeded start state, and the last
layer from the GPU's own 23-layer state (both against the numpy oracle, same
1e-5 rel_to_scale bar as config 1, ids exact), plus chain splitting and
run-to-run identity over all 24 layers."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd.model import DeviceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)
NL = 24


@pytest.fixture(scope="module")
def chain_model(gpu):
    print(f"building {NL} resident GLM layers", flush=True)
    dm = DeviceModel(GLM, seed=2, n_layers=NL)
    yield dm
    dm.close()


def _run(dm, h0, first, n, dh=None, dtmp=None):
    H = GLM["hidden"]
    if dh is None:
        dh, dtmp = make_io(H)
        dh.upload(h0)
    dm.ctx.run_chain(first, n, dh.ptr, dtmp.ptr)
    dm.ctx.check_error()
    return dh.download(np.float32), dh, dtmp


def test_chain24_ends_vs_oracle(gpu, chain_model):
    hip = gpu
    dm = chain_model
    H, I, K = GLM["hidden"], GLM["moe_inter"], GLM["n_experts_per_tok"]
    src = O.ExpertSource(H, I, dm.seed)
    h0 = synth.hidden_state(H, 31)

    h1, _, _ = _run(dm, h0, 0, 1)
    ref0 = O.moe_layer(h0, dm.dense[0], src, 0, GLM)
    r0 = O.rel_to_scale(ref0["out"], h1 - h0)
    print(f"chain layer 0: rel_to_scale {r0:.3e}", flush=True)
    assert r0 < TOL

    h23, _, _ = _run(dm, h0, 0, NL - 1)
    h24, _, _ = _run(dm, h0, 0, NL)
    idx = hip.download_ptr(dm.ctx.taps()["topk_idx"], np.int32, K)  # taps: the chain's last layer
    ref = O.moe_layer(h23, dm.dense[NL - 1], src, NL - 1, GLM)
    assert np.array_equal(idx, ref["topk_idx"]), (idx, ref["topk_idx"])
    r = O.rel_to_scale(ref["out"], h24 - h23)
    print(f"chain layer {NL - 1} (from the GPU's 23-layer state): rel_to_scale {r:.3e}, "
          f"|h| max {np.abs(h23).max():.2f}, |moe| max {np.abs(ref['out']).max():.2f}", flush=True)
    assert r < TOL


def test_chain24_split_and_repeat_identical(gpu, chain_model):
    dm = chain_model
    h0 = synth.hidden_state(GLM["hidden"], 32)
    a, _, _ = _run(dm, h0, 0, NL)
    b, _, _ = _run(dm, h0, 0, NL)
    part, dh, dtmp = _run(dm, h0, 0, 10)
    c, _, _ = _run(dm, None, 10, NL - 10, dh, dtmp)
    assert np.all(np.isfinite(a))
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_chain24_one_launch_equals_per_layer_launches(gpu, chain_model):
    """Under the fused schedule wl_run_chain runs all 24 resident layers in one
    launch (each layer's output handed to the next as tagged words); under
    the phased schedule it launches every layer on its own. Same arithmetic,
    so the results must match bit for bit."""
    from windlass_amd import moe
    dm = chain_model
    h0 = synth.hidden_state(GLM["hidden"], 33)
    dm.ctx.set_schedule(moe.SCHED_PHASED)
    try:
        a, _, _ = _run(dm, h0, 0, NL)
    finally:
        dm.ctx.set_schedule(moe.SCHED_FUSED)
    b, _, _ = _run(dm, h0, 0, NL)
    assert np.all(np.isfinite(a))
    assert np.array_equal(a, b)
