"""Routing edge cases on the GPU (run with -m gpu), against the numpy oracle
and the reference's tie rule (router_sigmoid_topk, src/glm_layer_runner.cuh:
304-336: equal biased scores go to the lowest expert id):

* exact ties: experts whose router rows and biases are identical have
  bit-equal scores; a tied pair inside the top-k comes out lowest id first,
  and a tie across the k-th place keeps the lower id and drops the higher;
* a zero hidden state: RMSNorm gives zeros, every logit is 0, the choice is
  the bias alone and the experts' outputs vanish, leaving the residual.

Both schedules, decode and batched (the batched layer must route each token
exactly as the decode layer does)."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import hip as H_, moe
from windlass_amd.model import DeviceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
C = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
         routed_scaling=2.5, rms_eps=1e-5)


def _set_router(dm, rw, bias):
    """New router rows and bias for layer 0 (device buffers and the oracle's copy)."""
    dm.bufs[0][0].upload(rw)
    dm.bufs[0][1].upload(bias)
    dm.dense[0]["router_w"] = rw
    dm.dense[0]["bias"] = bias


def _decode(dm, h, resid=None):
    H = h.shape[0]
    dh, dout = make_io(H)
    dh.upload(h)
    if resid is None:
        dm.ctx.run_moe(0, dh.ptr, dout.ptr)
    else:
        dr = H_.DeviceBuffer.from_array(resid)
        dm.ctx.run_moe_residual(0, dh.ptr, dr.ptr, dout.ptr)
    dm.ctx.check_error()
    t = dm.ctx.taps()
    ids = H_.download_ptr(t["topk_idx"], np.int32, C["n_experts_per_tok"])
    return dout.download(np.float32), ids


def test_exact_ties_take_the_lowest_id(gpu):
    H, E, K = C["hidden"], C["n_routed_experts"], C["n_experts_per_tok"]
    dm = DeviceModel(C, seed=31, n_layers=1)
    src = O.ExpertSource(H, C["moe_inter"], 31)
    rw = dm.dense[0]["router_w"].copy()
    bias = dm.dense[0]["bias"].copy()
    # inside the top-k: experts 7 and 30 identical and far ahead of the rest
    rw[30] = rw[7]
    bias[7] = bias[30] = 40.0
    # across the k-th place: 2 more clear winners, then 11 < 25 < 41 tied for
    # the last two places (K = 6) -> 11 and 25 kept, 41 dropped
    for e in (2, 3):
        bias[e] = 20.0
    rw[25] = rw[11]
    rw[41] = rw[11]
    bias[11] = bias[25] = bias[41] = 10.0
    _set_router(dm, rw, bias)
    hs = [synth.hidden_state(H, 3100 + i) for i in range(4)]
    for sched in (moe.SCHED_FUSED, moe.SCHED_PHASED):
        dm.ctx.set_schedule(sched)
        for h in hs:
            out, ids = _decode(dm, h)
            ref = O.moe_layer(h, dm.dense[0], src, 0, C)
            assert np.array_equal(ids, ref["topk_idx"]), (sched, ids, ref["topk_idx"])
            assert list(ids[:2]) == [7, 30]
            assert 11 in ids and 25 in ids and 41 not in ids
            assert list(ids).index(11) < list(ids).index(25)
            assert O.rel_to_scale(ref["out"], out) < TOL
    # the batched layer routes each token exactly as the decode layer
    dm.ctx.set_schedule(moe.SCHED_FUSED)
    T = len(hs)
    dh = H_.DeviceBuffer.from_array(np.stack(hs).astype(np.float32))
    do = H_.DeviceBuffer(4 * T * H)
    dm.ctx.run_moe_batched(0, T, dh.ptr, None, do.ptr)
    dm.ctx.check_error()
    _, ids_b, _ = dm.ctx.batched_routing(T)
    outs = do.download(np.float32).reshape(T, H)
    for t, h in enumerate(hs):
        out, ids = _decode(dm, h)
        assert np.array_equal(ids_b[t], ids), t
        assert O.rel_to_scale(out, outs[t]) < TOL, t
    dm.ctx.close()


def test_zero_hidden_state(gpu):
    H, E, K = C["hidden"], C["n_routed_experts"], C["n_experts_per_tok"]
    dm = DeviceModel(C, seed=32, n_layers=1)
    src = O.ExpertSource(H, C["moe_inter"], 32)
    h = np.zeros(H, np.float32)
    resid = synth.hidden_state(H, 3200)
    for sched in (moe.SCHED_FUSED, moe.SCHED_PHASED):
        dm.ctx.set_schedule(sched)
        out, ids = _decode(dm, h, resid)
        ref = O.moe_layer(h, dm.dense[0], src, 0, C)
        assert np.array_equal(ids, ref["topk_idx"]), sched
        # the choice is the bias alone: its K largest, ties to the lowest id
        order = np.lexsort((np.arange(E), -dm.dense[0]["bias"].astype(np.float64)))[:K]
        assert np.array_equal(np.sort(ids), np.sort(order))
        assert np.array_equal(out, resid), sched  # zero experts' outputs, the residual unchanged
    dm.ctx.close()
