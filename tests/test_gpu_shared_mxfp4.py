"""The MXFP4 shared expert on the GPU (run with -m gpu): the reference keeps
its shared expert in MXFP4 (src/glm_loader.cuh:271-273,608-610) and runs it
through dequant_matvec_mxfp4 (src/glm_layer_runner.cuh:431-436).

The decode layer and the batched layer with an MXFP4 shared expert must match
the oracle (whose shared expert is the dequantised block) within 1e-5, the
batched layer must match the decode layer per token, and the two ways of
handing the shared expert over (one packed block, or the six tensors of
LayerWeights) must give the same bits."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import hip as H_
from windlass_amd import moe, synthdata
from windlass_amd.model import DeviceModel, SourceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)


def _decode(dm, h, layer=0):
    dh, dout = make_io(h.shape[0])
    dh.upload(h)
    dm.ctx.run_moe(layer, dh.ptr, dout.ptr)
    dm.ctx.check_error()
    return dout.download(np.float32)


def _shared_f32(dm, src, layer=0):
    return src.get(*dm.shared_key(layer))


@pytest.mark.parametrize("shape", ["small", "glm"])
def test_decode_mxfp4_shared_vs_oracle(gpu, shape):
    c = GLM if shape == "glm" else SMALL
    H, I, K = c["hidden"], c["moe_inter"], c["n_experts_per_tok"]
    dm = DeviceModel(c, seed=41, n_layers=1, shared_mxfp4=True)
    src = O.ExpertSource(H, I, 41)
    sh = _shared_f32(dm, src)
    worst = 0.0
    for sched in (moe.SCHED_FUSED, moe.SCHED_PHASED):
        dm.ctx.set_schedule(sched)
        outs = []
        for t in range(3):
            h = synth.hidden_state(H, 900 + t)
            out = _decode(dm, h)
            outs.append(out)
            ref = O.moe_layer(h, dm.dense[0], src, 0, c, shared_f32=sh)
            tp = dm.ctx.taps()
            ids = H_.download_ptr(tp["topk_idx"], np.int32, K)
            assert np.array_equal(ids, ref["topk_idx"])
            assert O.rel_to_scale(ref["shared"], H_.download_ptr(tp["shared"], np.float32, H)) < TOL
            r = O.rel_to_scale(ref["out"], out)
            worst = max(worst, r)
            assert r < TOL, (sched, t, r)
        if sched == moe.SCHED_FUSED:
            fused = outs
        else:
            for a, b in zip(fused, outs):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    print(f"{shape}: MXFP4 shared decode worst rel_to_scale {worst:.2e}", flush=True)
    dm.close()


def test_six_tensor_form_equals_packed_block(gpu):
    """wl_set_layer_mxfp4 (LayerWeights' six tensors) == wl_set_layer with the
    packed block, bit for bit."""
    c = SMALL
    H = c["hidden"]
    dm = DeviceModel(c, seed=42, n_layers=1, shared_mxfp4=True)
    h = synth.hidden_state(H, 910)
    packed = _decode(dm, h)
    lay = moe.expert_layout(dm.cfg, dm.SI)
    rw, bb, sb, _ = dm.bufs[0]
    p = sb.ptr
    dm.ctx.set_layer_mxfp4(0, rw.ptr, bb.ptr, None, p + lay.gw_off, p + lay.gs_off, p + lay.uw_off, p + lay.us_off,
                           p + lay.dw_off, p + lay.ds_off)
    six = _decode(dm, h)
    assert np.array_equal(packed.view(np.uint32), six.view(np.uint32))
    dm.close()


@pytest.mark.parametrize("shape,T", [("small", 70), ("glm", 64)])
def test_batched_mxfp4_shared(gpu, shape, T):
    c = GLM if shape == "glm" else SMALL
    H, I, E, K = c["hidden"], c["moe_inter"], c["n_routed_experts"], c["n_experts_per_tok"]
    zipf = synthdata.zipf_bias_offset(E, 43, amplitude=0.25)
    dm = DeviceModel(c, seed=43, n_layers=1, bias_offset=zipf, shared_mxfp4=True)
    hs = np.stack([synth.hidden_state(H, 920, t) for t in range(T)]).astype(np.float32)
    dh = H_.DeviceBuffer.from_array(hs)
    do = H_.DeviceBuffer(4 * T * H)
    dm.ctx.run_moe_batched(0, T, dh.ptr, None, do.ptr)
    dm.ctx.check_error()
    out = do.download(np.float32).reshape(T, H)
    lg, ids, w = dm.ctx.batched_routing(T)
    worst = 0.0
    for t in range(T):
        dec = _decode(dm, hs[t])
        assert np.array_equal(ids[t], H_.download_ptr(dm.ctx.taps()["topk_idx"], np.int32, K)), t
        r = O.rel_to_scale(dec, out[t])
        worst = max(worst, r)
        assert r < TOL, (t, r)
    src = O.ExpertSource(H, I, 43, cache=24)
    sh = _shared_f32(dm, src)
    for t in [0, T // 2, T - 1]:
        ref = O.moe_layer(hs[t], dm.dense[0], src, 0, c, shared_f32=sh)
        assert O.rel_to_scale(ref["out"], out[t]) < TOL, t
    # through an expert source, the shared expert runs with the first chunk only
    sm = SourceModel(dm, native=True)
    do2 = H_.DeviceBuffer(4 * T * H)
    sm.ctx.run_moe_batched(0, T, dh.ptr, None, do2.ptr)
    sm.ctx.check_error()
    assert np.array_equal(do2.download(np.float32).view(np.uint32), out.reshape(-1).view(np.uint32))
    print(f"{shape} T={T}: MXFP4 shared batched worst vs decode {worst:.2e}", flush=True)
    sm.close()
    dm.close()


def test_mxfp4_shared_needs_one_shared_expert(gpu):
    c = dict(SMALL, n_shared=2)
    cfg = moe.make_config(hidden=c["hidden"], moe_inter=c["moe_inter"], n_routed_experts=c["n_routed_experts"],
                          n_experts_per_tok=c["n_experts_per_tok"], n_shared=2)
    ctx = moe.Context(cfg)
    buf = H_.DeviceBuffer(1 << 20)
    with pytest.raises(moe.WindlassError) as ei:
        ctx.set_layer(0, buf.ptr, buf.ptr, None, buf.ptr, moe.SHARED_MXFP4)
    assert ei.value.status == 1
    ctx.close()
