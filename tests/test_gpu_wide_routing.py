"""Routing wider than the GLM shape (GPU; run with -m gpu): more than 256
experts, where the decode kernel ranks the choices instead of running its
one-wave argmax, more than 512, where the bias and slot loads take a second
pass over the threads, and the largest top-k the reference allows
(MAX_TOPK = 32, src/glm_loader.cuh:86); also the widest hidden state (8192)
with 16 shared experts and the weights neither renormalised nor scaled
(norm_topk_prob false, routed_scaling 1). The decode layer (both schedules)
against the numpy oracle: ids exact, in order, and every tap and the output
within 1e-5 rel_to_scale; the batched layer (up to its 816-expert limit)
against the decode layer, routing bit for bit (reference router_sigmoid_topk, src/glm_layer_runner.cuh:304-336,
and run_moe_batched, :818-928)."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import hip as H_, moe
from windlass_amd.model import DeviceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
SHAPES = [
    dict(hidden=1024, moe_inter=256, n_routed_experts=384, n_experts_per_tok=8, n_shared=1),
    dict(hidden=768, moe_inter=128, n_routed_experts=1024, n_experts_per_tok=12, n_shared=2),
    dict(hidden=512, moe_inter=128, n_routed_experts=4096, n_experts_per_tok=32, n_shared=1),
    # the widest hidden state, 16 shared experts, weights not renormalised, no scaling
    dict(hidden=8192, moe_inter=128, n_routed_experts=64, n_experts_per_tok=4, n_shared=16,
         norm_topk_prob=False, routed_scaling=1.0),
]


def _taps(dm):
    t = dm.ctx.taps()
    c = dm.c
    H, E, K, I = c["hidden"], c["n_routed_experts"], c["n_experts_per_tok"], c["moe_inter"]
    return {"norm": H_.download_ptr(t["norm"], np.float32, H),
            "logits": H_.download_ptr(t["logits"], np.float32, E),
            "topk_idx": H_.download_ptr(t["topk_idx"], np.int32, K),
            "topk_w": H_.download_ptr(t["topk_w"], np.float32, K),
            "mid": H_.download_ptr(t["mid"], np.float32, K * I).reshape(K, I),
            "shared": H_.download_ptr(t["shared"], np.float32, H)}


@pytest.mark.parametrize("shape", SHAPES,
                         ids=lambda s: f"H{s['hidden']}_E{s['n_routed_experts']}_K{s['n_experts_per_tok']}")
def test_wide_routing_decode_vs_oracle_and_batched_vs_decode(gpu, shape):
    c = dict(dict(routed_scaling=2.5, rms_eps=1e-5), **shape)
    H, I, K = c["hidden"], c["moe_inter"], c["n_experts_per_tok"]
    dm = DeviceModel(c, seed=21, n_layers=1)
    src = O.ExpertSource(H, I, 21)
    T = 9
    hs = np.stack([synth.hidden_state(H, 2100, t) for t in range(T)]).astype(np.float32)
    decoded, routing = [], []
    for t in range(T):
        for sched in ([moe.SCHED_FUSED, moe.SCHED_PHASED] if t < 2 else [moe.SCHED_FUSED]):
            dm.ctx.set_schedule(sched)
            dh, dout = make_io(H)
            dh.upload(hs[t])
            dm.ctx.run_moe(0, dh.ptr, dout.ptr)
            dm.ctx.check_error()
            out = dout.download(np.float32)
            got = _taps(dm)
            if t < 2:
                ref = O.moe_layer(hs[t], dm.dense[0], src, 0, c)
                tag = (str(shape), t, sched)
                assert np.array_equal(ref["topk_idx"], got["topk_idx"]), (tag, ref["topk_idx"], got["topk_idx"])
                assert O.rel_to_scale(ref["norm"], got["norm"]) < TOL, tag
                assert O.rel_to_scale(ref["logits"], got["logits"]) < TOL, tag
                assert O.rel_to_scale(ref["topk_w"], got["topk_w"]) < TOL, tag
                assert O.rel_to_scale(ref["mid"], got["mid"]) < TOL, tag
                assert O.rel_to_scale(ref["shared"], got["shared"]) < TOL, tag
                assert O.rel_to_scale(ref["out"], out) < TOL, tag
        decoded.append(out)
        routing.append((got["logits"], got["topk_idx"], got["topk_w"]))
    dm.ctx.set_schedule(moe.SCHED_FUSED)
    # the batched layer over the same tokens (at most 816 experts: its GEMM
    # kernels keep the expert tables in LDS; wider configs are refused)
    dh = H_.DeviceBuffer.from_array(hs)
    do = H_.DeviceBuffer(4 * T * H)
    if c["n_routed_experts"] > 816:
        with pytest.raises(moe.WindlassError) as ei:
            dm.ctx.run_moe_batched(0, T, dh.ptr, None, do.ptr)
        assert ei.value.status == 1  # WL_ERR_INVALID
        dm.ctx.close()
        return
    dm.ctx.run_moe_batched(0, T, dh.ptr, None, do.ptr)
    dm.ctx.check_error()
    outs = do.download(np.float32).reshape(T, H)
    lg, ids, w = dm.ctx.batched_routing(T)
    for t in range(T):
        assert np.array_equal(lg[t].view(np.uint32), routing[t][0].view(np.uint32)), t
        assert np.array_equal(ids[t], routing[t][1]), t
        assert np.array_equal(w[t].view(np.uint32), routing[t][2].view(np.uint32)), t
        assert O.rel_to_scale(decoded[t], outs[t]) < TOL, t
    dm.ctx.close()
