"""Routing over many inputs at the GLM shape (GPU; run with -m gpu): 256
hidden states through the decode layer with the router bias as generated,
and 256 with the bias skewed by the Zipf(s=1.1) offset the batched and cache
benches use. Each call's taps against the numpy oracle's router
(GlmMoeDsaTopkRouter, tools/ref_glm_chain.py:127-149; the reference's device
top-k order, src/glm_layer_runner.cuh:304-336): ids exact and in order,
logits and routing weights within 1e-5 rel_to_scale, the norm within 1e-5.
The smallest top-8 margin seen is printed: a flip needs a logit error larger
than it. Full layer outputs are compared on every 64th input (the oracle's
expert FFNs are the slow part)."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import synthdata
from windlass_amd.model import DeviceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)
N = 256


@pytest.mark.parametrize("skew", [False, True], ids=["bias", "zipf_bias"])
def test_routing_many_inputs_vs_oracle(gpu, skew):
    hip = gpu
    H, E, K, I = GLM["hidden"], GLM["n_routed_experts"], GLM["n_experts_per_tok"], GLM["moe_inter"]
    off = synthdata.zipf_bias_offset(E, 1, amplitude=0.25) if skew else None
    dm = DeviceModel(GLM, seed=4, n_layers=1, bias_offset=off)
    d = dm.dense[0]
    W = synth.bf16_to_f32(d["router_w"]).reshape(E, H)
    src = O.ExpertSource(H, I, 4)
    dh, dout = make_io(H)
    worst = {"norm": 0.0, "logits": 0.0, "topk_w": 0.0, "out": 0.0}
    min_margin = np.inf
    counts = np.zeros(E, np.int64)
    for t in range(N):
        h = synth.hidden_state(H, 5000 + 1000 * int(skew) + t)
        dh.upload(h)
        dm.ctx.run_moe(0, dh.ptr, dout.ptr)
        dm.ctx.check_error()
        taps = dm.ctx.taps()
        norm = hip.download_ptr(taps["norm"], np.float32, H)
        logits = hip.download_ptr(taps["logits"], np.float32, E)
        ids = hip.download_ptr(taps["topk_idx"], np.int32, K)
        w = hip.download_ptr(taps["topk_w"], np.float32, K)
        xn = O.rms_norm(h, None, GLM["rms_eps"])
        lg, rid, rw, choice = O.route(xn, W, d["bias"], K, GLM["routed_scaling"], True)
        min_margin = min(min_margin, O.topk_margin(choice, K))
        assert np.array_equal(ids, rid), (skew, t, ids, rid)
        for k, (ref, got) in {"norm": (xn, norm), "logits": (lg, logits), "topk_w": (rw, w)}.items():
            r = O.rel_to_scale(ref, got)
            worst[k] = max(worst[k], r)
            assert r < TOL, (skew, t, k, r)
        counts[rid] += 1
        if t % 64 == 0:
            ref = O.moe_layer(h, d, src, 0, GLM)
            r = O.rel_to_scale(ref["out"], dout.download(np.float32))
            worst["out"] = max(worst["out"], r)
            assert r < TOL, (skew, t, r)
    print(f"routing {'zipf' if skew else 'plain'} bias, {N} inputs: ids exact; worst rel_to_scale "
          + ", ".join(f"{k} {v:.2e}" for k, v in worst.items())
          + f"; smallest top-{K} margin {min_margin:.2e}; experts used {int((counts > 0).sum())}, "
          f"most popular {int(counts.max())} of {N}", flush=True)
    dm.ctx.close()
