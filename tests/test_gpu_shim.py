"""The drop-in shim on the GPU (run with -m gpu).

tests/shim/reference_caller is a C++ program written against the reference's
call surface: stand-in Config / LayerWeights / ExpertLayout / ExpertSource /
PrefillBufs types with the reference's fields, and the reference's call
sites, compiled against include/windlass_glm.hpp instead of the reference's
headers. It runs a model of one dense layer and three MoE layers from layer 0:
run_layer's MoE half (run_moe into s_acc, then residual_add; reference
src/glm_layer_runner.cuh:674-675) over every layer as run_chain loops
(:1065-1068), and the layer-major prefill's MoE half (dense layers per
position, the others through run_moe_batched; :985-999). Experts come through
an ExpertSource of reference-layout blocks on every call ("source"), or are
made resident on first use (windlass_glm::set_resident, "resident").

Every layer's output is checked against the oracle from the GPU's own input to
that layer: ids exact, block output within 1e-5 rel_to_scale (dense layers
against oracle/attention.dense_mlp, MoE layers against moe_oracle.moe_layer
with the MXFP4 shared expert dequantised)."""
import os
import subprocess

import numpy as np
import pytest

from oracle import attention as A
from oracle import moe_oracle as O
from windlass_amd import synthdata

pytestmark = pytest.mark.gpu
TOL = 1e-5
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "shim", "_build", "reference_caller")
CFG = dict(hidden=512, moe_inter=256, n_routed_experts=32, n_experts_per_tok=4, n_shared=1, routed_scaling=2.5,
           rms_eps=1e-5)
NL, DENSE_FIRST, DI, T, SEED = 4, 1, 1024, 5, 7
SHARED_KEY = 0xFFFF


def _model(d):
    """Writes the caller's inputs into d; returns the oracle's view of them."""
    H, E, I = CFG["hidden"], CFG["n_routed_experts"], CFG["moe_inter"]
    with open(os.path.join(d, "cfg.txt"), "w") as f:
        f.write(f"{NL} {DENSE_FIRST} {H} {I} {E} {CFG['n_experts_per_tok']} 1 {DI} {T} {SEED} "
                f"{CFG['rms_eps']} {CFG['routed_scaling']}\n")
    layers = []
    for l in range(NL):
        p = os.path.join(d, f"l{l}_")
        if l < DENSE_FIRST:
            w = synthdata.dense_mlp(H, DI, SEED, l)
            for k, name in (("post_ln", "ln"), ("gate", "gate"), ("up", "up"), ("down", "down")):
                w[k].tofile(p + name + ".bin")
            layers.append({"dense": synthdata.as_f32(w)})
        else:
            r = synthdata.router_only(H, E, SEED, l)
            ln = synthdata._norm_w(SEED, l, synthdata.TAG_LN, H)
            ln.tofile(p + "ln.bin")
            r["router_w"].tofile(p + "router.bin")
            r["bias"].tofile(p + "bias.bin")
            layers.append({"router": r, "ln": synthdata.bf16_to_f32(ln)})
    h0 = np.stack([synthdata.hidden_state(H, 300 + t) for t in range(T)]).astype(np.float32)
    h0.tofile(os.path.join(d, "h0.bin"))
    return layers, h0


def _run(d, mode):
    r = subprocess.run([BIN, d, mode], capture_output=True, text=True, timeout=300)
    print(r.stdout.strip(), r.stderr.strip()[-2000:], flush=True)
    assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
    H, K = CFG["hidden"], CFG["n_experts_per_tok"]
    out = np.fromfile(os.path.join(d, "out_decode.bin"), np.float32).reshape(NL, H)
    ids = np.fromfile(os.path.join(d, "ids_decode.bin"), np.int32).reshape(NL, K)
    pre = np.fromfile(os.path.join(d, "out_prefill.bin"), np.float32).reshape(NL, T, H)
    return out, ids, pre


def _layer_ref(layers, experts, shared, l, h_in):
    """(block output, ids or None) of layer l for input h_in."""
    L = layers[l]
    if "dense" in L:
        taps = {}
        A.dense_mlp(h_in, L["dense"], CFG, taps)
        return taps["mlp_out"], None
    ref = O.moe_layer(h_in, L["router"], experts, l, CFG, ln_w=L["ln"], shared_f32=shared.get(l, SHARED_KEY))
    return ref["out"], ref["topk_idx"]


@pytest.fixture(scope="module")
def shim_runs(gpu, tmp_path_factory):
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build()"
    d = str(tmp_path_factory.mktemp("shim"))
    layers, h0 = _model(d)
    runs = {}
    for mode in ("source", "resident"):
        print(f"shim caller, mode {mode}: {NL} layers ({DENSE_FIRST} dense), {T} prefill positions", flush=True)
        runs[mode] = _run(d, mode)
    return layers, h0, runs


def test_shim_decode_from_layer0_vs_oracle(shim_runs):
    layers, h0, runs = shim_runs
    H, I = CFG["hidden"], CFG["moe_inter"]
    experts = O.ExpertSource(H, I, SEED)
    shared = O.ExpertSource(H, I, SEED)  # n_shared = 1: the shared expert has the routed experts' shape
    out, ids, _ = runs["source"]
    worst = 0.0
    for l in range(NL):
        h_in = h0[0] if l == 0 else out[l - 1]
        y, ref_ids = _layer_ref(layers, experts, shared, l, h_in)
        if ref_ids is not None:
            assert np.array_equal(ids[l], ref_ids), (l, ids[l], ref_ids)
        r = O.rel_to_scale(y, out[l].astype(np.float64) - h_in)
        worst = max(worst, r)
        print(f"shim decode layer {l} ({'dense' if ref_ids is None else 'moe'}): rel_to_scale {r:.2e}", flush=True)
        assert r < TOL, (l, r)
    assert np.all(ids[:DENSE_FIRST] == -1)


def test_shim_resident_equals_source(shim_runs):
    _, _, runs = shim_runs
    for a, b in zip(runs["source"], runs["resident"]):
        assert np.array_equal(a, b)


def test_shim_prefill_vs_oracle(shim_runs):
    layers, h0, runs = shim_runs
    H, I = CFG["hidden"], CFG["moe_inter"]
    experts = O.ExpertSource(H, I, SEED)
    shared = O.ExpertSource(H, I, SEED)
    out, _, pre = runs["source"]
    worst = 0.0
    for l in range(NL):
        for t in range(T):
            h_in = h0[t] if l == 0 else pre[l - 1, t]
            y, _ = _layer_ref(layers, experts, shared, l, h_in)
            r = O.rel_to_scale(y, pre[l, t].astype(np.float64) - h_in)
            worst = max(worst, r)
            assert r < TOL, (l, t, r)
    print(f"shim prefill: {NL} layers x {T} positions, worst rel_to_scale {worst:.2e}", flush=True)
    # position 0 of the prefill saw the decode path's input: the dense layer
    # runs the same GEMV launches (same bits), the batched MoE layers stay
    # within the bar of the decode layers
    assert np.array_equal(pre[:DENSE_FIRST, 0], out[:DENSE_FIRST])
    assert O.rel_to_scale(out[-1], pre[-1, 0]) < TOL
