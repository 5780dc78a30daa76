"""The allocation-free batched layer (wl_run_moe_batched_noalloc) against the
allocating one (wl_run_moe_batched), through the C ABI (GPU; -m gpu).

Both run the same kernels; the allocation-free one takes its scratch from the
library's static 64 MiB device array and runs at most 169 GLM tokens per chunk.
Two calls in a row, the second smaller, at a small shape and at the GLM shape;
the GLM call of 200 tokens runs as two chunks (169 + 31)."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import hip as H_
from windlass_amd import moe, synthdata
from windlass_amd.model import DeviceModel

pytestmark = pytest.mark.gpu
TOL = 1e-5
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)
GLM_CHUNK = 169


def _tokens(H, T, seed):
    return np.stack([synth.hidden_state(H, seed, t) for t in range(T)]).astype(np.float32)


def _run(dm, hs, resid, noalloc, t0=0, t1=None):
    t1 = hs.shape[0] if t1 is None else t1
    T, H = t1 - t0, hs.shape[1]
    dh = H_.DeviceBuffer.from_array(np.ascontiguousarray(hs[t0:t1]))
    dr = H_.DeviceBuffer.from_array(np.ascontiguousarray(resid[t0:t1])) if resid is not None else None
    do = H_.DeviceBuffer(4 * T * H)
    fn = dm.ctx.run_moe_batched_noalloc if noalloc else dm.ctx.run_moe_batched
    fn(0, T, dh.ptr, dr.ptr if dr else None, do.ptr)
    dm.ctx.check_error()
    return do.download(np.float32).reshape(T, H)


@pytest.mark.parametrize("shape", ["small", "glm"])
def test_noalloc_matches_batched(gpu, shape):
    c = SMALL if shape == "small" else GLM
    H = c["hidden"]
    off = synthdata.zipf_bias_offset(c["n_routed_experts"], 21, amplitude=0.25) if shape == "glm" else None
    dm = DeviceModel(c, seed=21, n_layers=1, bias_offset=off)
    sizes = [70, 5] if shape == "small" else [200, 20]
    for call, T in enumerate(sizes):
        print(f"noalloc {shape}: call {call}, T={T}", flush=True)
        hs = _tokens(H, T, 900 + 10 * call)
        resid = _tokens(H, T, 901 + 10 * call) if call == 0 else None
        got = _run(dm, hs, resid, noalloc=True)
        if shape == "glm" and T > GLM_CHUNK:
            # the same chunks through the allocating path: bit for bit
            ref = np.concatenate([_run(dm, hs, resid, False, 0, GLM_CHUNK), _run(dm, hs, resid, False, GLM_CHUNK, T)])
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
            # one chunk through the allocating path: passes of other sizes, same bar
            whole = _run(dm, hs, resid, False)
            worst = max(O.rel_to_scale(whole[t], got[t]) for t in range(T))
            assert worst < TOL, worst
        else:
            ref = _run(dm, hs, resid, False)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    dm.close()


def test_noalloc_allocates_nothing_and_replays_from_a_graph(gpu):
    """The resident path of the allocation-free entry point: device free
    memory is unchanged across a call; captured into a HIP graph on a stream,
    it replays to the eager call's bits three times, with eager work of the
    program (an allocating batched call on other tokens, a buffer clear,
    synchronisations) between the replays. A source-backed layer refuses to
    run under capture."""
    from windlass_amd.model import SourceModel
    c = SMALL
    H = c["hidden"]
    dm = DeviceModel(c, seed=22, n_layers=1)
    T = 40
    hs = _tokens(H, T, 950)
    dh = H_.DeviceBuffer.from_array(hs)
    do = H_.DeviceBuffer(4 * T * H)
    other = H_.DeviceBuffer.from_array(_tokens(H, 9, 951))
    other_out = H_.DeviceBuffer(4 * 9 * H)
    st = H_.Stream()
    # scratch of the allocating path grown beforehand, so later eager calls allocate nothing either
    dm.ctx.run_moe_batched(0, 9, other.ptr, None, other_out.ptr, st.handle)
    st.synchronize()
    free0, _ = H_.mem_info()
    dm.ctx.run_moe_batched_noalloc(0, T, dh.ptr, None, do.ptr, st.handle)
    dm.ctx.check_error(st.handle)
    assert H_.mem_info()[0] == free0
    eager = do.download(np.float32)
    g = H_.Graph(st)
    g.begin()
    dm.ctx.run_moe_batched_noalloc(0, T, dh.ptr, None, do.ptr, st.handle)
    g.end()
    try:
        for rep in range(3):
            do.zero()
            H_.synchronize()
            g.launch()
            st.synchronize()
            got = do.download(np.float32)
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), rep
            dm.ctx.run_moe_batched(0, 9, other.ptr, None, other_out.ptr, st.handle)
            dm.ctx.check_error(st.handle)
        print("noalloc graph: 3 replays bit-equal to the eager call", flush=True)
    finally:
        g.destroy()
    sm = SourceModel(dm, native=True)
    g2 = H_.Graph(st)
    g2.begin()
    with pytest.raises(moe.WindlassError) as ei:
        sm.ctx.run_moe_batched_noalloc(0, T, dh.ptr, None, do.ptr, st.handle)
    g2.end()
    g2.destroy()
    assert ei.value.status == 5  # WL_ERR_STATE
    sm.close()
    dm.close()
