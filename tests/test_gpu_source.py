"""The expert-source boundary on the GPU (run with -m gpu): the C form of
glm::ExpertSource (src/glm_layer_runner.cuh:34-48) behind wl_run_moe and
wl_run_moe_batched.

A layer whose experts come through a source must give exactly what the same
layer gives with every expert bound (the same kernels run on the same bytes),
with the reference's call pattern: run_moe announces the K routed experts
once and fetches each (:409-418); run_moe_batched fetches every unique expert
once, in chunks of at most 32 (:862-902). The built-in cache is one such
source."""
import numpy as np
import pytest

from oracle import synth
from windlass_amd import hip as H_
from windlass_amd import moe, synthdata
from windlass_amd.model import CachedModel, DeviceModel, SourceModel, make_io

pytestmark = pytest.mark.gpu
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)


def _decode(m, layer, h):
    dh, dout = make_io(h.shape[0])
    dh.upload(h)
    m.ctx.run_moe_residual(layer, dh.ptr, dh.ptr, dout.ptr)
    m.ctx.check_error()
    return dout.download(np.float32)


def _ids(m):
    K = m.cfg.n_experts_per_tok
    return H_.download_ptr(m.ctx.taps()["topk_idx"], np.int32, K)


def _batched(m, hs):
    T, H = hs.shape
    dh = H_.DeviceBuffer.from_array(hs)
    do = H_.DeviceBuffer(4 * T * H)
    m.ctx.run_moe_batched(0, T, dh.ptr, dh.ptr, do.ptr)
    m.ctx.check_error()
    return do.download(np.float32).reshape(T, H)


@pytest.mark.parametrize("shape,native", [("glm", True), ("small", True), ("small", False)])
def test_decode_through_source_equals_resident(gpu, shape, native):
    c = GLM if shape == "glm" else SMALL
    H, K, L = c["hidden"], c["n_experts_per_tok"], (1 if shape == "glm" else 3)
    zipf = synthdata.zipf_bias_offset(c["n_routed_experts"], 31, amplitude=0.25)
    dm = DeviceModel(c, seed=31, n_layers=L, bias_offset=zipf)
    sm = SourceModel(dm, native=native)
    for t in range(3):
        h = synth.hidden_state(H, 700 + t)
        for l in range(L):
            sm.calls.clear()
            got = _decode(sm, l, h)
            ref = _decode(dm, l, h)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (t, l)
            ids = _ids(sm)
            assert np.array_equal(ids, _ids(dm))
            # run_moe's pattern: one prefetch of the K ids, then one get_async per id, in slot order
            assert sm.calls == [("prefetch", l, tuple(int(i) for i in ids))] + \
                [("get_async", l, int(i)) for i in ids], sm.calls
            h = got
    sm.close()
    dm.close()


def test_get_only_source(gpu):
    """A source with get alone (prefetch and get_async NULL): get per id."""
    c = SMALL
    dm = DeviceModel(c, seed=32, n_layers=1)
    sm = SourceModel(dm, native=False, with_prefetch=False, with_async=False)
    h = synth.hidden_state(c["hidden"], 710)
    got = _decode(sm, 0, h)
    assert np.array_equal(got.view(np.uint32), _decode(dm, 0, h).view(np.uint32))
    assert sm.calls == [("get", 0, int(i)) for i in _ids(sm)]
    sm.close()
    dm.close()


def test_source_without_block_is_an_io_error(gpu):
    c = SMALL
    dm = DeviceModel(c, seed=33, n_layers=1)
    h = synth.hidden_state(c["hidden"], 720)
    _decode(dm, 0, h)
    first = int(_ids(dm)[0])
    sm = SourceModel(dm, native=True, missing=[(0, first)])
    with pytest.raises(moe.WindlassError) as ei:
        _decode(sm, 0, h)
    assert ei.value.status == 7  # WL_ERR_IO
    sm.close()
    dm.close()


@pytest.mark.parametrize("shape,native,T", [("small", True, 100), ("small", False, 100), ("glm", True, 256)])
def test_batched_through_source_equals_resident(gpu, shape, native, T):
    """Each unique expert fetched once, ascending, in chunks of at most 32
    (prefetch of the chunk, then get_async of each); output bit-identical to
    the resident layer."""
    c = GLM if shape == "glm" else SMALL
    zipf = synthdata.zipf_bias_offset(c["n_routed_experts"], 34, amplitude=0.25)
    dm = DeviceModel(c, seed=34, n_layers=1, bias_offset=zipf)
    sm = SourceModel(dm, native=native)
    hs = np.stack([synth.hidden_state(c["hidden"], 800, t) for t in range(T)]).astype(np.float32)
    got = _batched(sm, hs)
    ref = _batched(dm, hs)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    uniq = [int(e) for e in np.nonzero(dm.ctx.batched_counts())[0]]
    pre = [x[2] for x in sm.calls if x[0] == "prefetch"]
    fetched = [x[2] for x in sm.calls if x[0] == "get_async"]
    assert fetched == uniq and [e for ch in pre for e in ch] == uniq
    assert all(0 < len(ch) <= 32 for ch in pre) and len(pre) == -(-len(uniq) // 32)
    print(f"{shape} T={T}: {len(uniq)} experts in {len(pre)} chunks", flush=True)
    sm.close()
    dm.close()


def test_batched_through_cache_equals_resident(gpu):
    """The built-in cache as the batched layer's source: bit-identical to the
    resident layer, each unique expert requested once."""
    c = SMALL
    zipf = synthdata.zipf_bias_offset(c["n_routed_experts"], 35)
    cm = CachedModel(c, seed=35, n_layers=1, capacity=24, n_host=60, bias_offset=zipf)
    rm = DeviceModel(c, seed=35, n_layers=1, bias_offset=zipf, expert_key=cm.expert_source_key)
    hs = np.stack([synth.hidden_state(c["hidden"], 810, t) for t in range(40)]).astype(np.float32)
    got = _batched(cm, hs)
    ref = _batched(rm, hs)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    st = cm.ctx.cache_stats()
    n_uniq = int((rm.ctx.batched_counts() > 0).sum())
    assert st["hits"] + st["misses"] == n_uniq, (st, n_uniq)
    cm.close()
    rm.close()


def test_partly_bound_layer_is_not_resident(gpu):
    c = SMALL
    dm = DeviceModel(c, seed=36, n_layers=1)
    dm.ctx.slot_unbind(0, 5)
    h = synth.hidden_state(c["hidden"], 730)
    with pytest.raises(moe.WindlassError) as ei:
        _decode(dm, 0, h)
    assert ei.value.status == 4  # WL_ERR_NOT_RESIDENT
    dm.close()
