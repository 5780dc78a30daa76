"""The HBM expert cache (config 4's mechanism) on the GPU (run with -m gpu).

A cache-backed layer must give exactly what the same layer gives with every
expert resident (both run the same decode kernel on the same bytes), its
routing must match the oracle, and its counters must equal a replay of the
requested ids through the LRU oracle (reference semantics,
src/glm_expert_cache.cuh:198-308). The prefetch/get path repeats the
reference's case 4 (src/test_glm_expert_cache.cu:125-178): 24 batches of 8
from a 20-expert pool against 16 slots, every returned block checked against
its host bytes."""
import numpy as np
import pytest

from oracle import lru as OL
from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import moe, synthdata
from windlass_amd.model import CachedModel, DeviceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)


class _MappedSource:
    """Oracle experts under the model's (layer, expert) -> synthetic key map."""

    def __init__(self, base, key):
        self.base, self.key = base, key

    def get(self, layer, expert):
        return self.base.get(*self.key(layer, expert))


def _decode_bytes(cfg):
    """The first regions of a native block (gu, gus, dn, dns): what a decode
    call's cache miss copies."""
    from oracle import native_layout
    return sum(native_layout.native_sizes(cfg.hidden, cfg.moe_inter)[:4])


def _pair(c, seed, L, capacity, n_host):
    zipf = synthdata.zipf_bias_offset(c["n_routed_experts"], seed)
    cm = CachedModel(c, seed=seed, n_layers=L, capacity=capacity, n_host=n_host, bias_offset=zipf)
    rm = DeviceModel(c, seed=seed, n_layers=L, bias_offset=zipf, expert_key=cm.expert_source_key)
    return cm, rm


def test_cached_layers_equal_resident_and_counters_match_replay(gpu):
    hip = gpu
    c = SMALL
    H, E, K, L = c["hidden"], c["n_routed_experts"], c["n_experts_per_tok"], 6
    cm, rm = _pair(c, 4, L, capacity=20, n_host=100)
    src = _MappedSource(O.ExpertSource(H, c["moe_inter"], 4), cm.expert_source_key)
    keys = []
    for t in range(8):
        h = synth.hidden_state(H, 50 + t)
        for l in range(L):
            outs = []
            for m in (cm, rm):
                dh, dout = make_io(H)
                dh.upload(h)
                m.ctx.run_moe_residual(l, dh.ptr, dh.ptr, dout.ptr)
                m.ctx.check_error()
                outs.append(dout.download(np.float32))
            ids = hip.download_ptr(cm.ctx.taps()["topk_idx"], np.int32, K)
            keys += [l * E + int(i) for i in ids]
            assert np.array_equal(outs[0], outs[1]), (t, l)
            if t == 0 and l in (0, L - 1):
                ref = O.moe_layer(h, cm.dense[l], src, l, c)
                assert np.array_equal(ids, ref["topk_idx"])
                assert O.rel_to_scale(ref["out"], outs[0] - h) < TOL
            h = outs[0]
    st = cm.ctx.cache_stats()
    _, hits, misses, ev = OL.replay(20, keys, K)
    print(f"cache: {st}", flush=True)
    assert (st["hits"], st["misses"], st["evictions"]) == (hits, misses, ev)
    # a decode miss copies the decode kernel's regions of the native block only
    assert st["used"] == 20 and st["bytes_h2d"] == misses * _decode_bytes(cm.cfg)
    cm.close()
    rm.close()


def test_speculative_chain_equals_resident(gpu):
    c = SMALL
    H, K, L = c["hidden"], c["n_experts_per_tok"], 6
    cm, rm = _pair(c, 5, L, capacity=24, n_host=120)
    cm.ctx.cache_set_speculation(True)
    for t in range(6):
        res = []
        for m in (cm, rm):
            dh, dtmp = make_io(H)
            dh.upload(synth.hidden_state(H, 70 + t))
            m.ctx.run_chain(0, L, dh.ptr, dtmp.ptr)
            m.ctx.check_error()
            res.append(dh.download(np.float32))
        assert np.array_equal(res[0], res[1]), t
    st = cm.ctx.cache_stats()
    print(f"speculative cache: {st}", flush=True)
    assert st["hits"] + st["misses"] == 6 * L * K
    assert st["spec_requests"] == 6 * (L - 1) * K
    assert st["spec_hits"] <= st["spec_copies"] <= st["spec_requests"]
    cm.close()
    rm.close()


def test_prefetch_get_reference_case4(gpu):
    hip = gpu
    c = dict(SMALL, n_experts_per_tok=8)
    cm = CachedModel(c, seed=6, n_layers=1, capacity=16, n_host=48)
    for b in range(24):
        ids = [(b * 3 + k) % 20 for k in range(8)]
        cm.ctx.cache_prefetch(0, ids)
        for e in ids:
            p = cm.ctx.cache_get(0, e)
            got = hip.download_ptr(p, np.uint8, 256)
            want = cm.host.view(np.uint8, 256, cm.host_block_index(0, e) * cm.nb)
            assert np.array_equal(got, want), (b, e)
    st = cm.ctx.cache_stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (115, 77, 61)
    cm.close()


def test_missing_host_block_is_an_io_error(gpu):
    c = SMALL
    H = c["hidden"]
    cm = CachedModel(c, seed=7, n_layers=1, capacity=12, n_host=48)
    ctx = moe.Context(cm.cfg)  # a second context over the same dense weights, with a failing source
    rw, bb, sb, _ = cm.bufs[0]
    ctx.set_layer(0, rw.ptr, bb.ptr, None, sb.ptr)
    ctx.cache_create(12, lambda l, e: 0)
    dh, dout = make_io(H)
    dh.upload(synth.hidden_state(H, 3))
    with pytest.raises(moe.WindlassError) as ei:
        ctx.run_moe(0, dh.ptr, dout.ptr)
    assert ei.value.status == 7
    ctx.close()
    cm.close()


def test_glm_shape_cached_equals_resident(gpu):
    GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
               routed_scaling=2.5, rms_eps=1e-5)
    H = GLM["hidden"]
    cm, rm = _pair(GLM, 8, 2, capacity=24, n_host=64)
    cm.ctx.cache_set_speculation(True)
    for t in range(3):
        res = []
        for m in (cm, rm):
            dh, dtmp = make_io(H)
            dh.upload(synth.hidden_state(H, 90 + t))
            m.ctx.run_chain(0, 2, dh.ptr, dtmp.ptr)
            m.ctx.check_error()
            res.append(dh.download(np.float32))
        assert np.array_equal(res[0], res[1]), t
    print(f"GLM cache: {cm.ctx.cache_stats()}", flush=True)
    cm.close()
    rm.close()


@pytest.mark.parametrize("kind", ["lfu", "slru", "2q", "tinylfu"])
def test_policy_cached_equals_resident(gpu, kind):
    """Every policy (and pinned keys) keeps the layer's bits: cached outputs
    equal the resident layer's (decode and batched), and the decode part's
    counters equal the oracle's replay of the requested ids under that policy
    (oracle/policies.py), misses not retained included."""
    from oracle import policies as OP
    hip = gpu
    c = SMALL
    H, E, K, L, cap = c["hidden"], c["n_routed_experts"], c["n_experts_per_tok"], 4, 16
    cm, rm = _pair(c, 9, L, capacity=cap, n_host=120)
    cm.ctx.cache_set_policy(kind)
    pins = [0 * E + 3, 2 * E + 11]
    for k in pins:
        cm.ctx.cache_pin(k // E, k % E)
    keys = []
    for t in range(6):
        h = synth.hidden_state(H, 980 + t)
        for l in range(L):
            outs = []
            for m in (cm, rm):
                dh, dout = make_io(H)
                dh.upload(h)
                m.ctx.run_moe_residual(l, dh.ptr, dh.ptr, dout.ptr)
                m.ctx.check_error()
                outs.append(dout.download(np.float32))
            keys += [l * E + int(i) for i in hip.download_ptr(cm.ctx.taps()["topk_idx"], np.int32, K)]
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), (kind, t, l)
            h = outs[0]
    st = cm.ctx.cache_stats()
    out, hits, misses, ev = OP.replay(kind, cap, keys, K, pinned=pins)
    print(f"{kind}: {st}", flush=True)
    assert (st["hits"], st["misses"], st["evictions"]) == (hits, misses, ev)
    assert st["bypassed"] == sum(1 for x in out if x == 3)
    T = 30  # the batched layer through the same cache
    hs = np.stack([synth.hidden_state(H, 990, i) for i in range(T)]).astype(np.float32)
    bo = []
    for m in (cm, rm):
        dh = hip.DeviceBuffer.from_array(hs)
        do = hip.DeviceBuffer(4 * T * H)
        m.ctx.run_moe_batched(1, T, dh.ptr, None, do.ptr)
        m.ctx.check_error()
        bo.append(do.download(np.float32))
    assert np.array_equal(bo[0].view(np.uint32), bo[1].view(np.uint32)), kind
    cm.close()
    rm.close()
