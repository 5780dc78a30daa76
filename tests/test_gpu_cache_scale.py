"""Config 4 at its own scale (GPU; run with -m gpu): 75 GLM MoE layers behind
a 3,094-slot HBM expert cache (62 GB), filled from 512 pinned host blocks,
router bias with the Zipf popularity offset. Layer by layer over 12 tokens
(7,200 expert requests, more distinct experts than slots, so blocks are
evicted and refilled), every cached layer must equal the same layer run with
every expert resident (AliasedModel binds the same 512 blocks), and the
cache's counters must equal a replay of the requested ids through the LRU
oracle (reference semantics, src/glm_expert_cache.cuh:198-308). The first
layer of the first token is also checked against the numpy oracle."""
import numpy as np
import pytest

from oracle import lru as OL
from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import synthdata
from windlass_amd.model import AliasedModel, CachedModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)
L, SLOTS, NHOST, TOKENS, SEED = 75, 3094, 512, 12, 12


class _MappedSource:
    def __init__(self, base, key):
        self.base, self.key = base, key

    def get(self, layer, expert):
        return self.base.get(*self.key(layer, expert))


def _decode_bytes(cfg):
    """The first regions of a native block (gu, gus, dn, dns): what a decode
    call's cache miss copies."""
    from oracle import native_layout
    return sum(native_layout.native_sizes(cfg.hidden, cfg.moe_inter)[:4])


def test_config4_scale_cached_equals_resident_and_counters_match_replay(gpu):
    hip = gpu
    H, E, K = GLM["hidden"], GLM["n_routed_experts"], GLM["n_experts_per_tok"]
    zipf = synthdata.zipf_bias_offset(E, SEED)
    print(f"building {L} cached layers ({SLOTS} slots, {NHOST} host blocks) and the resident twin", flush=True)
    cm = CachedModel(GLM, seed=SEED, n_layers=L, capacity=SLOTS, n_host=NHOST, bias_offset=zipf, shared_alias=True)
    rm = AliasedModel(GLM, seed=SEED, n_layers=L, n_blocks=NHOST, bias_offset=zipf, shared_alias=True)
    for l in (0, 37, L - 1):
        for e in (0, 101, E - 1):
            assert cm.expert_source_key(l, e) == rm.expert_source_key(l, e)
    keys = []
    bufs = {m: make_io(H) for m in ("c", "r")}
    for t in range(TOKENS):
        h = synth.hidden_state(H, 1200 + t)
        for m in ("c", "r"):
            bufs[m][0].upload(h)
        for l in range(L):
            outs = []
            for name, model in (("c", cm), ("r", rm)):
                dh, dout = bufs[name]
                model.ctx.run_moe_residual(l, dh.ptr, dh.ptr, dout.ptr)
                model.ctx.check_error()
                outs.append(dout.download(np.float32))
                bufs[name] = (dout, dh)  # this layer's output is the next layer's input
            ids = hip.download_ptr(cm.ctx.taps()["topk_idx"], np.int32, K)
            keys += [l * E + int(i) for i in ids]
            assert np.array_equal(outs[0], outs[1]), (t, l)
            if t == 0 and l == 0:
                src = _MappedSource(O.ExpertSource(H, GLM["moe_inter"], SEED), cm.expert_source_key)
                ref = O.moe_layer(h, cm.dense[0], src, 0, GLM)
                assert np.array_equal(ids, ref["topk_idx"])
                assert O.rel_to_scale(ref["out"], outs[0] - h) < TOL
        print(f"token {t}: {len(set(keys))} distinct experts requested so far", flush=True)
    st = cm.ctx.cache_stats()
    _, hits, misses, ev = OL.replay(SLOTS, keys, K)
    print(f"cache: {st}", flush=True)
    assert len(set(keys)) > SLOTS  # the run evicted
    assert (st["hits"], st["misses"], st["evictions"]) == (hits, misses, ev)
    # a decode miss copies the decode kernel's regions of the native block only
    assert st["used"] == SLOTS and st["bytes_h2d"] == misses * _decode_bytes(cm.cfg)
    cm.close()
    rm.close()
