"""The packed-file tier of the expert cache on the GPU (run with -m gpu):
wl_cache_create_files over layer_N.bin files in the reference's format
(tools/repack_experts_glm.py:5-14,46-55; reference I/O path
src/glm_expert_cache.cuh:29-62,339-475).

The files are written here from the oracle's numpy generator (record e of
layer l = the synthetic expert (l, e) in the reference layout). Cases follow
the reference's cache test (src/test_glm_expert_cache.cu:46-181): a cold miss
then a hit, a block's bytes against the file's bytes at the expert's offset
(here: its native conversion), LRU eviction at capacity 4, and 24 batches of
8 from a 20-expert pool against 16 slots with 4 I/O threads; plus whole
layers (decode, chain with speculation, batched) equal to the resident layers
bit for bit, and the I/O errors."""
import os

import numpy as np
import pytest

from oracle import lru as OL
from oracle import native_layout, synth
from windlass_amd import moe, synthdata
from windlass_amd.model import DeviceModel, FileModel, make_io

pytestmark = pytest.mark.gpu
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)


def write_layers(directory, c, seed, n_layers, first_layer=0):
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    for l in range(n_layers):
        with open(os.path.join(directory, f"layer_{first_layer + l}.bin"), "wb") as f:
            for e in range(E):
                for part in synth.expert_block(H, I, seed, l, e):
                    f.write(np.ascontiguousarray(part).tobytes())


def record(c, seed, layer, expert):
    return synth.expert_block(c["hidden"], c["moe_inter"], seed, layer, expert)


@pytest.mark.parametrize("io_threads", [0, 4])
def test_reference_cases_1_2_3(gpu, tmp_path, io_threads):
    hip = gpu
    c = dict(SMALL, n_experts_per_tok=2)  # capacity 4 >= 2 x K
    write_layers(tmp_path, c, 51, 1)
    fm = FileModel(c, seed=51, n_layers=1, capacity=4, directory=str(tmp_path), io_threads=io_threads)
    nb = moe.native_block_bytes(fm.cfg)
    # case 1: cold miss, then a hit
    fm.ctx.cache_prefetch(0, [7])
    p = fm.ctx.cache_get(0, 7)
    st = fm.ctx.cache_stats()
    assert (st["hits"], st["misses"]) == (0, 1)
    fm.ctx.cache_prefetch(0, [7])
    assert fm.ctx.cache_get(0, 7) == p
    assert fm.ctx.cache_stats()["hits"] == 1
    # case 2: the block equals the file's record at offset 7 x block bytes, converted
    want = native_layout.to_native(record(c, 51, 0, 7), c["hidden"], c["moe_inter"])
    hip.synchronize()
    assert np.array_equal(hip.download_ptr(p, np.uint8, nb), want)
    # case 3: LRU order at capacity 4 — 7 is the oldest after 0, 1, 2, so 3 evicts it
    for e in (0, 1, 2):
        fm.ctx.cache_prefetch(0, [e])
        fm.ctx.cache_get(0, e)
    fm.ctx.cache_prefetch(0, [3])
    fm.ctx.cache_get(0, 3)
    st = fm.ctx.cache_stats()
    assert st["evictions"] == 1 and st["used"] == 4
    fm.ctx.cache_prefetch(0, [7])  # a miss again
    assert fm.ctx.cache_stats()["misses"] == 6
    fm.close()


def test_reference_case4_four_io_threads(gpu, tmp_path):
    hip = gpu
    c = dict(SMALL, n_experts_per_tok=8)
    write_layers(tmp_path, c, 52, 1)
    fm = FileModel(c, seed=52, n_layers=1, capacity=16, directory=str(tmp_path), io_threads=4)
    nb = moe.native_block_bytes(fm.cfg)
    native = {}
    keys = []
    for b in range(24):
        ids = [(b * 3 + k) % 20 for k in range(8)]
        keys += ids
        fm.ctx.cache_prefetch(0, ids)
        for e in ids:
            p = fm.ctx.cache_get(0, e)
            hip.synchronize()
            if e not in native:
                native[e] = native_layout.to_native(record(c, 52, 0, e), c["hidden"], c["moe_inter"])
            assert np.array_equal(hip.download_ptr(p, np.uint8, nb), native[e]), (b, e)
    st = fm.ctx.cache_stats()
    assert (st["hits"], st["misses"], st["evictions"]) == (115, 77, 61)
    assert OL.replay(16, keys, 8)[1:] == (115, 77, 61)
    fm.close()


def test_file_layers_equal_resident(gpu, tmp_path):
    """Decode, the speculative chain and the batched layer through files give
    the resident layers' bits; the counters equal an LRU replay of the ids."""
    hip = gpu
    c = SMALL
    H, E, K, L = c["hidden"], c["n_routed_experts"], c["n_experts_per_tok"], 4
    write_layers(tmp_path, c, 53, L, first_layer=3)
    zipf = synthdata.zipf_bias_offset(E, 53)
    fm = FileModel(c, seed=53, n_layers=L, capacity=20, directory=str(tmp_path), first_layer=3, bias_offset=zipf)
    rm = DeviceModel(c, seed=53, n_layers=L, bias_offset=zipf)
    keys = []
    for t in range(5):
        h = synth.hidden_state(H, 950 + t)
        for l in range(L):
            outs = []
            for m in (fm, rm):
                dh, dout = make_io(H)
                dh.upload(h)
                m.ctx.run_moe_residual(l, dh.ptr, dh.ptr, dout.ptr)
                m.ctx.check_error()
                outs.append(dout.download(np.float32))
            keys += [l * E + int(i) for i in hip.download_ptr(fm.ctx.taps()["topk_idx"], np.int32, K)]
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), (t, l)
            h = outs[0]
    st = fm.ctx.cache_stats()
    _, hits, misses, ev = OL.replay(20, keys, K)
    assert (st["hits"], st["misses"], st["evictions"]) == (hits, misses, ev)
    assert st["bytes_h2d"] == misses * moe.expert_layout(fm.cfg).total
    # the chain with cross-layer speculation
    fm.ctx.cache_set_speculation(True)
    for t in range(3):
        res = []
        for m in (fm, rm):
            dh, dtmp = make_io(H)
            dh.upload(synth.hidden_state(H, 960 + t))
            m.ctx.run_chain(0, L, dh.ptr, dtmp.ptr)
            m.ctx.check_error()
            res.append(dh.download(np.float32))
        assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32)), t
    # the batched layer, every unique expert read once
    fm.ctx.cache_set_speculation(False)
    T = 40
    hs = np.stack([synth.hidden_state(H, 970, i) for i in range(T)]).astype(np.float32)
    outs = []
    for m in (fm, rm):
        dh = hip.DeviceBuffer.from_array(hs)
        do = hip.DeviceBuffer(4 * T * H)
        m.ctx.run_moe_batched(1, T, dh.ptr, dh.ptr, do.ptr)
        m.ctx.check_error()
        outs.append(do.download(np.float32))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    print(f"file tier: {fm.ctx.cache_stats()}", flush=True)
    fm.close()
    rm.close()


def test_destroy_with_reads_in_flight(gpu, tmp_path):
    """Regression: reads queued but never waited for when the context is
    destroyed (the workers are joined before the events and the pool go)."""
    c = dict(SMALL, n_experts_per_tok=8)
    write_layers(tmp_path, c, 55, 1)
    for _ in range(3):
        fm = FileModel(c, seed=55, n_layers=1, capacity=32, directory=str(tmp_path), io_threads=4)
        for b in range(3):
            fm.ctx.cache_prefetch(0, [(8 * b + k) % 48 for k in range(8)])
        fm.close()


def test_missing_or_short_file_is_an_io_error(gpu, tmp_path):
    c = SMALL
    write_layers(tmp_path, c, 54, 1)
    cfg = moe.make_config(hidden=c["hidden"], moe_inter=c["moe_inter"], n_routed_experts=c["n_routed_experts"],
                          n_experts_per_tok=c["n_experts_per_tok"], n_layers=2)
    ctx = moe.Context(cfg)
    with pytest.raises(moe.WindlassError) as ei:  # layer_1.bin is missing
        ctx.cache_create_files(12, str(tmp_path), 0, 2)
    assert ei.value.status == 7 and "layer_1.bin" in str(ei.value)
    with open(tmp_path / "layer_1.bin", "wb") as f:  # one record short
        f.write(b"\0" * ((c["n_routed_experts"] - 1) * moe.expert_layout(cfg).total))
    with pytest.raises(moe.WindlassError) as ei:
        ctx.cache_create_files(12, str(tmp_path), 0, 2)
    assert ei.value.status == 7
    ctx.close()
