"""Checkpoint → slot table → layer on the GPU (run with -m gpu): the MoE
fields of glm::load_layer (src/glm_loader.cuh:524-620) and the routed experts
read from safetensors shards into pool slots, then run.

A checkpoint written from the synthetic generator under the reference's
tensor names holds the same bytes that DeviceModel binds: the loaded context
must give the DeviceModel's outputs bit for bit, and the oracle's within
1e-5 rel_to_scale."""
import os

import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from tests import st_writer
from windlass_amd import hip as H_
from windlass_amd import moe
from windlass_amd.model import DeviceModel, FileModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)
FIRST = 3  # checkpoint layer of context layer 0 (layers 0-2 of GLM are dense)


def _cfg(c, n_layers):
    return moe.make_config(hidden=c["hidden"], moe_inter=c["moe_inter"], n_routed_experts=c["n_routed_experts"],
                           n_experts_per_tok=c["n_experts_per_tok"], n_shared=c["n_shared"], n_layers=n_layers,
                           routed_scaling=c["routed_scaling"], rms_eps=c["rms_eps"])


def _decode(ctx, h, layer):
    dh, dout = make_io(h.shape[0])
    dh.upload(h)
    ctx.run_moe(layer, dh.ptr, dout.ptr)
    ctx.check_error()
    return dout.download(np.float32)


def _batched(ctx, hs, layer):
    T, H = hs.shape
    dh = H_.DeviceBuffer.from_array(hs)
    do = H_.DeviceBuffer(4 * T * H)
    ctx.run_moe_batched(layer, T, dh.ptr, None, do.ptr)
    ctx.check_error()
    return do.download(np.float32).reshape(T, H)


@pytest.mark.parametrize("shared", ["bf16", "mxfp4"])
def test_small_checkpoint_load_bind_run(gpu, tmp_path, shared):
    c = SMALL
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    seed, L = 61, 2
    mx = shared == "mxfp4"
    ts = []
    for l in range(L):
        ts += st_writer.moe_layer_tensors(c, seed, FIRST + l, l, shared_mxfp4=mx)
    st_writer.write_checkpoint(str(tmp_path), ts, n_shards=3)
    print(f"checkpoint: {len(ts)} tensors in 3 shards, shared {shared}", flush=True)
    st = moe.SafeTensors(str(tmp_path))
    ctx = moe.Context(_cfg(c, L))
    ctx.slot_pool_create(L * E)
    for l in range(L):
        ctx.load_layer(st, FIRST + l, l)
        ctx.load_experts(st, FIRST + l, l, n=E, first_slot=l * E)
    ln = [st_writer.ln_weight(H, seed, l) for l in range(L)]
    dm = DeviceModel(c, seed=seed, n_layers=L, ln_weights=ln, shared_mxfp4=mx)
    src = O.ExpertSource(H, I, seed)
    worst = 0.0
    for l in range(L):
        sh = src.get(*dm.shared_key(l)) if mx else None
        for t in range(3):
            h = synth.hidden_state(H, 700 + 10 * l + t)
            got = _decode(ctx, h, l)
            ref_dm = _decode(dm.ctx, h, l)
            assert np.array_equal(got.view(np.uint32), ref_dm.view(np.uint32)), (l, t)
            ref = O.moe_layer(h, dm.dense[l], src, l, c, ln_w=synth.bf16_to_f32(ln[l]), shared_f32=sh)
            r = O.rel_to_scale(ref["out"], got)
            worst = max(worst, r)
            assert r < TOL, (l, t, r)
        hs = np.stack([synth.hidden_state(H, 800 + l, t) for t in range(40)]).astype(np.float32)
        assert np.array_equal(_batched(ctx, hs, l).view(np.uint32), _batched(dm.ctx, hs, l).view(np.uint32)), l
    print(f"small, shared {shared}: loaded == synthetic bit for bit; worst vs oracle {worst:.2e}", flush=True)
    # binding a layer again (the context frees the buffers of the first load)
    ctx.load_layer(st, FIRST, 0)
    h = synth.hidden_state(H, 790)
    assert np.array_equal(_decode(ctx, h, 0).view(np.uint32), _decode(dm.ctx, h, 0).view(np.uint32))
    dm.close()
    ctx.close()
    st.close()


def test_glm_checkpoint_layer_fields_and_some_experts(gpu, tmp_path):
    """The GLM shape: router [256, 6144], bias, norm and the MXFP4 shared
    expert from the checkpoint; 8 routed experts from the checkpoint over a
    pool the synthetic generator filled (same bytes): bit-identical to the
    synthetic model, within 1e-5 of the oracle."""
    c = GLM
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    seed = 62
    load = [0, 5, 77, 128, 200, 201, 254, 255]
    ts = st_writer.moe_layer_tensors(c, seed, FIRST, 0, shared_mxfp4=True, experts=load)
    st_writer.write_checkpoint(str(tmp_path), ts, n_shards=4)
    print(f"GLM checkpoint: {sum(len(t[3]) for t in ts) / 1e6:.0f} MB", flush=True)
    st = moe.SafeTensors(str(tmp_path))
    ln = [st_writer.ln_weight(H, seed, 0)]
    dm = DeviceModel(c, seed=seed, n_layers=1, ln_weights=ln, shared_mxfp4=True)
    ctx = moe.Context(_cfg(c, 1))
    ctx.slot_pool_create(E + len(load))
    for e in range(E):
        p = ctx.slot_pool_ptr(e)
        moe.synth_expert_native(ctx.cfg, seed, 0, e, p)
        ctx.slot_bind(0, e, p)
    H_.synchronize()
    ctx.load_layer(st, FIRST, 0)
    ctx.load_experts(st, FIRST, 0, experts=load, first_slot=E)  # rebinds them to the extra slots
    src = O.ExpertSource(H, I, seed)
    sh = src.get(*dm.shared_key(0))
    for t in range(2):
        h = synth.hidden_state(H, 730 + t)
        got = _decode(ctx, h, 0)
        assert np.array_equal(got.view(np.uint32), _decode(dm.ctx, h, 0).view(np.uint32)), t
        ref = O.moe_layer(h, dm.dense[0], src, 0, c, ln_w=synth.bf16_to_f32(ln[0]), shared_f32=sh)
        assert O.rel_to_scale(ref["out"], got) < TOL, t
    # tokens routed to loaded experts: a bias that makes them win
    off = np.zeros(E, np.float32)
    off[load] = 5.0
    h = synth.hidden_state(H, 740)
    ref_dm = DeviceModel(c, seed=seed, n_layers=1, ln_weights=ln, shared_mxfp4=True, bias_offset=off)
    ts2 = st_writer.moe_layer_tensors(c, seed, FIRST + 1, 0, shared_mxfp4=True, experts=[], bias_offset=off)
    st_writer.write_checkpoint(str(tmp_path / "b"), ts2, n_shards=1)
    st2 = moe.SafeTensors(str(tmp_path / "b"))
    ctx.load_layer(st2, FIRST + 1, 0)
    got = _decode(ctx, h, 0)
    ids = H_.download_ptr(ctx.taps()["topk_idx"], np.int32, c["n_experts_per_tok"])
    assert set(int(i) for i in ids) <= set(load)
    assert np.array_equal(got.view(np.uint32), _decode(ref_dm.ctx, h, 0).view(np.uint32))
    print("GLM: checkpoint layer fields + 8 loaded experts == synthetic bit for bit", flush=True)
    ref_dm.close()
    dm.close()
    ctx.close()


def test_packed_file_from_checkpoint_feeds_the_file_tier(gpu, tmp_path):
    """Checkpoint -> wl_st_pack_layer -> layer_N.bin -> the cache's file tier:
    the same outputs as the resident synthetic model."""
    c = SMALL
    H, E = c["hidden"], c["n_routed_experts"]
    seed, L = 63, 2
    ts = []
    for l in range(L):
        ts += st_writer.moe_layer_tensors(c, seed, l, l)
    st_writer.write_checkpoint(str(tmp_path / "ck"), ts, n_shards=2)
    st = moe.SafeTensors(str(tmp_path / "ck"))
    cfg = _cfg(c, L)
    os.makedirs(tmp_path / "packed")
    for l in range(L):
        st.pack_layer(cfg, l, str(tmp_path / "packed" / f"layer_{l}.bin"))
    fm = FileModel(c, seed, L, capacity=2 * c["n_experts_per_tok"] + 4, directory=str(tmp_path / "packed"),
                   io_threads=2, ln_weights=[st_writer.ln_weight(H, seed, l) for l in range(L)])
    dm = DeviceModel(c, seed=seed, n_layers=L, ln_weights=[st_writer.ln_weight(H, seed, l) for l in range(L)])
    for l in range(L):
        for t in range(4):
            h = synth.hidden_state(H, 750 + 10 * l + t)
            assert np.array_equal(_decode(fm.ctx, h, l).view(np.uint32), _decode(dm.ctx, h, l).view(np.uint32)), (l, t)
    fm.close()
    dm.close()


def test_loader_errors(gpu, tmp_path):
    c = SMALL
    H, E = c["hidden"], c["n_routed_experts"]
    ts = st_writer.moe_layer_tensors(c, 64, 0, 0, experts=[0, 1, 2])
    drop = {"model.layers.0.mlp.experts.2.down_proj.weight_scale"}
    st_writer.write_checkpoint(str(tmp_path), [t for t in ts if t[0] not in drop], n_shards=1)
    st = moe.SafeTensors(str(tmp_path))
    ctx = moe.Context(_cfg(c, 1))

    def status(fn, *a, **k):
        with pytest.raises(moe.WindlassError) as ei:
            fn(*a, **k)
        return ei.value.status

    assert status(ctx.load_experts, st, 0, 0, experts=[0]) == 5      # no slot pool: WL_ERR_STATE
    ctx.slot_pool_create(4)
    assert status(ctx.load_experts, st, 0, 0, experts=[0, 1], first_slot=3) == 1  # past the pool
    assert status(ctx.load_experts, st, 0, 0, experts=[2]) == 9      # no _scale: WL_ERR_FORMAT
    assert status(ctx.load_experts, st, 0, 0, experts=[5]) == 8      # absent: WL_ERR_NOT_FOUND
    assert status(ctx.load_experts, st, 0, 0, experts=[1, 1]) == 1   # listed twice
    assert status(ctx.load_experts, st, 0, 0, experts=[E]) == 1      # out of range
    assert status(ctx.load_layer, st, 9, 0) == 8                     # no such checkpoint layer
    assert status(ctx.load_layer, st, 0, 1) == 1                     # no such context layer
    ctx.load_experts(st, 0, 0, experts=[0, 1])                       # the good ones load
    # a wrong shape (router transposed) and a wrong dtype (bias in bf16)
    bad = [(n, d, (s[1], s[0]) if n.endswith("mlp.gate.weight") else s, b) for n, d, s, b in ts]
    st_writer.write_checkpoint(str(tmp_path / "t"), bad, n_shards=1)
    assert status(ctx.load_layer, moe.SafeTensors(str(tmp_path / "t")), 0, 0) == 9
    bias_bf16 = [(n, "BF16", (2 * s[0],), b) if n.endswith("e_score_correction_bias") else (n, d, s, b)
                 for n, d, s, b in ts]
    st_writer.write_checkpoint(str(tmp_path / "d"), bias_bf16, n_shards=1)
    assert status(ctx.load_layer, moe.SafeTensors(str(tmp_path / "d")), 0, 0) == 9
    ctx.close()
