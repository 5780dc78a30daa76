"""The safetensors reader and the packed-file writer (host only, no GPU):
reference st::open / st::info / st::read_bytes (src/safetensors_io.cuh:
89-230) and the packed layer files of tools/repack_experts_glm.py:5-14,46-55.

The reader is pinned against the `safetensors` library (files it writes are
read back byte for byte, and files the test writer makes are read by both);
malformed files are refused with a status instead of being read past."""
import json
import os
import struct

import numpy as np
import pytest

from oracle import synth
from tests import st_writer
from windlass_amd import moe

NOT_FOUND, FORMAT, IO, INVALID = 8, 9, 7, 1
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1)


def _status(fn, *a, **k):
    with pytest.raises(moe.WindlassError) as ei:
        fn(*a, **k)
    return ei.value.status


def test_reads_files_of_the_safetensors_library(tmp_path):
    sn = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(3)
    arrays = {"a.u8": rng.integers(0, 255, (7, 9), dtype=np.uint8),
              "b.f32": rng.standard_normal(33).astype(np.float32),
              "c.u16": rng.integers(0, 65535, (2, 3, 4), dtype=np.uint16),
              "d.i64": np.arange(5, dtype=np.int64),
              "e.scalar": np.array(2.5, dtype=np.float64),
              "f.empty": np.zeros((0, 4), np.float32)}
    path = str(tmp_path / "lib.safetensors")
    sn.save_file(arrays, path, metadata={"format": "np"})
    st = moe.SafeTensors(path)
    assert st.names() == sorted(arrays)
    dt = {np.uint8: "U8", np.float32: "F32", np.uint16: "U16", np.int64: "I64", np.float64: "F64"}
    for name, a in arrays.items():
        info = st.info(name)
        assert info["dtype"] == dt[a.dtype.type]
        assert info["shape"] == a.shape
        assert info["nbytes"] == a.nbytes
        assert st.read(name).tobytes() == a.tobytes()
    assert st.info("nope") is None
    assert _status(st.read, "nope") == NOT_FOUND
    assert _status(st.read, "b.f32", capacity=8) == INVALID
    st.close()


def test_writer_agrees_with_the_library(tmp_path):
    """The test writer's files (BF16 included) read back through the
    library's torch loader and through wl_st_read give the same bytes."""
    safe_open = pytest.importorskip("safetensors").safe_open
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    bf = rng.integers(0, 65535, (5, 6), dtype=np.uint16)
    f32 = rng.standard_normal(7).astype(np.float32)
    u8 = rng.integers(0, 255, (3, 8), dtype=np.uint8)
    path = str(tmp_path / "w.safetensors")
    st_writer.write_safetensors(path, [("x.bf16", "BF16", bf.shape, bf.tobytes()),
                                       ("y.f32", "F32", f32.shape, f32.tobytes()),
                                       ("z.u8", "U8", u8.shape, u8.tobytes())], metadata={"format": "pt"})
    with safe_open(path, framework="pt") as f:
        assert sorted(f.keys()) == ["x.bf16", "y.f32", "z.u8"]
        t = f.get_tensor("x.bf16")
        assert t.dtype == torch.bfloat16 and tuple(t.shape) == bf.shape
        assert t.view(torch.int16).numpy().view(np.uint16).tobytes() == bf.tobytes()
        assert f.get_tensor("y.f32").numpy().tobytes() == f32.tobytes()
    st = moe.SafeTensors(path)
    assert st.read("x.bf16").tobytes() == bf.tobytes()
    assert st.read("y.f32").tobytes() == f32.tobytes()
    assert st.info("z.u8")["shape"] == (3, 8)


def test_sharded_index(tmp_path):
    ts = [(f"t{i}", "U8", (i + 1,), bytes(range(i, 2 * i + 1))) for i in range(10)]
    st_writer.write_checkpoint(str(tmp_path), ts, n_shards=3)
    st = moe.SafeTensors(str(tmp_path))
    assert st.names() == sorted(t[0] for t in ts)
    for i, (name, _, shape, data) in enumerate(ts):
        info = st.info(name)
        assert info["shape"] == shape
        assert st.read(name).tobytes() == data
    shards = {st.info(t[0])["shard"] for t in ts}
    assert len(shards) == 3
    # a missing shard: refused, or skipped with allow_missing_shards
    os.remove(tmp_path / "model-00002-of-00003.safetensors")
    assert _status(moe.SafeTensors, str(tmp_path)) == IO
    st2 = moe.SafeTensors(str(tmp_path), allow_missing_shards=True)
    present = {t[0] for i, t in enumerate(ts) if i % 3 != 1}
    assert set(st2.names()) == present
    assert st2.info("t1") is None
    assert st2.read("t3").tobytes() == ts[3][3]


def test_unicode_and_escaped_names(tmp_path):
    names = ["café.weight", 'q"uote', "back\\slash", "emoji\U0001F600", "tab\tname"]
    ts = [(n, "U8", (2,), bytes([i, i + 1])) for i, n in enumerate(names)]
    path = str(tmp_path / "u.safetensors")
    st_writer.write_safetensors(path, ts)  # json.dumps writes \\u escapes and surrogate pairs
    st = moe.SafeTensors(path)
    assert st.names() == sorted(names, key=lambda s: s.encode())
    for n, _, _, data in ts:
        assert st.read(n).tobytes() == data


def _raw(path, header_bytes, data=b""):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header_bytes)))
        f.write(header_bytes)
        f.write(data)


@pytest.mark.parametrize("case", ["json", "trailing", "dup", "offsets_past_end", "shape_mismatch", "reversed",
                                  "no_dtype", "header_too_long", "short_file", "deep", "neg_dim"])
def test_malformed_files_refused(tmp_path, case):
    p = str(tmp_path / "bad.safetensors")
    ok = {"t": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}}
    if case == "json":
        _raw(p, b'{"t": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]', b"abcd")
    elif case == "trailing":
        _raw(p, json.dumps(ok).encode() + b" x", b"abcd")
    elif case == "dup":
        _raw(p, b'{"t": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}, '
                b'"t": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}}', b"abcd")
    elif case == "offsets_past_end":
        _raw(p, json.dumps(ok).encode(), b"abc")
    elif case == "shape_mismatch":
        _raw(p, json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 4]}}).encode(), b"abcd")
    elif case == "reversed":
        _raw(p, json.dumps({"t": {"dtype": "U8", "shape": [0], "data_offsets": [4, 0]}}).encode(), b"abcd")
    elif case == "no_dtype":
        _raw(p, json.dumps({"t": {"shape": [4], "data_offsets": [0, 4]}}).encode(), b"abcd")
    elif case == "header_too_long":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 1 << 40))
            f.write(b"{}")
    elif case == "short_file":
        with open(p, "wb") as f:
            f.write(b"\x02\x00")
    elif case == "deep":
        _raw(p, b"[" * 100 + b"]" * 100)
    elif case == "neg_dim":
        _raw(p, json.dumps({"t": {"dtype": "U8", "shape": [-4], "data_offsets": [0, 4]}}).encode(), b"abcd")
    assert _status(moe.SafeTensors, p) == FORMAT, moe.load().wl_st_last_error(None)


def test_index_errors(tmp_path):
    d = tmp_path / "ck"
    st_writer.write_checkpoint(str(d), [("a", "U8", (1,), b"\x01"), ("b", "U8", (1,), b"\x02")], n_shards=1)
    idx = json.loads((d / "model.safetensors.index.json").read_text())
    # a name the index lists but the shard lacks
    idx["weight_map"]["c"] = "model-00001-of-00001.safetensors"
    (d / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert _status(moe.SafeTensors, str(d)) == FORMAT
    # a shard path that leaves the directory
    idx["weight_map"] = {"a": "../model-00001-of-00001.safetensors"}
    (d / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert _status(moe.SafeTensors, str(d)) == FORMAT
    (d / "model.safetensors.index.json").write_text('{"metadata": {}}')
    assert _status(moe.SafeTensors, str(d)) == FORMAT
    # no index and no model.safetensors
    e = tmp_path / "empty"
    e.mkdir()
    assert _status(moe.SafeTensors, str(e)) == IO
    # an index-less directory with model.safetensors is one shard
    st_writer.write_safetensors(str(e / "model.safetensors"), [("z", "U8", (3,), b"xyz")])
    assert moe.SafeTensors(str(e)).read("z").tobytes() == b"xyz"


def test_pack_layer_matches_the_synthetic_blocks(tmp_path):
    """wl_st_pack_layer writes record e as the six expert tensors in layout
    order: byte-equal to the oracle's packed block of the same expert."""
    c = SMALL
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    cfg = moe.make_config(hidden=H, moe_inter=I, n_routed_experts=E, n_experts_per_tok=c["n_experts_per_tok"],
                          n_shared=1, n_layers=1)
    st_writer.write_checkpoint(str(tmp_path / "ck"), st_writer.moe_layer_tensors(c, 5, 7, 2), n_shards=3)
    st = moe.SafeTensors(str(tmp_path / "ck"))
    out = str(tmp_path / "layer_7.bin")
    st.pack_layer(cfg, 7, out)
    blk = moe.expert_layout(cfg).total
    data = np.fromfile(out, np.uint8)
    assert data.size == E * blk
    for e in [0, 1, 17, E - 1]:
        assert np.array_equal(data[e * blk:(e + 1) * blk], synth.expert_block_bytes(H, I, 5, 2, e)), e
    # a layer without experts: NOT_FOUND, and no partial file is left
    bad = str(tmp_path / "layer_8.bin")
    assert _status(st.pack_layer, cfg, 8, bad) == NOT_FOUND
    assert not os.path.exists(bad)


def test_pack_layer_refuses_a_non_mxfp4_expert(tmp_path):
    c = SMALL
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    cfg = moe.make_config(hidden=H, moe_inter=I, n_routed_experts=E, n_experts_per_tok=c["n_experts_per_tok"],
                          n_shared=1, n_layers=1)
    ts = [t for t in st_writer.moe_layer_tensors(c, 5, 0, 0) if t[0] != "model.layers.0.mlp.experts.3.up_proj.weight_scale"]
    st_writer.write_checkpoint(str(tmp_path), ts, n_shards=2)
    st = moe.SafeTensors(str(tmp_path))
    assert _status(st.pack_layer, cfg, 0, str(tmp_path / "x.bin")) == FORMAT
    assert "no _scale" in moe.load().wl_st_last_error(st.h).decode()
