"""Safetensors files of the published format (host side): an 8-byte
little-endian header length, a JSON header {name: {dtype, shape,
data_offsets}} padded with spaces to a multiple of 8 bytes, the data; and a
sharded checkpoint directory (model.safetensors.index.json + shards), the
layout wl_st_open reads. Used to write synthetic checkpoints (the benchmark,
the tests); tensors are streamed to the file one at a time."""
import json
import os
import struct


def _nbytes(data):
    return data.nbytes if hasattr(data, "nbytes") else len(data)


def write_safetensors(path, tensors, metadata=None):
    """tensors: list of (name, dtype, shape, data) in file order; data is
    bytes or a numpy array (written as its raw bytes), or a callable
    returning one (called when the tensor is written)."""
    header = {}
    if metadata is not None:
        header["__metadata__"] = metadata
    sizes = []
    for name, dtype, shape, data in tensors:
        n = data[1] if isinstance(data, tuple) else _nbytes(data)
        sizes.append(n)
    off = 0
    for (name, dtype, shape, _), n in zip(tensors, sizes):
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for (_, _, _, data), n in zip(tensors, sizes):
            if isinstance(data, tuple):  # (callable, nbytes): produced when written
                data = data[0]()
            b = data.tobytes() if hasattr(data, "tobytes") else data
            assert len(b) == n
            f.write(b)


def write_checkpoint(directory, tensors, n_shards=2):
    """A sharded checkpoint: tensors dealt round robin over n_shards files
    model-0000i-of-0000n.safetensors, plus model.safetensors.index.json."""
    os.makedirs(directory, exist_ok=True)
    shards = [[] for _ in range(n_shards)]
    for i, t in enumerate(tensors):
        shards[i % n_shards].append(t)
    weight_map, total = {}, 0
    for s, ts in enumerate(shards):
        fn = f"model-{s + 1:05d}-of-{n_shards:05d}.safetensors"
        write_safetensors(os.path.join(directory, fn), ts, metadata={"format": "pt"})
        for name, _, _, data in ts:
            weight_map[name] = fn
            total += data[1] if isinstance(data, tuple) else _nbytes(data)
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": total}, "weight_map": weight_map}, f, indent=2)
