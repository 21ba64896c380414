"""Test helper: write safetensors checkpoints (header + raw bytes), including the checkpoint dtypes numpy and the
safetensors package do not model (F8_E8M0, F8_E4M3), so the reader is exercised on exactly the on-disk format."""
import json
import os
import struct

import numpy as np

ESIZE = {"F8_E4M3": 1, "F8_E8M0": 1, "I8": 1, "U8": 1, "BF16": 2, "F16": 2, "F32": 4, "I32": 4, "I64": 8}


def write_file(path, tensors):
    """tensors: {name: (dtype string, shape, numpy array of the raw bytes / values)}; data in name order."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        dtype, shape, arr = tensors[name]
        raw = np.ascontiguousarray(arr).tobytes()
        assert len(raw) == ESIZE[dtype] * int(np.prod(shape)), name
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def write_checkpoint(dirpath, tensors, n_files=2, config=None):
    """Split `tensors` over n_files shards with a model.safetensors.index.json weight map (and config.json)."""
    os.makedirs(dirpath, exist_ok=True)
    names = sorted(tensors)
    shards = [names[i::n_files] for i in range(n_files)]
    wmap = {}
    for i, part in enumerate(shards):
        fn = f"model-{i + 1:05d}-of-{n_files:05d}.safetensors"
        write_file(os.path.join(dirpath, fn), {n: tensors[n] for n in part})
        wmap.update({n: fn for n in part})
    with open(os.path.join(dirpath, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
    if config is not None:
        with open(os.path.join(dirpath, "config.json"), "w") as f:
            json.dump(config, f)
