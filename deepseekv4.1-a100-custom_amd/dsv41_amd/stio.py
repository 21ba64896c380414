"""Safetensors checkpoint reader over memory maps, with the call surface of the reference's stio.Checkpoint
(stio.py:24-69): names / meta / get / __contains__, tensors as zero-copy CPU views of the mapped file (or a copy on a
device), a `rows` slice of the leading dimension that touches only those rows, and the checkpoint dtypes torch has no
arithmetic for kept as raw bytes (F8_E8M0 scales as uint8; I8 packed FP4 weights as int8).

A checkpoint directory holds model.safetensors.index.json ({"weight_map": name -> file}) and the files it names, or
a single model.safetensors (then the weight map is read from its header). A safetensors file is an 8-byte little-endian
header length, a JSON header {name: {"dtype", "shape", "data_offsets": [begin, end]}} (offsets relative to the end of
the header), then the data.
"""
from __future__ import annotations

import json
import mmap
import os
import struct

import numpy as np
import torch

# checkpoint dtype -> (torch dtype of the view, bytes per element)
DTYPES = {
    "F8_E4M3": (torch.float8_e4m3fn, 1),
    "F8_E8M0": (torch.uint8, 1),     # raw E8M0 bytes (quant.e8m0_to_float gives their values)
    "I8": (torch.int8, 1),           # packed E2M1 pairs in the expert weights
    "U8": (torch.uint8, 1),
    "BF16": (torch.bfloat16, 2),
    "F16": (torch.float16, 2),
    "F32": (torch.float32, 4),
    "I32": (torch.int32, 4),
    "I64": (torch.int64, 8),
}


class _File:
    """One mapped safetensors file: its parsed header and the byte offset where the data begins."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            self.header = json.loads(f.read(n))
            self.base = 8 + n
            # copy-on-write: tensors handed out are views of the file's pages, and a caller that writes into one
            # gets private pages (the file is never modified) instead of a fault on a read-only mapping
            self.map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_COPY)
        self.header.pop("__metadata__", None)


class Checkpoint:
    def __init__(self, path: str):
        self.path = path
        index = os.path.join(path, "model.safetensors.index.json")
        self._files: dict[str, _File] = {}
        if os.path.exists(index):
            with open(index) as f:
                self.weight_map: dict[str, str] = json.load(f)["weight_map"]
        else:
            single = "model.safetensors"
            self.weight_map = {name: single for name in self._file(single).header}

    def _file(self, fn: str) -> _File:
        f = self._files.get(fn)
        if f is None:
            f = self._files[fn] = _File(os.path.join(self.path, fn))
        return f

    def __contains__(self, name: str) -> bool:
        return name in self.weight_map

    def names(self, prefix: str = "") -> list[str]:
        return [n for n in self.weight_map if n.startswith(prefix)]

    def meta(self, name: str) -> tuple[str, list[int]]:
        m = self._file(self.weight_map[name]).header[name]
        return m["dtype"], list(m["shape"])

    def config(self) -> dict:
        """The model's config.json beside the weights ({} when absent)."""
        p = os.path.join(self.path, "config.json")
        if not os.path.exists(p):
            return {}
        with open(p) as f:
            return json.load(f)

    def get(self, name: str, device=None, rows: slice | None = None) -> torch.Tensor:
        """`name` as a CPU tensor viewing the mapped file (device None), or a copy on `device`. `rows` selects a range
        of the leading dimension; only those bytes are mapped into the view. The views of one Checkpoint share its
        copy-on-write mapping: writing into one never changes the file, but later get()s of the same bytes from this
        Checkpoint see the write (clone() for a tensor of its own)."""
        f = self._file(self.weight_map[name])
        m = f.header[name]
        tdtype, esize = DTYPES[m["dtype"]]
        shape = list(m["shape"])
        begin, end = m["data_offsets"]
        if rows is not None:
            per_row = esize * (int(np.prod(shape[1:])) if len(shape) > 1 else 1)
            r0, r1, step = rows.indices(shape[0])
            assert step == 1, "rows must be a contiguous range"
            begin, end = begin + r0 * per_row, begin + r1 * per_row
            shape[0] = r1 - r0
        if end - begin != esize * int(np.prod(shape)):
            raise ValueError(f"{name}: {end - begin} bytes for shape {shape} of {m['dtype']}")
        if end == begin:
            t = torch.empty(shape, dtype=tdtype)
        else:
            t = torch.frombuffer(f.map, dtype=torch.uint8, count=end - begin, offset=f.base + begin)
            t = t.view(tdtype).view(shape)
        return t if device is None else t.to(device)
