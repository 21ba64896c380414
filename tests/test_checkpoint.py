"""Checkpoint ingest on the CPU: the safetensors reader (stio.Checkpoint surface, stio.py:24-69) against the published
safetensors library on the standard dtypes and against the bytes written for the checkpoint-only ones (F8_E8M0, I8,
F8_E4M3); row slices; the expert stacking w13 = [w1; w3] of load.load_layer (load.py:128-148) and its tiling."""
import os

import numpy as np
import pytest
import torch

from _safetensors import write_checkpoint, write_file
from dsv41_amd import load, quant, stio


def _layer_tensors(rng, E, H, I, prefix="layers.0."):
    t = {}
    for e in range(E):
        q = f"{prefix}ffn.experts.{e}."
        for k, (n, kk) in {"w1": (I, H), "w3": (I, H), "w2": (H, I)}.items():
            t[q + k + ".weight"] = ("I8", (n, kk // 2), rng.integers(0, 256, (n, kk // 2), dtype=np.uint8))
            t[q + k + ".scale"] = ("F8_E8M0", (n, kk // 32), rng.integers(119, 124, (n, kk // 32), dtype=np.uint8))
    return t


def test_reader_matches_safetensors_library_and_raw_bytes(tmp_path):
    rng = np.random.default_rng(1)
    a32 = rng.standard_normal((6, 10)).astype(np.float32)
    bf = (rng.standard_normal((4, 8)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    e8 = rng.integers(0, 256, (5, 3), dtype=np.uint8)
    i8 = rng.integers(0, 256, (7, 16), dtype=np.uint8)
    f8 = rng.integers(0, 256, (3, 4), dtype=np.uint8)
    f8[f8 & 0x7F == 0x7F] = 0   # no NaN codes
    path = tmp_path / "model.safetensors"
    write_file(str(path), {"a": ("F32", a32.shape, a32), "b": ("BF16", bf.shape, bf), "s": ("F8_E8M0", e8.shape, e8),
                           "w": ("I8", i8.shape, i8), "f": ("F8_E4M3", f8.shape, f8)})
    ck = stio.Checkpoint(str(tmp_path))
    assert sorted(ck.names()) == ["a", "b", "f", "s", "w"] and "s" in ck and "x" not in ck
    assert ck.meta("s") == ("F8_E8M0", [5, 3]) and ck.meta("b") == ("BF16", [4, 8])
    assert np.array_equal(ck.get("a").numpy(), a32)
    assert ck.get("s").dtype == torch.uint8 and np.array_equal(ck.get("s").numpy(), e8)
    assert ck.get("w").dtype == torch.int8 and np.array_equal(ck.get("w").view(torch.uint8).numpy(), i8)
    assert ck.get("f").dtype == torch.float8_e4m3fn and np.array_equal(ck.get("f").view(torch.uint8).numpy(), f8)
    assert np.array_equal(ck.get("b").view(torch.int16).numpy().view(np.uint16), bf)
    assert np.array_equal(ck.get("w", rows=slice(2, 5)).view(torch.uint8).numpy(), i8[2:5])
    # the published reader agrees on the dtypes it knows
    pytest.importorskip("safetensors")
    from safetensors import safe_open
    try:
        with safe_open(str(path), framework="pt") as f:
            assert torch.equal(f.get_tensor("a"), ck.get("a"))
            assert torch.equal(f.get_tensor("b"), ck.get("b"))
            assert torch.equal(f.get_tensor("w"), ck.get("w"))
    except Exception as err:   # a library version that rejects the whole file for its F8_E8M0 entry
        if "E8M0" not in str(err) and "dtype" not in str(err).lower():
            raise


def test_written_views_stay_private(tmp_path):
    """A caller may write into a returned tensor: the pages become private to the process (copy-on-write), a new
    Checkpoint of the same file reads the original bytes, and the file is unchanged."""
    a32 = np.arange(24, dtype=np.float32).reshape(4, 6)
    path = tmp_path / "model.safetensors"
    write_file(str(path), {"a": ("F32", a32.shape, a32)})
    ck = stio.Checkpoint(str(tmp_path))
    t = ck.get("a")
    t.mul_(2.0)
    assert np.array_equal(t.numpy(), a32 * 2.0)
    assert np.array_equal(stio.Checkpoint(str(tmp_path)).get("a").numpy(), a32)
    assert a32.tobytes() in open(path, "rb").read()


def test_sharded_checkpoint_and_expert_stacking(tmp_path):
    rng = np.random.default_rng(2)
    E, H, I = 3, 256, 128
    t = _layer_tensors(rng, E, H, I)
    write_checkpoint(str(tmp_path), t, n_files=3, config={"n_activated_experts": 2})
    ck = stio.Checkpoint(str(tmp_path))
    assert ck.config()["n_activated_experts"] == 2
    ex = load.load_experts(ck, 0, "cpu", tiled=False)
    assert ex.w13.shape == (E, 2 * I, H // 2) and ex.s2.shape == (E, H, I // 32)
    for e in range(E):
        q = f"layers.0.ffn.experts.{e}."
        assert np.array_equal(ex.w13[e, :I].numpy(), t[q + "w1.weight"][2])
        assert np.array_equal(ex.w13[e, I:].numpy(), t[q + "w3.weight"][2])
        assert np.array_equal(ex.s13[e, I:].numpy(), t[q + "w3.scale"][2])
        assert np.array_equal(ex.w2[e].numpy(), t[q + "w2.weight"][2])
    tl = load.load_experts(ck, 0, "cpu", tiled=True)
    assert torch.equal(tl.w13, quant.tile_fp4(ex.w13)) and torch.equal(tl.s2, quant.tile_fp4_scales(ex.s2))


def test_fp8_block_dequant_closed_form():
    """dequant_fp8_block: E4M3 code value x 2^(block scale byte - 127), exact in bf16 for moderate scales."""
    from oracle import moe_oracle as O
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 256, (40, 70), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    sc = rng.integers(110, 140, (2, 3), dtype=np.uint8)
    got = load.dequant_fp8_block(torch.from_numpy(codes).view(torch.float8_e4m3fn), torch.from_numpy(sc))
    ref = O.e4m3_decode(codes) * np.repeat(np.repeat(O.e8m0_to_f32(sc), 32, 0)[:40], 32, 1)[:, :70]
    assert np.array_equal(got.float().numpy(), ref.astype(np.float32))
