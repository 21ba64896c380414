"""Write the golden fixtures under tests/golden/ by running the reference's own `dsv41/quant.py` on CPU.

Only `quant.py` is imported (it needs `os` and `torch` only, quant.py:10-12); nothing else from the
reference is loaded. The output is data: inputs and the reference's outputs, saved with numpy
(`allow_pickle=False`). The fixtures pin the parts of the oracle that no closed form fixes:
torch's exp2/bf16/float8 bit patterns at the edges (scale byte 0 and 255, NaN, -0.0, E4M3 ties).

Usage (in a container that has /root/reference):  python tests/golden/make_golden.py
"""
import importlib.util
import os
import sys

import numpy as np
import torch

REF_QUANT = os.environ.get("DSV41_REF_QUANT", "/root/reference/dsv41/quant.py")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")


def load_ref_quant():
    os.environ["DSV41_COMPILE"] = "0"
    spec = importlib.util.spec_from_file_location("ref_quant", REF_QUANT)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main():
    q = load_ref_quant()
    out = {}

    # 1. dequant_fp4 over every (code, scale byte): 256 rows (one per scale byte), 32 codes per row
    #    (16 packed bytes: low nibbles 0..15, high nibbles 15..0), quant.py:106-110
    lo = np.arange(16, dtype=np.uint8)
    hi = (15 - np.arange(16)).astype(np.uint8)
    row = (lo | (hi << 4)).astype(np.uint8)
    packed = np.tile(row, (256, 1))
    scale = np.arange(256, dtype=np.uint8).reshape(256, 1)
    deq = q.dequant_fp4(torch.from_numpy(packed), torch.from_numpy(scale))
    out["deq_all_packed"] = packed
    out["deq_all_scale"] = scale
    out["deq_all_bf16"] = bf16_bits(deq)

    # 2. dequant_fp4 + the tiled layout on seeded random experts (the kernels' realistic input)
    g = torch.Generator().manual_seed(1234)
    E, N, K = 2, 32, 256
    w = torch.randint(0, 256, (E, N, K // 2), generator=g, dtype=torch.uint8)
    s = torch.randint(110, 135, (E, N, K // 32), generator=g, dtype=torch.uint8)
    out["rand_w"] = w.numpy()
    out["rand_s"] = s.numpy()
    out["rand_deq_bf16"] = np.stack([bf16_bits(q.dequant_fp4(w[e], s[e])) for e in range(E)])
    out["rand_w_tiled"] = q.tile_fp4(w).numpy()
    out["rand_s_tiled"] = q.tile_fp4_scales(s).numpy()

    # 3. fake_quant_fp8 / quant_fp8 on bf16 and fp32 inputs, with edge groups, quant.py:45-64
    x = torch.randn(4, 7168, generator=g) * 3.0
    x[0, :32] = 0.0                                   # all-zero group (amax clamp 1e-4)
    x[0, 32:64] = torch.linspace(-5e-5, 5e-5, 32)    # amax below 1e-4
    x[0, 64:96] = -0.0                                # negative zeros
    x[1, :32] = 448.0 * torch.linspace(-1, 1, 32)     # amax exactly 448 -> scale 1
    # E4M3 ties: values halfway between neighbours at scale 1 (amax = 448 in the group)
    mids = torch.tensor([1.0625, 1.1875, 3.25, 3.75, 17.0, 19.0, 0.0068359375, 0.0029296875, 300.0, 440.0], dtype=torch.float32)
    x[1, 32:64] = 0.0
    x[1, 32] = 448.0
    x[1, 33:33 + mids.numel()] = mids
    x[2, :32] = 1e4 * torch.randn(32, generator=g)  # large
    x[3, :32] = 1e-3 * torch.randn(32, generator=g)  # small
    xb = x.to(torch.bfloat16)
    out["fq8_in_bf16"] = bf16_bits(xb)
    out["fq8_out_bf16"] = bf16_bits(q.fake_quant_fp8(xb, 32))
    qv, qs = q.quant_fp8(xb, 32)
    out["qfp8_codes_bf16in"] = qv.view(torch.uint8).numpy().copy()
    out["qfp8_scales_bf16in"] = qs.numpy().copy()
    out["fq8_in_f32"] = x.numpy().copy()
    out["fq8_out_f32"] = q.fake_quant_fp8(x, 32).numpy().copy()

    # 4. ceil_log2 / pow2_scale on awkward inputs, quant.py:34-42
    a = torch.tensor([1e-4, 2.2e-7, 0.5, 1.0, 1.5, 2.0, 447.9, 448.0, 448.1, 3.0e38, 1.17549435e-38, 2.0**-127], dtype=torch.float32)
    out["cl2_in"] = a.numpy()
    out["cl2_out"] = q.ceil_log2(a).numpy().astype(np.int32)
    out["pow2_in"] = a.numpy()
    out["pow2_out"] = q.pow2_scale(a.clamp_min(1e-4), q.FP8_MAX).numpy()

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays) with torch {torch.__version__}")


if __name__ == "__main__":
    sys.exit(main())
