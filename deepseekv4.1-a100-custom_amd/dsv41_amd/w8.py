"""Dense weights kept as FP8 on the device (E4M3 bytes + one E8M0 byte per 32 x 32 block) instead of bf16, with the
call surface of the reference's dsv41/w8.py (W8, linear_w, oproj_a, permute_k / tile helpers) and its
model.linear_fp8 (model.py:55-58).

Up to 64 rows run through dsv41_fp8_gemm (csrc/dense_fp8.hip): the weights are streamed once as FP8 (half the bytes
of bf16), decoded in registers to bf16 MFMA operands with their block scale and accumulated in fp32, which gives the
same numbers as the bf16 product up to the order of the fp32 additions (w8.py:1-7). More rows (prefill) dequantize
to a bf16 matrix, or use the kept bf16 copy, and call the library GEMM, as the reference does past its kernels'
row limits (w8.py:102-113).

Stored byte order: the MFMA fragments of the HIP kernel take k in natural order, so permute_k is the identity
(PERM_K is kept for drop-in code that indexes it). tile() is this build's 1 KiB tile order
[N/16][K/64][4][16 rows][16 B]: lane l of a wave reads bytes 16 l .. 16 l + 15 of a tile (rows l % 16, k 16 (l / 16)
.. +15), so one wave-load is one contiguous 1 KiB block.
"""
from __future__ import annotations

import os

import torch
import torch.nn.functional as F

from . import hipkern
from .fused import fake_quant_fp8
from .quant import dequant_fp8_block

ENABLED = os.environ.get("DSV41_W8", "1") == "1"
MAX_TC_ROWS = hipkern.FP8_ROWS  # rows one FP8 launch handles (weights read once); more rows use the bf16 GEMM

PERM_K = list(range(16))
_INV_PERM_K = list(range(16))


def permute_k(w8: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K] natural k order -> the in-memory order of the FP8 kernel (natural: a copy)."""
    N, K = w8.shape
    assert K % 16 == 0
    return w8.clone(memory_format=torch.contiguous_format)


def unpermute_k(w8: torch.Tensor) -> torch.Tensor:
    return permute_k(w8)


TILED = os.environ.get("DSV41_FP8_TILED", "1") == "1"


def tile(w8: torch.Tensor) -> torch.Tensor:
    """[N, K] row-major -> [N/16][K/64][4][16 rows][16 B] (same shape [N, K], contiguous)."""
    N, K = w8.shape
    assert N % 16 == 0 and K % 64 == 0
    return w8.reshape(N // 16, 16, K // 64, 4, 16).permute(0, 2, 3, 1, 4).reshape(N, K).contiguous()


def untile(w8: torch.Tensor) -> torch.Tensor:
    N, K = w8.shape
    return w8.reshape(N // 16, K // 64, 4, 16, 16).permute(0, 3, 1, 2, 4).reshape(N, K).contiguous()


# Environment switches with the reference's names and defaults (w8.py:51-53). DSV41_W8_BF16_COPY: whether loaders call
# keep_bf16(); DSV41_W8_BF16_ROWS: the row count at which linear_w / oproj_a switch from the FP8 launch to the library
# GEMM on a kept copy (here one past the launch's row limit: the FP8 launch is faster up to it); DSV41_W8_BF16_RESERVE_GB:
# device memory a loader leaves free when it keeps copies.
BF16_COPY = os.environ.get("DSV41_W8_BF16_COPY", "1") == "1"
BF16_ROWS = int(os.environ.get("DSV41_W8_BF16_ROWS", str(MAX_TC_ROWS + 1)))
BF16_RESERVE_GB = float(os.environ.get("DSV41_W8_BF16_RESERVE_GB", "4"))


class W8:
    __slots__ = ("w8", "s8", "shape", "device", "tiled", "bf16w")

    def __init__(self, w8: torch.Tensor, s8: torch.Tensor, permuted: bool = False, tiled: bool | None = None):
        """w8: uint8 E4M3 bytes [N, K]; s8: E8M0 [ceil(N/32), K/32] (w8.py:57-76). Bytes given in natural order are
        stored in the 1 KiB tile order when N % 16 == 0 and K % 64 == 0; permuted=True takes w8 as already stored,
        tiled or not as `tiled` says."""
        assert w8.dtype == torch.uint8 and s8.dtype == torch.uint8 and w8.dim() == 2
        N, K = w8.shape
        if permuted:
            self.w8 = w8.contiguous()
            self.tiled = bool(tiled)
        else:
            self.tiled = TILED and N % 16 == 0 and K % 64 == 0
            self.w8 = tile(w8) if self.tiled else w8.contiguous()
        self.s8 = s8.contiguous()
        self.shape = (N, K)
        self.device = w8.device
        self.bf16w = None

    @property
    def dtype(self):
        return torch.bfloat16

    def bf16(self) -> torch.Tensor:
        """The dequantized weights, bf16 [N, K] (dequant_fp8_block of the natural-order bytes)."""
        if self.bf16w is not None:
            return self.bf16w
        return dequant_fp8_block(self.w8, self.s8, tiled=self.tiled)

    def keep_bf16(self) -> "W8":
        """Dequantise once and hold the bf16 result beside the FP8 bytes (three times the memory in all); linear_w
        and oproj_a use it from BF16_ROWS rows on (w8.py:84-89)."""
        if self.bf16w is None:
            self.bf16w = self.bf16().contiguous()
        return self

    def natural(self) -> torch.Tensor:
        """The E4M3 bytes in natural row-major order [N, K]."""
        return untile(self.w8) if self.tiled else self.w8

    @staticmethod
    def cat(ws: list) -> "W8":
        """One W8 whose rows are the given weights' rows in order (w8.py:91-95). Each part's row count must be a
        multiple of 32: a 32 x 32 scale block, and so a 16-row tile, never straddles two parts."""
        assert all(w.shape[0] % 32 == 0 for w in ws) and len({w.tiled for w in ws}) == 1
        return W8(torch.cat([w.w8 for w in ws], dim=0), torch.cat([w.s8 for w in ws], dim=0), permuted=True, tiled=ws[0].tiled)


def linear_w(x: torch.Tensor, w) -> torch.Tensor:
    """y = x . w^T with bf16 activations and a bf16 result, for w a plain bf16 tensor (library GEMM) or a W8
    (w8.py:102-113): up to MAX_TC_ROWS rows the FP8 launch reads the E4M3 bytes directly, beyond that (or from
    BF16_ROWS rows with a kept copy) the library GEMM runs on the dequantised weights."""
    if not isinstance(w, W8):
        return F.linear(x, w)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[0] <= MAX_TC_ROWS and (w.bf16w is None or x2.shape[0] < BF16_ROWS):
        y = hipkern.fp8_gemm_tc(x2.contiguous().to(torch.bfloat16), w.w8, w.s8, tiled=w.tiled)
    else:
        y = F.linear(x2.to(torch.bfloat16), w.bf16())
    return y.view(*lead, w.shape[0])


def linear_fp8(x: torch.Tensor, w) -> torch.Tensor:
    """model.linear_fp8 (model.py:55-58): the activations are rounded to FP8 (per-32 power-of-two scale) first."""
    return linear_w(fake_quant_fp8(x, 32), w)


def oproj_a(o: torch.Tensor, wo_a, n_groups: int, rank: int) -> torch.Tensor:
    """Grouped output projection (w8.py:116-124): o [b, s, g, d], wo_a [g * rank, d]; output columns
    g' * rank .. (g' + 1) * rank - 1 are o[..., g', :] times rows g' * rank .. of wo_a, so the result is [b, s, g * rank]
    (a block-diagonal weight applied without materialising its zero blocks)."""
    b, s, g, d = o.shape
    if isinstance(wo_a, W8) and b * s <= MAX_TC_ROWS and (wo_a.bf16w is None or b * s < BF16_ROWS):
        y = hipkern.fp8_gemm_tc(o.reshape(b * s * g, d).contiguous().to(torch.bfloat16), wo_a.w8, wo_a.s8, group_cols=rank,
                                tiled=wo_a.tiled)
        return y.view(b, s, -1)
    wb = wo_a.bf16() if isinstance(wo_a, W8) else wo_a
    # one bmm per group with contiguous operands: [g, b*s, d] @ [g, d, rank]
    og = o.reshape(b * s, g, d).transpose(0, 1).contiguous()
    wg = wb.view(g, rank, d).transpose(1, 2).contiguous()
    return torch.bmm(og, wg).transpose(0, 1).reshape(b, s, g * rank)
