"""The no-allocation decode entry point (dsv41_moe_experts_noalloc) through the C ABI: the same results as the
existing entry points (dsv41_moe_decode_up + dsv41_moe_down_sum with caller-owned workspaces, the one-launch down
projection also for 16 tokens), bit for bit, on two calls in a row, the second with a smaller input, so the second runs
over the scratch contents the first left."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _layer(E, H, I, seed):
    from dsv41_amd import moe
    g = torch.Generator(device=DEV).manual_seed(seed)
    w13 = torch.randint(0, 256, (E, 2 * I, H // 2), generator=g, dtype=torch.uint8, device=DEV)
    s13 = torch.randint(119, 124, (E, 2 * I, H // 32), generator=g, dtype=torch.uint8, device=DEV)
    w2 = torch.randint(0, 256, (E, H, I // 2), generator=g, dtype=torch.uint8, device=DEV)
    s2 = torch.randint(119, 124, (E, H, I // 32), generator=g, dtype=torch.uint8, device=DEV)
    return moe.ExpertWeights(w13, s13, w2, s2, tiled=True)


def _noalloc(ex, xq, k, limit, logits=None, eid=None, wt=None, ys=None):
    from dsv41_amd import _lib
    M, H = xq.shape
    y = torch.full((M, H), float("nan"), device=DEV)
    yb = torch.zeros(M, H, dtype=torch.bfloat16, device=DEV)
    eo = torch.full((M, k), -7, dtype=torch.int32, device=DEV)
    wo = torch.zeros(M, k, device=DEV)
    route = ((_lib.ptr(logits), ex.E, 1, 0, None, 1.0, 1.0, 2, 1, None, None) if logits is not None else
             (None, ex.E, 1, 0, None, 1.0, 1.0, 0, 0, _lib.ptr(eid), _lib.ptr(wt)))
    r = _lib.lib().dsv41_moe_experts_noalloc(*route, M, k, ex.E, _lib.ptr(xq), xq.stride(0), _lib.ptr(ex.w13), ex.w13.stride(0),
                                             _lib.ptr(ex.s13), ex.s13.stride(0), _lib.ptr(ex.w2), ex.w2.stride(0), _lib.ptr(ex.s2),
                                             ex.s2.stride(0), 1, H, ex.I, ctypes.c_float(limit), _lib.ptr(eo), _lib.ptr(wo), _lib.ptr(y), H,
                                             _lib.ptr(ys), H, _lib.ptr(yb), H, _lib.stream(DEV))
    assert r == 0, f"dsv41_moe_experts_noalloc returned {r}"
    return y, yb, eo, wo


def _existing(ex, xq, k, limit, logits=None, eid=None, wt=None, ys=None):
    from dsv41_amd import moe
    M, H = xq.shape
    eo = torch.full((M, k), -7, dtype=torch.int32, device=DEV)
    wo = torch.zeros(M, k, device=DEV)
    if logits is not None:
        ws = moe.decode_up(xq, ex, limit, k, logits=logits, gate=(None, 1.0, 1.0, "softmax", True), eid_out=eo, wt_out=wo)
    else:
        ws = moe.decode_up(xq, ex, limit, k, eid=eid, wt=wt, eid_out=eo, wt_out=wo)
    y = torch.empty(M, H, device=DEV)
    yb = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    moe.decode_down(ws, ex, ys=ys, out=yb, y32=y, split=False)
    return y, yb, eo, wo


def test_noalloc_matches_existing_entry_points():
    from dsv41_amd import quant
    E, H, I, k = 64, 7168, 1664, 8
    ex = _layer(E, H, I, 909)
    g = torch.Generator(device=DEV).manual_seed(910)
    # call 1: 16 tokens routed from logits inside the up launch, with a shared-expert term in the bf16 output
    M1 = 16
    xq1 = quant.fake_quant_fp8(torch.randn(M1, H, generator=g, device=DEV).to(torch.bfloat16))
    lg1 = torch.randn(M1, E, generator=g, device=DEV)
    ys1 = torch.randn(M1, H, generator=g, device=DEV).to(torch.bfloat16)
    got1 = _noalloc(ex, xq1, k, 10.0, logits=lg1, ys=ys1)
    ref1 = _existing(ex, xq1, k, 10.0, logits=lg1, ys=ys1)
    torch.cuda.synchronize()
    for a, b, name in zip(got1, ref1, ("y", "yb", "eid", "wt")):
        assert torch.equal(a, b), f"call 1 (M = 16): {name} differs"
    assert float(got1[0].abs().max()) > 0
    # call 2, smaller: one token with given routing (the scratch still holds call 1's 128 h rows)
    M2 = 1
    xq2 = quant.fake_quant_fp8(torch.randn(M2, H, generator=g, device=DEV).to(torch.bfloat16))
    eid2 = torch.tensor([[3, 60, 17, 9, 44, 1, 28, 51]], dtype=torch.int32, device=DEV)
    wt2 = torch.softmax(torch.randn(M2, k, generator=g, device=DEV), -1)
    got2 = _noalloc(ex, xq2, k, 10.0, eid=eid2, wt=wt2)
    ref2 = _existing(ex, xq2, k, 10.0, eid=eid2, wt=wt2)
    torch.cuda.synchronize()
    for a, b, name in zip(got2, ref2, ("y", "yb", "eid", "wt")):
        assert torch.equal(a, b), f"call 2 (M = 1): {name} differs"
    # and one token routed from logits, after both
    lg3 = torch.randn(1, E, generator=g, device=DEV)
    got3 = _noalloc(ex, xq2, k, 0.0, logits=lg3)
    ref3 = _existing(ex, xq2, k, 0.0, logits=lg3)
    torch.cuda.synchronize()
    for a, b, name in zip(got3, ref3, ("y", "yb", "eid", "wt")):
        assert torch.equal(a, b), f"call 3 (M = 1, logits): {name} differs"
