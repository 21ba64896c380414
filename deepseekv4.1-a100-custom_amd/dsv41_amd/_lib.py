"""ctypes binding of libdsv41_amd.so, the C ABI of the HIP kernels (declared in include/dsv41_amd.h).

This replaces the reference's libcuda/cubin launch layer (cukern.py:1-57): instead of loading code objects and
calling cuLaunchKernel, the library's extern "C" entry points launch their own kernels on the stream they are
given. Python passes raw device pointers, sizes and torch's current HIP stream, so every call is stream-ordered
and is recorded by torch.cuda.graph capture. Errors raise RuntimeError like cukern._check (cukern.py:19-21).

torch is imported first on purpose: the library's HIP runtime dependency (libamdhip64.so.7) then binds to the
runtime torch already loaded, so both share one device context and one set of streams.
"""
from __future__ import annotations

import ctypes
import os

import torch

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("DSV41_AMD_LIB", os.path.join(_PKG_ROOT, "lib", "libdsv41_amd.so"))

P = ctypes.c_void_p
I = ctypes.c_int
LL = ctypes.c_longlong
F = ctypes.c_float

# name -> argtypes (every entry returns int: 0 ok, < 0 invalid arguments, > 0 hipError_t)
SIGNATURES = {
    "dsv41_dequant_fp4": [P, P, LL, I, I, P, P],
    "dsv41_quant_fp8": [P, I, LL, I, LL, I, P, P, P, P],
    "dsv41_swiglu_quant": [P, I, LL, P, I, I, F, P, P, P, I, P],
    "dsv41_quant_fp8_split": [P, LL, I, LL, I, P, P, P, P, P, P],
    "dsv41_fp4_grouped_gemm": [P, LL, P, LL, I, I, I, P, LL, P, LL, I, P, P, P, P, P, I, P, I, P, LL, I, P, P, I, I, I, I, I, I, I, P],
    "dsv41_fp4_grouped_gemm_bf16": [P, LL, P, LL, I, I, I, P, LL, I, I, P, P, I, P, I, P, LL, I, P, P, I, I, I, I, I, I, I, P],
    "dsv41_moe_decode_up": [P, LL, I, LL, P, F, F, I, I, P, P, I, I, I, P, LL, P, LL, P, LL, I, I, I, F, P, LL, P, LL, P, P, P, P, P, P,
                            P, LL, I, P, LL, P, LL, P],
    "dsv41_moe_decode_up_pairs": [P, LL, I, LL, P, F, F, I, I, P, P, I, I, I, P, LL, P, LL, P, LL, I, I, I, F, P, LL, P, LL, P, P, P, P, P,
                                  P, P, LL, I, P, LL, P, LL, P],
    "dsv41_moe_down_sum": [P, LL, P, LL, I, I, I, P, LL, P, LL, I, P, P, P, I, I, P, LL, P, LL, P, LL, I, I, P, LL, P, LL, I, F, P, LL,
                           P, P, P, P, LL, P],
    "dsv41_moe_down_sum_split": [P, LL, P, LL, I, I, I, P, LL, P, LL, P, P, P, I, I, P, LL, P, LL, P, LL, I, I, P, P, P, P, LL, P],
    "dsv41_prefill_up": [P, LL, P, LL, I, P, LL, P, LL, I, I, I, I, P, P, I, P, P, F, P, LL, P, LL, P, P],
    "dsv41_prefill_down": [P, LL, P, LL, I, P, LL, P, LL, I, I, I, I, P, P, I, P, LL, P, P],
    "dsv41_group_order": [P, P, I, I, P, P],
    "dsv41_fp4_grouped_gemm_t128": [P, LL, P, LL, I, P, P, P, P, P, LL, P, LL, I, I, I, I, P, P, I, I, P, LL, P],
    "dsv41_rows_distinct": [P, I, P, I, P, P],
    "dsv41_fp4_grouped_gemm_scatter": [P, LL, P, LL, I, P, P, P, P, P, LL, P, LL, I, I, I, I, P, P, I, I, P, P, P, I, P, LL, I, P, LL, P],
    "dsv41_combine_pairs": [P, LL, P, I, I, I, P, LL, P, LL, P, LL, P],
    "dsv41_dense_gemv_bf16": [P, LL, I, I, I, P, LL, I, P, LL, P, LL, P],
    "dsv41_residual_rmsnorm_quant": [P, LL, P, LL, P, F, I, I, P, LL, P, LL, P],
    "dsv41_gate_topk": [P, LL, P, I, I, F, I, F, I, I, P, P, I, LL, P],
    "dsv41_router_logits_f32w": [P, LL, P, LL, I, I, I, P, P],
    "dsv41_fp8_gemm": [P, LL, I, P, LL, I, I, P, LL, I, I, P, LL, P, LL, P],
    "dsv41_dequant_fp8": [P, LL, I, P, LL, I, I, P, LL, P],
    "dsv41_hc_pre_norm_quant": [P, LL, I, P, LL, P, F, I, I, P, LL, P, LL, P, LL, P, LL, P],
    "dsv41_hc_post": [P, LL, P, LL, LL, I, P, LL, P, LL, P, LL, P, LL, I, I, P],
    "dsv41_router_logits": [P, LL, P, LL, P, F, P, LL, I, I, I, P, P, LL, P, LL, P],
    "dsv41_moe_dispatch": [P, P, I, I, I, I, P, P, P, P, P, P, P],
    "dsv41_moe_experts_noalloc": [P, LL, I, LL, P, F, F, I, I, P, P, I, I, I, P, LL, P, LL, P, LL, P, LL, P, LL, I, I, I, F, P, P, P, LL, P, LL,
                                  P, LL, P],
    "dsv41_selftest_mfma_scale": [P, P, P, P, P, I, I, P],
    "dsv41_selftest_mfma_rate": [I, I, I, P, P],
    "dsv41_selftest_stream": [P, LL, I, I, I, P, P],
    "dsv41_selftest_mfma_bf16": [P, P, P, P],
    "dsv41_selftest_fp8_cvt": [P, P, I, P, P],
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it was not built (there is no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP library {LIB_PATH} is not built: run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        _lib = L
    return _lib


def check(err: int, what: str) -> None:
    if err != 0:
        if err == -2:
            raise RuntimeError(f"{what}: the call needs more than the library's scratch array (status -2)")
        if err < 0:
            raise RuntimeError(f"{what}: invalid arguments (status {err})")
        raise RuntimeError(f"{what} failed with HIP error {err}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_cuda(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("dsv41_amd kernels run on the GPU only: got a CPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev
