"""The C ABI: the library loads (no GPU needed) and exports every entry point include/dsv41_amd.h declares,
with the Python binding's argument counts matching the header."""
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "dsv41_amd.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for m in re.finditer(r"\bint\s+(dsv41_\w+)\s*\(([^)]*)\)\s*;", src):
        out[m.group(1)] = len([a for a in m.group(2).split(",") if a.strip()])
    return out


def test_header_parses():
    d = declared()
    assert len(d) >= 10 and "dsv41_fp4_grouped_gemm" in d and "dsv41_moe_down_sum" in d


def test_library_exports_every_declared_symbol():
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (dsv41_\w+)", nm))
    for name, nargs in declared().items():
        assert name in exported, f"{name} declared but not exported"
        assert hasattr(L, name)
        assert name in _lib.SIGNATURES, f"{name} has no Python binding"
        assert len(_lib.SIGNATURES[name]) == nargs, f"{name}: binding has {len(_lib.SIGNATURES[name])} args, header {nargs}"
    assert exported == set(declared()), f"undeclared exports: {exported - set(declared())}"


def test_invalid_arguments_are_rejected_without_launch():
    """Argument checks run on the host before any launch: no GPU is touched."""
    import ctypes
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    assert L.dsv41_dequant_fp4(None, None, 16, 64, 0, None, None) == -1
    assert L.dsv41_quant_fp8(ctypes.c_void_p(16), 0, 4, 33, 33, 0, ctypes.c_void_p(16), None, None, None) == -1  # K % 32
    assert L.dsv41_moe_dispatch(ctypes.c_void_p(16), None, 8, 8, 1000, 64, *[ctypes.c_void_p(16)] * 5, None, None) == -1  # E > 512
    assert L.dsv41_dense_gemv_bf16(ctypes.c_void_p(16), 64, 0, 16, 64, ctypes.c_void_p(16), 64, 17, ctypes.c_void_p(16), 16, None, 0, None) == -1
    # decode down projection: h rows shorter than K (codes or scales), an output row stride below N
    p = ctypes.c_void_p(16)
    down = lambda ldh, ldhs, ldy: L.dsv41_moe_down_sum(p, 7168 * 832, p, 7168 * 52, 1, 7168, 1664, p, ldh, p, ldhs, 8, p, p, p, 8, 1,
                                                      p, ldy, None, 7168, None, 7168, 0, 384, None, 0, None, 0, 0, 0.0, None, 0, None, None, None,
                                                      None, 0, None)
    assert down(1600, 52, 7168) == -1
    assert down(1664, 51, 7168) == -1
    assert down(1664, 52, 7000) == -1


def test_bound_checks_reject_oversized_shapes_without_launch():
    """Host-side bounds of the grouped GEMM (an N or K larger than one expert's bytes), the decode up projection (h rows
    narrower than I) and the decode down projection (a zero row beyond the kernel's 16-bit pair table): -1, nothing
    launched (the pointers are never dereferenced)."""
    import ctypes
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    N, K = 3328, 7168
    we, se = N * K // 2, N * K // 32

    def grouped(n, k, stride_we, stride_se, x_rows=1, n_pairs=8, out_rows=8, shard_n=384, lo=(None, None, None)):
        return L.dsv41_fp4_grouped_gemm(p, stride_we, p, stride_se, 1, n, k, p, k, p, k // 32, x_rows, *lo, p, p, 8, p, n_pairs, p, n,
                                        out_rows, None, None, 0, 1, 0, shard_n, 0, 0, 1 << 30, None)
    assert grouped(2 * N, K, we, se) == -1           # N rows past one expert's weight bytes
    assert grouped(N, 2 * K, we, 2 * se) == -1       # K past the weight bytes
    assert grouped(N, K, we, se - 1) == -1           # scales shorter than N K / 32
    assert grouped(N, K, we, se, x_rows=-1) == -1
    assert grouped(N, K, we, se, n_pairs=-1) == -1
    assert grouped(N, K, we, se, out_rows=-1) == -1
    assert grouped(N, K, we, se, shard_n=-1) == -1
    assert grouped(N, K, we, se, n_pairs=0) == 0     # nothing to do: returns before any launch
    # the second FP8 term: codes and scales together (its flag optional, not without them), 16-byte aligned
    assert grouped(N, K, we, se, lo=(p, None, p)) == -1
    assert grouped(N, K, we, se, lo=(p, None, None)) == -1
    assert grouped(N, K, we, se, lo=(None, p, p)) == -1
    assert grouped(N, K, we, se, lo=(None, None, p)) == -1
    assert grouped(N, K, we, se, lo=(ctypes.c_void_p(24), p, p)) == -1
    assert grouped(N, K, we, se, lo=(p, p, p), n_pairs=0) == 0
    # the split quantiser: K % 32, row stride % 8, alignment of x and of the code outputs, every output given
    q = ctypes.c_void_p(32)
    assert L.dsv41_quant_fp8_split(q, 4, 48, 48, 0, q, q, q, q, q, None) == -1
    assert L.dsv41_quant_fp8_split(q, 4, 64, 68, 0, q, q, q, q, q, None) == -1
    assert L.dsv41_quant_fp8_split(ctypes.c_void_p(40), 4, 64, 64, 0, q, q, q, q, q, None) == -1
    assert L.dsv41_quant_fp8_split(q, 4, 64, 64, 0, q, q, ctypes.c_void_p(40), q, q, None) == -1

    H, I = 7168, 1664

    def up(ldhc, ldhs):
        return L.dsv41_moe_decode_up(None, 0, 1, 0, None, 1.0, 1.0, 2, 1, p, p, 1, 8, 384, p, H, p, 2 * I * H // 2, p, 2 * I * H // 32,
                                     1, H, I, ctypes.c_float(10.0), p, ldhc, p, ldhs, None, None, p, p, p, p, None, 0, 0, None, 0, None, 0, None)
    assert up(I - 32, I // 32) == -1
    assert up(I, I // 32 - 1) == -1

    # the pair-by-pair entry: the same checks, and its one-row staging needs H / 16 <= 448 (H = 8192 is too wide)
    def up_pairs(ldhc, ldhs, M=2, H_=H):
        return L.dsv41_moe_decode_up_pairs(None, 0, 1, 0, None, 1.0, 1.0, 2, 1, p, p, M, 8, 384, p, H_, p, 2 * I * H_ // 2, p,
                                           2 * I * H_ // 32, 1, H_, I, ctypes.c_float(10.0), p, ldhc, p, ldhs, None, None, p, p, p, p,
                                           None, 0, 0, None, 0, None, 0, None)
    assert up_pairs(I - 32, I // 32) == -1
    assert up_pairs(I, I // 32, M=17) == -1
    assert up_pairs(I, I // 32, H_=8192) == -1

    def down(zero_row, Ws2=None, M=1, ys=None):
        return L.dsv41_moe_down_sum(p, H * (I // 2), p, H * (I // 32), 1, H, I, p, I, p, I // 32, zero_row, p, p, p, 8, M,
                                    p, H, ys, H, None, H, 0, 384, p if Ws2 else None, 2 * I, Ws2, I, 0, ctypes.c_float(10.0), None, H, None, None, None,
                                    None, 0, None)
    assert down(32768) == -1
    assert down(-1) == -1
    # the fused shared expert: not together with a given ys, and only while its M h_s rows fit (M I / 32 <= 128)
    assert down(8, Ws2=p, ys=p) == -1
    assert down(8, Ws2=p, M=3) == -1


def test_down_split_rejects_invalid_calls_without_launch():
    """dsv41_moe_down_sum_split: -1 on the host, nothing launched, for a workspace smaller than its runs' partial sums,
    an output row count not a multiple of 128, K past 2048, more than 16 tokens or a misaligned workspace."""
    import ctypes
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    H, I = 7168, 1664

    def split(M=16, N=H, K=I, part_floats=None, part=p):
        P = M * 8
        q = max(1, min(32 - M, (P + 7) // 8))
        need = -(-P // q) * M * N
        return L.dsv41_moe_down_sum_split(p, N * (K // 2), p, N * (K // 32), 1, N, K, p, K, p, K // 32, p, p, p, P, M, p, N, None, N,
                                          None, N, 0, 384, None, None, None, part, need if part_floats is None else part_floats, None)
    assert split(part_floats=8 * 16 * H - 1) == -1   # 8 runs of 16 rows at M = 16
    assert split(M=8, part_floats=8 * 8 * H - 1) == -1
    assert split(N=H - 64) == -1
    assert split(K=2176) == -1
    assert split(M=17) == -1
    assert split(part=ctypes.c_void_p(24)) == -1


def test_grouped_scatter_rejects_invalid_calls_without_launch():
    """dsv41_fp4_grouped_gemm_scatter: -1 on the host, nothing launched, for a missing output-row table, an accum flag
    other than 0 / 1, N not a multiple of 256, K below 384, a misaligned output, a row stride below N, a missing or
    misaligned workspace or more groups than one launch's grid rows; 0 with no pairs or no output rows."""
    import ctypes
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    N, K = 512, 768

    def call(n=N, k=K, row_out=p, accum=0, out=p, ldo=N, n_pairs=8, out_rows=8, y2=p, G=4, lo=(None, None, None)):
        return L.dsv41_fp4_grouped_gemm_scatter(p, k, p, k // 32, 8, *lo, p, p, n * (k // 2), p, n * (k // 32), 1, 4, n, k, p, p, G,
                                                n_pairs, row_out, p, None, accum, out, ldo, out_rows, y2, n, None)
    assert call(row_out=None) == -1
    assert call(accum=2) == -1
    assert call(n=N + 128) == -1
    assert call(k=256) == -1
    assert call(out=ctypes.c_void_p(24)) == -1
    assert call(ldo=N - 4) == -1
    assert call(y2=None) == -1
    assert call(y2=ctypes.c_void_p(20)) == -1
    assert call(G=65536) == -1
    assert call(lo=(None, None, p)) == -1
    assert call(lo=(p, None, p)) == -1
    assert call(lo=(ctypes.c_void_p(24), p, p)) == -1
    assert call(lo=(ctypes.c_void_p(48), ctypes.c_void_p(50), p)) == -1   # lo scales not 4-byte aligned
    assert L.dsv41_fp4_grouped_gemm_t128(p, K, p, K // 32, 8, p, None, p, p, p, N * (K // 2), p, N * (K // 32), 1, 4, N, K, p, p, 4, 8,
                                         p, N, None) == -1
    assert L.dsv41_rows_distinct(None, 4, None, 4, p, None) == -1
    assert L.dsv41_rows_distinct(p, -1, None, 4, p, None) == -1
    assert call(n_pairs=0) == 0
    assert call(out_rows=0) == 0


def test_noalloc_rejects_calls_beyond_its_scratch():
    """dsv41_moe_experts_noalloc returns -2 (nothing launched, no GPU touched) for a call whose h rows exceed its 2 MiB
    array, and -1 for invalid arguments."""
    import ctypes
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    H = 7168

    def call(M, topk, I, stride_w2=None):
        sw2 = H * (I // 2) if stride_w2 is None else stride_w2
        return L.dsv41_moe_experts_noalloc(None, 0, 1, 0, None, 1.0, 1.0, 0, 0, p, p, M, topk, 512, p, H, p, 2 * I * H // 2, p,
                                           2 * I * H // 32, p, sw2, p, H * (I // 32), 1, H, I, ctypes.c_float(10.0), None, None, p, H,
                                           None, H, None, H, None)
    assert call(16, 16, 8192) == -2            # 257 rows of 8448 bytes > 2 MiB
    assert call(16, 8, 1664, stride_w2=100) == -1
    assert call(17, 8, 1664) == -1
    assert call(16, 8, 1600) == -1             # I % 128
