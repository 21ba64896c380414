"""The layer oracle against the reference's own CPU MoE library (dsv41/cpu/moe_cpu.cpp compiled from the
reference sources into oracle/_ref by oracle/Makefile). bf16 mode (cpumoe_set_int8(0)) computes the same
math as the GPU path with bf16 dot products (moe_cpu.cpp:177-205, 357-377, 386-503), so it pins the
rounding points of the layer: routing weight folded into h, bf16 cast, per-32 FP8 fake quant, w2.
Intermediate sizes are multiples of 256 here: the reference library skips the tail columns otherwise
(moe_cpu.cpp:444), which test_reference_tail_bug documents."""
import ctypes
import os

import numpy as np
import pytest

from oracle import moe_oracle as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "oracle", "_ref", "libmoe_cpu_ref.so")


def _cpu_has_isa():
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512_vnni", "avx512vbmi", "avx512_bf16"))


pytestmark = pytest.mark.skipif(not (os.path.exists(LIB) and _cpu_has_isa()),
                                reason="oracle/_ref not built (make -C oracle) or host lacks the AVX-512 ISA it needs")


@pytest.fixture(scope="module")
def ref():
    L = ctypes.CDLL(LIB)
    L.cpumoe_init(4, 4)
    L.cpumoe_forward.restype = ctypes.c_int
    return L


def run_ref(L, mode, w13, s13, w2, s2, ids, wts, xq_bits, K, inter, dim, limit):
    L.cpumoe_set_int8(mode)
    E = len(ids)
    P = ctypes.c_void_p * E
    keep = [np.ascontiguousarray(a[e]) for a in (w13, s13, w2, s2) for e in ids]
    ptr = lambda arr: ctypes.c_void_p(arr.ctypes.data)
    p13 = P(*[keep[i].ctypes.data for i in range(0, E)])
    ps13 = P(*[keep[i].ctypes.data for i in range(E, 2 * E)])
    p2 = P(*[keep[i].ctypes.data for i in range(2 * E, 3 * E)])
    ps2 = P(*[keep[i].ctypes.data for i in range(3 * E, 4 * E)])
    x = np.ascontiguousarray(xq_bits, np.uint16)
    wv = (ctypes.c_float * E)(*wts)
    out = np.zeros(dim, np.float32)
    gu = np.zeros(16 * 2 * inter, np.float32)
    h = np.zeros(16 * inter, np.uint16)
    r = L.cpumoe_forward(p13, ps13, p2, ps2, E, ptr(x), wv, ptr(out), K, inter, dim, ctypes.c_float(limit), ptr(gu), ptr(h))
    assert r == 0
    return out, gu[:E * 2 * inter].reshape(E, 2 * inter), h[:E * inter].reshape(E, inter)


def make_layer(seed, E, inter, dim):
    rng = np.random.default_rng(seed)
    w13 = rng.integers(0, 256, (E, 2 * inter, dim // 2), dtype=np.uint8)
    s13 = rng.integers(118, 128, (E, 2 * inter, dim // 32), dtype=np.uint8)
    w2 = rng.integers(0, 256, (E, dim, inter // 2), dtype=np.uint8)
    s2 = rng.integers(118, 128, (E, dim, inter // 32), dtype=np.uint8)
    x = O.bf16_round(rng.standard_normal((1, dim)).astype(np.float32) * 2)
    xq = O.fake_quant_fp8(x)
    return w13, s13, w2, s2, xq


@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_layer_oracle_matches_reference_cpu_bf16(ref, limit):
    E, inter, dim = 12, 256, 512
    w13, s13, w2, s2, xq = make_layer(1, E, inter, dim)
    ids = [0, 2, 3, 5, 9, 11]
    wts = [0.3, 0.2, 0.15, 0.15, 0.1, 0.1]
    out, gu, h = run_ref(ref, 0, w13, s13, w2, s2, ids, wts, O.f32_to_bf16_bits(xq[0]), dim, inter, dim, limit)
    y = O.moe_layer_routed(xq, np.array([ids]), np.array([wts], np.float32), w13, s13, w2, s2, inter, limit)[0]
    # stage 1: gu agrees to fp32 summation order
    for j, e in enumerate(ids):
        g_ref = (O.deq64(w13[e], s13[e]) @ xq[0].astype(np.float64)).astype(np.float32)
        assert O.rel_l2(gu[j], g_ref) < 1e-6
        # stage 2: h = fq8(bf16(w * silu * u)); identical except where fp32 order flips a rounding
        h_or = O.swiglu_quant(g_ref.reshape(1, -1), np.array([wts[j]], np.float32), inter, limit)[0]
        h_ref = O.bf16_bits_to_f32(h[j])
        assert (h_ref == h_or).mean() > 0.99
    # the layer
    assert O.rel_l2(out, y) < 2e-4
    assert O.max_abs_over_rms(out, y) < 1e-2


def test_reference_int8_mode_is_close(ref):
    """The reference's default W4A8 mode (int8 activations, moe_cpu.cpp:237-275) is an approximation of the
    same layer; the reference publishes no threshold (test_cpumoe.py:31). Recorded here for the baseline."""
    E, inter, dim = 12, 256, 512
    w13, s13, w2, s2, xq = make_layer(2, E, inter, dim)
    ids, wts = [1, 4, 7, 8, 10, 11], [0.25, 0.25, 0.2, 0.1, 0.1, 0.1]
    out, _, _ = run_ref(ref, 2, w13, s13, w2, s2, ids, wts, O.f32_to_bf16_bits(xq[0]), dim, inter, dim, 10.0)
    y = O.moe_layer_routed(xq, np.array([ids]), np.array([wts], np.float32), w13, s13, w2, s2, inter, 10.0)[0]
    assert O.rel_l2(out, y) < 3e-2


def test_reference_tail_bug(ref):
    """At I = 1664 (not a multiple of 256) the reference skips h columns 1536..1663 in stage 2
    (moe_cpu.cpp:444): the oracle (and the GPU path) include them, so the two differ by those columns."""
    E, inter, dim = 3, 320, 256
    w13, s13, w2, s2, xq = make_layer(3, E, inter, dim)
    ids, wts = [0, 1, 2], [0.5, 0.3, 0.2]
    out, _, h = run_ref(ref, 0, w13, s13, w2, s2, ids, wts, O.f32_to_bf16_bits(xq[0]), dim, inter, dim, 10.0)
    y = O.moe_layer_routed(xq, np.array([ids]), np.array([wts], np.float32), w13, s13, w2, s2, inter, 10.0)[0]
    assert np.all(h[:, 256:] == 0) and np.abs(h[:, :256]).max() > 0   # tail of h never written
    assert O.rel_l2(out, y) > 0.1
