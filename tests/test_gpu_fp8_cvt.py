"""The gfx950 FP8 conversion instructions (v_cvt_pk_fp8_f32, v_cvt_f32_fp8) against the bit-arithmetic E4M3 rounding
the kernels were built on (quant.py:45-54: clamp to +-448, round to nearest even on the float8_e4m3fn grid): every
bf16 value, every rounding midpoint of the grid with its fp32 neighbours, and random fp32 inputs at random scales,
through dsv41_selftest_fp8_cvt. The hardware forms may replace the arithmetic ones only where these agree bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _run(v: np.ndarray, e: np.ndarray) -> np.ndarray:
    from dsv41_amd import _lib as L
    dev = torch.device("cuda:0")
    tv = torch.from_numpy(np.ascontiguousarray(v.astype(np.float32))).to(dev)
    te = torch.from_numpy(np.ascontiguousarray(e.astype(np.int32))).to(dev)
    out = torch.empty(v.size * 5, dtype=torch.int32, device=dev)
    L.call("dsv41_selftest_fp8_cvt", L.ptr(tv), L.ptr(te), int(v.size), L.ptr(out), L.stream(dev))
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32).reshape(-1, 5)


def _check(v, e, what):
    o = _run(v, e)
    for col, name in ((1, "hw code (low half)"), (2, "hw code (high half)")):
        bad = np.nonzero(o[:, 0] != o[:, col])[0]
        assert bad.size == 0, (f"{what}: {name} differs at {bad.size} inputs, e.g. v={v[bad[:4]]!r} e={e[bad[:4]]!r} "
                               f"sw={o[bad[:4], 0]} hw={o[bad[:4], col]}")
    bad = np.nonzero(o[:, 3] != o[:, 4])[0]
    assert bad.size == 0, f"{what}: decoded values differ at {bad.size} inputs, e.g. codes {o[bad[:4], 0]}"
    return o


def _grid():
    """The non-negative float8_e4m3fn grid (codes 0 .. 0x7E) as float64."""
    c = np.arange(0x7F)
    ex, m = c >> 3, c & 7
    return np.where(ex == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (ex - 7.0))


def test_every_bf16_value():
    bits = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    for e in (0, -21, -9, 3, 8, 20, 120):
        o = _check(bits, np.full(bits.size, e), f"bf16 at e={e}")
    # known codes at e = 0: 448 -> 0x7E, 2^-9 -> 0x01, -0.0 -> 0x80, 1.0 -> 0x38, 1000 -> 0x7E (clamped)
    o = _run(np.array([448.0, 2.0 ** -9, -0.0, 1.0, 1000.0, -1000.0], np.float32), np.zeros(6))
    assert list(o[:, 0]) == [0x7E, 0x01, 0x80, 0x38, 0x7E, 0xFE]


def test_rounding_midpoints_and_neighbours():
    g = _grid()
    mid = ((g[:-1] + g[1:]) / 2).astype(np.float32)           # exact in fp32
    assert np.array_equal(mid.astype(np.float64), (g[:-1] + g[1:]) / 2)
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(-np.inf))
    v = np.concatenate([mid, up, dn, g.astype(np.float32), np.float32(448.0) + np.float32(16.0) * np.arange(4, dtype=np.float32)])
    v = np.concatenate([v, -v])
    for e in (0, 5, -17):
        _check(v * np.float32(2.0 ** e), np.full(v.size, e), f"midpoints at e={e}")


def test_random_fp32_at_random_scales():
    rng = np.random.default_rng(11)
    n = 1 << 21
    raw = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)   # every class, NaN and inf too
    _check(raw, rng.integers(-126, 121, n), "random bit patterns")
    e = rng.integers(-126, 119, n)
    inr = (rng.uniform(-480.0, 480.0, n) * 2.0 ** e.astype(np.float64)).astype(np.float32)   # in and just past range
    _check(inr, e, "in-range values")
    sub = rng.uniform(-2.0 ** -5, 2.0 ** -5, n).astype(np.float32)                          # the E4M3 subnormal range
    _check(sub, np.zeros(n), "subnormal range")
