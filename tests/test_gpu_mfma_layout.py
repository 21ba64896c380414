"""The lane layouts the kernels assume for the gfx950 matrix instructions, checked on random operands against a
CPU evaluation (an in-bounds check of the compiler builtins' lane layout). g = lane / 16:

  block-scaled 16x16x128, A = E2M1: lane l holds row l%16, k [32g, 32g+32) (16 bytes, low nibble first);
  B = E4M3: lane l holds column l%16, bytes 0-15 = k [16g, +16), bytes 16-31 = k [64+16g, +16);
  scales: byte 0 of lane l's register scales 32-k block g of row (A) / column (B) l%16;
  result: lane l holds D[4g + i][l%16], i = 0..3.
  bf16 16x16x32: lane l holds 8 consecutive k of row/column l%16, k-block g; same result layout.

If an assumption fails, one-hot probes and alternative scale mappings are printed before the assertion."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _lib():
    from dsv41_amd import _lib
    return _lib


def run_scale(a, b, sa, sb, fa=4, fb=0):
    L = _lib()
    dev = torch.device("cuda:0")
    ta = torch.from_numpy(np.ascontiguousarray(a.view(np.int32))).to(dev)
    tb = torch.from_numpy(np.ascontiguousarray(b.view(np.int32))).to(dev)
    tsa = torch.from_numpy(sa.astype(np.int32)).to(dev)
    tsb = torch.from_numpy(sb.astype(np.int32)).to(dev)
    c = torch.zeros(64, 4, dtype=torch.float32, device=dev)
    L.call("dsv41_selftest_mfma_scale", L.ptr(ta), L.ptr(tb), L.ptr(tsa), L.ptr(tsb), L.ptr(c), fa, fb, L.stream(dev))
    torch.cuda.synchronize()
    return c.cpu().numpy()


def b_k(g, j):
    """k of byte j of a B (E4M3) lane in lane group g."""
    return 16 * g + j if j < 16 else 64 + 16 * g + (j - 16)


def expected_scale(a, b, sa, sb, scale_map="block"):
    """a: uint8 [64][32] (first 16 bytes used: E2M1 pairs), b: uint8 [64][32] E4M3.
    scale_map "block": the scale of 32-k block kb of row/column c is byte 0 of lane c + 16 kb (the model the
    kernels use); "holder": each lane's scale multiplies the values that lane holds."""
    A = np.zeros((16, 128))
    B = np.zeros((128, 16))
    for l in range(64):
        r, g = l % 16, l // 16
        A[r, 32 * g:32 * g + 32] = O.unpack_fp4(a[l, :16]).astype(np.float64)
        vals = O.e4m3_decode(b[l]).astype(np.float64)
        for j in range(32):
            B[b_k(g, j), r] = vals[j] * (2.0 ** (int(sb[l]) - 127) if scale_map == "holder" else 1.0)
        if scale_map == "holder":
            A[r, 32 * g:32 * g + 32] *= 2.0 ** (int(sa[l]) - 127)
    if scale_map == "block":
        for l in range(64):
            r, g = l % 16, l // 16
            A[r, 32 * g:32 * g + 32] *= 2.0 ** (int(sa[l]) - 127)
            B[32 * g:32 * g + 32, r] *= 2.0 ** (int(sb[l]) - 127)
    D = A @ B
    out = np.zeros((64, 4))
    for l in range(64):
        for i in range(4):
            out[l, i] = D[4 * (l // 16) + i, l % 16]
    return out


def random_e4m3(rng, shape):
    c = rng.integers(0, 256, shape).astype(np.uint8)
    c[(c & 0x7F) == 0x7F] = 0x38  # no NaN codes
    return c


def probe_report(rng):
    """One-hot probes: which D entries a single A nibble / B byte reaches."""
    lines = []
    ones_a = np.zeros((64, 32), np.uint8)
    ones_a[:, :16] = 0x22                      # every A value 1.0
    ones_b = np.full((64, 32), 0x38, np.uint8)  # every B value 1.0
    s127 = np.full(64, 127)
    for lb, jb in [(0, 0), (1, 0), (16, 0), (0, 1), (0, 16), (17, 5), (33, 31), (48, 8)]:
        b = np.zeros((64, 32), np.uint8)
        b[lb, jb] = 0x38
        d = run_scale(ones_a, b, s127, s127)
        nz = np.argwhere(d != 0)
        lines.append(f"B one-hot lane {lb} byte {jb}: D nonzero at (lane,i) {nz[:6].tolist()} ... ({len(nz)} entries)")
    for la, ja, hi in [(0, 0, 0), (0, 0, 1), (1, 0, 0), (16, 0, 0), (0, 8, 0), (33, 3, 1)]:
        a = np.zeros((64, 32), np.uint8)
        a[la, ja] = 0x20 if hi else 0x02
        d = run_scale(a, ones_b, s127, s127)
        nz = np.argwhere(d != 0)
        lines.append(f"A one-hot lane {la} byte {ja} {'hi' if hi else 'lo'}: D nonzero at {nz[:6].tolist()} ... ({len(nz)} entries)")
    # k pairing: B carries distinct values per (lane, byte) so D reveals the partner of an A one-hot
    vals = np.array([c for c in range(1, 255) if (c & 0x7F) not in (0, 0x7F)], np.uint8)  # 252 distinct values
    for la, ja, hi in [(0, 0, 0), (0, 0, 1), (0, 1, 0), (0, 7, 1), (0, 8, 0), (0, 15, 1), (16, 0, 0), (32, 4, 1), (48, 15, 1)]:
        a = np.zeros((64, 32), np.uint8)
        a[la, ja] = 0x20 if hi else 0x02
        b = np.zeros((64, 32), np.uint8)
        key = {}
        for l in range(0, 64, 16):   # column 0 lanes only
            for j in range(32):
                v = vals[(l // 16 * 32 + j) % len(vals)]
                b[l, j] = v
                key[float(O.e4m3_decode(np.array([v]))[0])] = (l, j)
        d = run_scale(a, b, s127, s127)
        col0 = [(l, i, d[l, i]) for l in range(64) for i in range(4) if d[l, i] != 0 and l % 16 == 0]
        lines.append(f"A lane {la} byte {ja} {'hi' if hi else 'lo'} pairs with B (lane, byte) {[key.get(float(v)) for _, _, v in col0]} at D {[(l, i) for l, i, _ in col0]}")
    return "\n".join(lines)


def test_block_scaled_mfma_layout_fp4_x_fp8():
    rng = np.random.default_rng(0)
    for trial in range(3):
        a = rng.integers(0, 256, (64, 32)).astype(np.uint8)
        a[:, 16:] = 0
        b = random_e4m3(rng, (64, 32))
        sa = rng.integers(122, 133, 64)
        sb = rng.integers(122, 133, 64)
        got = run_scale(a, b, sa, sb)
        exp = expected_scale(a, b, sa, sb)
        # the instruction's internal accumulation is not an fp64 sum: allow 1e-4 of the largest output
        ok = np.allclose(got, exp, rtol=0, atol=1e-4 * np.abs(exp).max())
        if not ok:
            alt = expected_scale(a, b, sa, sb, "holder")
            print("holder scale mapping matches:", np.allclose(got, alt, rtol=0, atol=1e-4 * np.abs(alt).max()))
            print("MFMA layout mismatch; probes:\n" + probe_report(rng))
        assert ok, f"trial {trial}: max |diff| {np.abs(got - exp).max()} (max |exp| {np.abs(exp).max()})"


def test_bf16_mfma_layout():
    rng = np.random.default_rng(1)
    L = _lib()
    dev = torch.device("cuda:0")
    a = O.f32_to_bf16_bits(rng.standard_normal((64, 8)).astype(np.float32))
    b = O.f32_to_bf16_bits(rng.standard_normal((64, 8)).astype(np.float32))
    ta = torch.from_numpy(a.view(np.int16)).to(dev)
    tb = torch.from_numpy(b.view(np.int16)).to(dev)
    c = torch.zeros(64, 4, dtype=torch.float32, device=dev)
    L.call("dsv41_selftest_mfma_bf16", L.ptr(ta), L.ptr(tb), L.ptr(c), L.stream(dev))
    torch.cuda.synchronize()
    A = np.zeros((16, 32))
    B = np.zeros((32, 16))
    af, bf = O.bf16_bits_to_f32(a), O.bf16_bits_to_f32(b)
    for l in range(64):
        A[l % 16, 8 * (l // 16):8 * (l // 16) + 8] = af[l]
        B[8 * (l // 16):8 * (l // 16) + 8, l % 16] = bf[l]
    D = A @ B
    exp = np.array([[D[4 * (l // 16) + i, l % 16] for i in range(4)] for l in range(64)])
    assert np.allclose(c.cpu().numpy(), exp, rtol=1e-5, atol=1e-5)
