"""Pins of the CPU oracle (oracle/moe_oracle.py): golden vectors written by the reference's own quant.py,
the library routine the reference relies on (torch's float8_e4m3fn cast), closed forms and brute force.
Each check is chosen so that a plausible slip in the oracle (wrong nibble order, sign of code 8, E8M0
bias, tie rounding, lowest-index tie break) fails it."""
import os

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quant_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def same_bits_nan_aware(a, b):
    """bf16 bit equality; NaN == NaN whatever its sign/payload (torch's CPU NaN bits are not a format rule)."""
    a = np.asarray(a, np.uint16)
    b = np.asarray(b, np.uint16)
    an = ((a & 0x7F80) == 0x7F80) & ((a & 0x7F) != 0)
    bn = ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    return bool(np.all(np.where(an | bn, an == bn, a == b)))


def test_dequant_every_code_and_scale_bit_exact(gold):
    out = O.dequant_fp4(gold["deq_all_packed"], gold["deq_all_scale"])
    assert out.shape == (256, 32)
    # bit-exact including -0.0 (code 8), subnormal scale byte 0 and overflow to +-inf at 253..255
    assert np.array_equal(out, gold["deq_all_bf16"]) or same_bits_nan_aware(out, gold["deq_all_bf16"])
    assert same_bits_nan_aware(out, gold["deq_all_bf16"])
    # the oracle reproduces torch's CPU NaN bits too
    assert np.array_equal(out, gold["deq_all_bf16"])


def test_dequant_random_and_tiling(gold):
    w, s = gold["rand_w"], gold["rand_s"]
    for e in range(w.shape[0]):
        assert np.array_equal(O.dequant_fp4(w[e], s[e]), gold["rand_deq_bf16"][e])
    assert np.array_equal(O.tile_fp4(w), gold["rand_w_tiled"])
    assert np.array_equal(O.tile_fp4_scales(s), gold["rand_s_tiled"])
    assert np.array_equal(O.untile_fp4(O.tile_fp4(w)), w)
    assert np.array_equal(O.untile_fp4_scales(O.tile_fp4_scales(s)), s)


def test_e8m0_identity():
    b = np.arange(256)
    v = O.e8m0_to_f32(b)
    assert v[127] == 1.0 and v[128] == 2.0 and v[126] == 0.5 and np.isinf(v[255])
    assert v[0] == np.float32(2.0 ** -127) and v[0] > 0
    assert np.all(v[1:255] == np.ldexp(np.float32(1), b[1:255] - 127))


def test_ceil_log2_and_pow2(gold):
    assert np.array_equal(O.ceil_log2(gold["cl2_in"]), gold["cl2_out"])
    assert np.array_equal(O.pow2_scale(np.maximum(gold["pow2_in"], np.float32(1e-4)), 448.0), gold["pow2_out"])
    # brute force: exact powers of two and their neighbours
    for e in range(-30, 30):
        p = np.float32(2.0 ** e)
        assert O.ceil_log2(p) == e
        assert O.ceil_log2(np.nextafter(p, np.float32(np.inf))) == e + 1


def test_round_e4m3_matches_torch_cast():
    """fused.py:24-34 formula == torch's float8_e4m3fn cast for |v| <= 448 (test_fused.py:17 states this)."""
    g = torch.Generator().manual_seed(7)
    v = torch.cat([torch.randn(1 << 20, generator=g) * 40, torch.randn(1 << 16, generator=g) * 1e-2,
                   (torch.rand(1 << 16, generator=g) - 0.5) * 896]).clamp(-448, 448)
    ref = v.to(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(O.round_e4m3(v.numpy()), ref)
    # every E4M3 code value is a fixed point, and encode/decode round trips (except NaN codes)
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    vals = O.e4m3_decode(codes)
    assert np.array_equal(O.round_e4m3(vals), vals)
    enc = O.e4m3_encode(vals)
    ok = (enc == codes) | ((codes & 0x7F) == 0)  # +-0 encode to their sign
    assert ok.all()
    assert np.array_equal(O.e4m3_decode(codes).view(np.uint32),
                          torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().view(np.uint32))


def test_fake_quant_fp8_golden(gold):
    xb = O.bf16_bits_to_f32(gold["fq8_in_bf16"])
    fq = O.fake_quant_fp8(xb)
    assert np.array_equal(O.f32_to_bf16_bits(fq), gold["fq8_out_bf16"])
    fq32 = O.fake_quant_fp8(gold["fq8_in_f32"])
    assert np.array_equal(fq32.view(np.uint32), gold["fq8_out_f32"].view(np.uint32))
    q, s = O.quant_fp8(xb)
    assert np.array_equal(s, gold["qfp8_scales_bf16in"])
    codes, e8 = O.quant_fp8_e8m0(xb)
    assert np.array_equal(codes, gold["qfp8_codes_bf16in"])
    assert np.array_equal(O.e8m0_to_f32(e8), gold["qfp8_scales_bf16in"])
    # idempotent on values (a caller's already fake-quantised x re-quantises to the same values)
    assert np.array_equal(O.fake_quant_fp8(fq), fq)


def test_permute_x_round_trip():
    x = np.arange(2 * 64, dtype=np.float32).reshape(2, 64)
    xp = O.permute_x(x)
    assert list(xp[0, :8]) == [0, 4, 2, 6, 1, 5, 3, 7]
    assert np.array_equal(O.unpermute_x(xp), x)


def test_swiglu_quant_closed_form():
    rng = np.random.default_rng(3)
    gu = (rng.standard_normal((5, 2 * 64)) * 6).astype(np.float32)
    w = rng.random(5).astype(np.float32)
    h = O.swiglu_quant(gu, w, 64, 10.0)
    # independent float64 evaluation, then the same two rounding points
    g = np.minimum(gu[:, :64].astype(np.float64), 10.0)
    u = np.clip(gu[:, 64:].astype(np.float64), -10.0, 10.0)
    ref = w[:, None] * g / (1.0 + np.exp(-g)) * u
    ref = O.fake_quant_fp8(O.bf16_round(ref.astype(np.float32)))
    diff = np.abs(h - ref) / np.maximum(np.abs(ref), 1e-30)
    assert (diff[ref != 0] <= 0.07).all()          # at most one E4M3 ulp from fp32 rounding differences
    assert (h == ref).mean() > 0.97
    assert np.array_equal(O.swiglu_quant(gu, w, 64, 10.0, permute=True), O.permute_x(h))
    # limit 0 disables the clamps
    big = np.full((1, 128), 30.0, np.float32)
    assert O.swiglu_quant(big, None, 64, 0.0).max() > 400 and O.swiglu_quant(big, None, 64, 10.0).max() < 101


def test_gate_topk_brute_force():
    rng = np.random.default_rng(5)
    for func in ("softmax", "sigmoid", "sqrtsoftplus"):
        sc = rng.standard_normal((6, 384)).astype(np.float32)
        bias = (rng.standard_normal(384) * 0.1).astype(np.float32)
        idx, w = O.gate_topk(sc, bias, 1.0, 8, 2.5, func, True)
        t = torch.from_numpy(sc)
        s = {"softmax": t.softmax(-1), "sigmoid": t.sigmoid(), "sqrtsoftplus": torch.nn.functional.softplus(t).sqrt()}[func]
        ref_idx = (s + torch.from_numpy(bias)).topk(8, dim=-1)[1]
        assert np.array_equal(np.sort(idx, -1), np.sort(ref_idx.numpy(), -1))
        ref_w = s.gather(1, torch.from_numpy(idx.astype(np.int64)))
        ref_w = ref_w / (ref_w.sum(-1, keepdim=True) + 1e-20) * 2.5
        assert np.allclose(w, ref_w.numpy(), rtol=1e-6, atol=0)
    # ties: the lowest index wins (fused2.py:441)
    tied = np.zeros((1, 16), np.float32)
    idx, _ = O.gate_topk(tied, None, 1.0, 4, 1.0, "softmax", True)
    assert list(idx[0]) == [0, 1, 2, 3]


def test_moe_dispatch_invariants_and_brute_force():
    rng = np.random.default_rng(9)
    for M, k, E, gmax in [(1, 8, 384, 64), (4, 8, 16, 64), (16, 8, 8, 4), (3, 2, 5, 1)]:
        eid = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
        wt = rng.random((M, k)).astype(np.float32)
        tok, wts, inv, ge, gs, G = O.moe_dispatch(eid, wt, k, E, gmax)
        n = M * k
        flat = eid.reshape(-1)
        assert sorted(inv.tolist()) == list(range(n))
        assert np.array_equal(tok[inv], np.arange(n) // k)
        assert np.array_equal(wts[inv], wt.reshape(-1))
        # groups: expert-ascending, <= gmax pairs, covering the sorted pairs exactly, padded with -1 / n
        assert np.all(ge[G:] == -1) and np.all(gs[G:] == n)
        for g in range(G):
            a, b = gs[g], gs[g + 1]
            assert 0 < b - a <= gmax
            assert np.all(flat[np.argsort(inv)][a:b] == ge[g])
        assert np.all(np.diff(ge[:G]) >= 0)


def test_grouped_gemm_textbook():
    rng = np.random.default_rng(11)
    E, N, K = 3, 32, 256
    w = rng.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    s = rng.integers(118, 130, (E, N, K // 32), dtype=np.uint8)
    x = O.fake_quant_fp8(rng.standard_normal((4, K)).astype(np.float32))
    ge = np.array([2, 0], np.int32)
    gs = np.array([0, 3, 5], np.int32)
    tok = np.array([0, 1, 3, 2, 0], np.int32)
    out = O.grouped_gemm(x, w, s, ge, gs, tok, 2)
    # brute-force scalar loop on one entry per pair
    for p, (g, t) in enumerate([(0, 0), (0, 1), (0, 3), (1, 2), (1, 0)]):
        e = ge[g]
        n = (7 * p) % N
        acc = 0.0
        for kk in range(K):
            code = (w[e, n, kk // 2] >> (4 * (kk % 2))) & 15
            acc += float(x[tok[p], kk]) * float(O.FP4_TABLE[code]) * 2.0 ** (int(s[e, n, kk // 32]) - 127)
        assert abs(out[p, n] - acc) <= 1e-5 * max(1.0, abs(acc))


def test_dequant_shortcut_matches_full_path():
    rng = np.random.default_rng(12)
    w = rng.integers(0, 256, (64, 128), dtype=np.uint8)
    s = rng.integers(2, 251, (64, 8), dtype=np.uint8)
    assert np.array_equal(O.dequant_fp4_values(w, s), O.bf16_bits_to_f32(O.dequant_fp4(w, s)))


def test_residual_rmsnorm_quant_matches_torch_rms_norm():
    """Closed form pin: torch's own rms_norm (fp32, CPU) on the bf16 residual sum, then the golden-pinned fq8."""
    import torch
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(3, 512, generator=g) * 3).to(torch.bfloat16)
    y = (torch.randn(3, 512, generator=g)).to(torch.bfloat16)
    w = (torch.rand(512, generator=g) + 0.5).to(torch.bfloat16)
    xn, xq = O.residual_rmsnorm_quant(x.float().numpy(), y.float().numpy(), w.float().numpy(), 1e-6)
    r = (x + y).float()
    ref = torch.nn.functional.rms_norm(r, (512,), w.float(), eps=1e-6).to(torch.bfloat16).float().numpy()
    # fp32 evaluation order may move a value across a bf16 rounding boundary: at most one bf16 ulp
    assert np.all(np.abs(xn - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)
    assert (xn == ref).mean() > 0.99
    assert np.array_equal(xq, O.fake_quant_fp8(xn))
