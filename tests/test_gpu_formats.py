"""Format kernels against the golden vectors written by the reference's quant.py and against the oracle:
dequant_fp4 bit-exact over every (code, scale byte) and both layouts; fake_quant_fp8 / quant_fp8 bit-exact;
swiglu_quant against the oracle (identical up to an E4M3 ulp where fp32 evaluation order flips a rounding)."""
import os

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quant_golden.npz")
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def test_dequant_every_code_and_scale(gold):
    from dsv41_amd import quant
    p = torch.from_numpy(gold["deq_all_packed"]).to(DEV)
    s = torch.from_numpy(gold["deq_all_scale"]).to(DEV)
    # K = 32 per row: one scale byte per row, all 256 bytes and all 16 codes
    out = u16(quant.dequant_fp4(p, s))
    assert np.array_equal(out, gold["deq_all_bf16"])


def test_dequant_random_row_major_and_tiled(gold):
    from dsv41_amd import quant
    w = torch.from_numpy(gold["rand_w"]).to(DEV)
    s = torch.from_numpy(gold["rand_s"]).to(DEV)
    assert np.array_equal(u16(quant.dequant_fp4(w, s)), gold["rand_deq_bf16"])
    wt = torch.from_numpy(gold["rand_w_tiled"]).to(DEV)
    st = torch.from_numpy(gold["rand_s_tiled"]).to(DEV)
    assert np.array_equal(u16(quant.dequant_fp4(wt, st, tiled=True)), gold["rand_deq_bf16"])
    # torch-side tiling helpers agree with the reference's layout
    assert torch.equal(quant.tile_fp4(w), wt) and torch.equal(quant.tile_fp4_scales(s), st)


def test_fake_quant_fp8_golden(gold):
    from dsv41_amd import quant
    xb = torch.from_numpy(gold["fq8_in_bf16"].view(np.int16)).view(torch.bfloat16).to(DEV)
    assert np.array_equal(u16(quant.fake_quant_fp8(xb)), gold["fq8_out_bf16"])
    xf = torch.from_numpy(gold["fq8_in_f32"]).to(DEV)
    assert np.array_equal(quant.fake_quant_fp8(xf).cpu().numpy().view(np.uint32), gold["fq8_out_f32"].view(np.uint32))
    q, s = quant.quant_fp8(xb)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), gold["qfp8_codes_bf16in"])
    assert np.array_equal(s.cpu().numpy(), gold["qfp8_scales_bf16in"])


def test_quant_permuted_input_gives_natural_codes():
    from dsv41_amd import hipkern, quant
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 1024, generator=g).to(torch.bfloat16).to(DEV)
    c0, s0 = quant.quant_fp8_e8m0(x)
    c1, s1 = quant.quant_fp8_e8m0(hipkern.permute_x(x), permuted=True)
    assert torch.equal(c0, c1) and torch.equal(s0, s1)
    codes, e8 = O.quant_fp8_e8m0(O.bf16_bits_to_f32(u16(x)))
    assert np.array_equal(c0.cpu().numpy(), codes) and np.array_equal(s0.cpu().numpy(), e8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quant_fp8_vector_and_strided_paths_agree(dtype):
    # a row stride that is not a multiple of 16 bytes takes the one-value-per-thread kernel, a packed tensor the
    # 16-values-per-thread one; both must give the oracle's codes, scales and fake-quantised values
    from dsv41_amd import hipkern, quant
    g = torch.Generator().manual_seed(5)
    base = (torch.randn(37, 2048 + 1, generator=g) * torch.logspace(-3, 3, 37).unsqueeze(1)).to(dtype).to(DEV)
    strided, packed = base[:, 1:], base[:, 1:].contiguous()
    for permuted in (False, True):
        a = hipkern.permute_x(strided.contiguous())[:, :] if permuted else strided
        if permuted:
            a = torch.cat([torch.zeros(37, 1, dtype=dtype, device=DEV), a], 1)[:, 1:]   # strided again
        b = a.contiguous()
        assert a.stride(0) == 2049 and b.stride(0) == 2048
        ca, sa = quant.quant_fp8_e8m0(a, permuted=permuted)
        cb, sb = quant.quant_fp8_e8m0(b, permuted=permuted)
        assert torch.equal(ca, cb) and torch.equal(sa, sb)
    x32 = packed.float().cpu().numpy()
    codes, e8 = O.quant_fp8_e8m0(x32)
    assert np.array_equal(cb.cpu().numpy(), codes) and np.array_equal(sb.cpu().numpy(), e8)
    fa, fb = quant.fake_quant_fp8(strided), quant.fake_quant_fp8(packed)
    assert torch.equal(fa, fb)
    ref = O.fake_quant_fp8(x32)
    got = fb.float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32)) if dtype == torch.float32 else \
        np.array_equal(u16(fb), O.f32_to_bf16_bits(ref))


@pytest.mark.parametrize("limit,weighted,permute", [(10.0, True, False), (0.0, True, True), (10.0, False, False)])
def test_swiglu_quant(limit, weighted, permute):
    from dsv41_amd import fused
    g = torch.Generator().manual_seed(4)
    rows, inter = 9, 1664
    gu = torch.randn(rows, 2 * inter, generator=g) * 5
    wt = torch.rand(rows, generator=g)
    h = fused.swiglu_quant(gu.to(DEV), wt.to(DEV) if weighted else None, inter, limit, permute=permute)
    ref = O.swiglu_quant(gu.numpy(), wt.numpy() if weighted else None, inter, limit, permute=permute)
    got = O.bf16_bits_to_f32(u16(h))
    # identical except where an ulp-level difference of silu/exp flips a bf16 or E4M3 rounding
    assert (got == ref).mean() > 0.995
    assert O.rel_l2(got, ref) < 2e-3
    # the codes output decodes to exactly the bf16 output's values
    c, s = fused.swiglu_quant_codes(gu.to(DEV), wt.to(DEV) if weighted else None, inter, limit)
    vals = O.e4m3_decode(c.cpu().numpy()) * np.repeat(O.e8m0_to_f32(s.cpu().numpy()), 32, axis=-1)
    assert np.array_equal(vals, got if not permute else O.unpermute_x(got))


@pytest.mark.parametrize("bf16_in,weighted,permute", [(False, True, False), (False, False, True), (True, True, False)])
def test_swiglu_quant_vector_equals_per_element(bf16_in, weighted, permute):
    """The 16-column-per-lane kernel (16-byte aligned rows) and the per-element kernel (taken for a row base 4 or 8 bytes
    off alignment) give the same bf16 values, codes and scales bit for bit."""
    from dsv41_amd import fused
    g = torch.Generator().manual_seed(6)
    rows, inter = 37, 1664
    dt = torch.bfloat16 if bf16_in else torch.float32
    vals = (torch.randn(rows, 2 * inter, generator=g) * 5).to(dt).to(DEV)
    wt = torch.rand(rows, generator=g).to(DEV) if weighted else None
    buf = torch.zeros(rows, 2 * inter + 8, dtype=dt, device=DEV)
    buf[:, :2 * inter] = vals
    aligned = buf[:, :2 * inter]
    buf2 = torch.zeros(rows, 2 * inter + 8, dtype=dt, device=DEV)
    buf2[:, 2:2 * inter + 2] = vals
    shifted = buf2[:, 2:2 * inter + 2]
    assert aligned.data_ptr() % 16 == 0 and shifted.data_ptr() % 16 != 0
    assert torch.equal(fused.swiglu_quant(aligned, wt, inter, 10.0, permute=permute), fused.swiglu_quant(shifted, wt, inter, 10.0, permute=permute))
    ca, sa = fused.swiglu_quant_codes(aligned, wt, inter, 10.0)
    cs, ss = fused.swiglu_quant_codes(shifted, wt, inter, 10.0)
    assert torch.equal(ca, cs) and torch.equal(sa, ss)


@pytest.mark.parametrize("bf16_in,weighted,permute", [(False, True, False), (False, False, True), (True, True, True)])
def test_swiglu_quant_three_kernels_agree(bf16_in, weighted, permute):
    """The three SwiGLU kernels -- 4 columns per lane (inputs of <= 262,144 values: decode rows), 16 columns per lane
    (larger aligned inputs) and one column per thread (misaligned rows) -- give the same bf16 values, codes and scales
    bit for bit: 200 rows x 1664 on the 16-column kernel against its first 36 rows on the 4-column one and against a
    misaligned copy on the per-element one."""
    from dsv41_amd import fused
    g = torch.Generator().manual_seed(8)
    rows, inter, small = 200, 1664, 36
    dt = torch.bfloat16 if bf16_in else torch.float32
    vals = (torch.randn(rows, 2 * inter, generator=g) * 5).to(dt).to(DEV)
    wt = torch.rand(rows, generator=g).to(DEV) if weighted else None
    buf2 = torch.zeros(rows, 2 * inter + 8, dtype=dt, device=DEV)
    buf2[:, 2:2 * inter + 2] = vals
    shifted = buf2[:, 2:2 * inter + 2]
    big = fused.swiglu_quant(vals, wt, inter, 10.0, permute=permute)
    part = fused.swiglu_quant(vals[:small], wt[:small] if weighted else None, inter, 10.0, permute=permute)
    assert torch.equal(big[:small], part)
    assert torch.equal(big, fused.swiglu_quant(shifted, wt, inter, 10.0, permute=permute))
    cb, sb = fused.swiglu_quant_codes(vals, wt, inter, 10.0)
    cp, sp = fused.swiglu_quant_codes(vals[:small], wt[:small] if weighted else None, inter, 10.0)
    assert torch.equal(cb[:small], cp) and torch.equal(sb[:small], sp)


def test_swiglu_quant_bf16_input():
    """bf16 gate/up (the shared expert's linear output, fused.py:294): the same values as the fp32 path on the
    bf16 values, bit for bit."""
    from dsv41_amd import fused
    g = torch.Generator().manual_seed(5)
    gu = (torch.randn(5, 2 * 1664, generator=g) * 4).to(torch.bfloat16)
    hb = fused.swiglu_quant(gu.to(DEV), None, 1664, 10.0)
    hf = fused.swiglu_quant(gu.float().to(DEV), None, 1664, 10.0)
    assert torch.equal(hb, hf)
    ref = O.swiglu_quant(gu.float().numpy(), None, 1664, 10.0)
    got = O.bf16_bits_to_f32(u16(hb))
    assert (got == ref).mean() > 0.995 and O.rel_l2(got, ref) < 2e-3


@pytest.mark.parametrize("M,H,weighted", [(1, 7168, False), (4, 7168, True), (3, 256, True)])
def test_residual_rmsnorm_quant(M, H, weighted):
    """The stack's layer-to-layer step against the oracle: xn within one bf16 ulp (fp32 sum order of the
    variance), xq exactly fake_quant_fp8 of the kernel's own xn."""
    from dsv41_amd import moe
    g = torch.Generator().manual_seed(M * 31 + H)
    x = (torch.randn(M, H, generator=g) * 2).to(torch.bfloat16)
    y = torch.randn(M, H, generator=g).to(torch.bfloat16)
    w = (torch.rand(H, generator=g) + 0.5).to(torch.bfloat16) if weighted else None
    xn, xq = moe.residual_rmsnorm_quant(x.to(DEV), y.to(DEV), None if w is None else w.to(DEV), 1e-6)
    f = lambda t: O.bf16_bits_to_f32(u16(t.contiguous()))
    ref_n, _ = O.residual_rmsnorm_quant(f(x), f(y), None if w is None else f(w), 1e-6)
    got_n = f(xn)
    assert np.all(np.abs(got_n - ref_n) <= np.abs(ref_n) * 2.0 ** -7 + 1e-30)
    assert (got_n == ref_n).mean() > 0.99
    assert np.array_equal(f(xq), O.fake_quant_fp8(got_n))


@pytest.mark.parametrize("B,want_perm", [(1, True), (4, False)])
def test_hc_pre_norm_quant(B, want_perm):
    """The hyper-connection pre-mix + rmsnorm + FP8 quant against the oracle (y within one bf16 ulp, fp32 order of the
    statistics; yq exactly fq8 of the kernel's own y; yf = y; yqp = yq in the 8-k permuted order)."""
    from dsv41_amd import fused2
    g = torch.Generator().manual_seed(60 + B)
    hc, d = 4, 7168
    x = (torch.randn(B, 1, hc, d, generator=g) * 2).to(torch.bfloat16)
    pre = torch.rand(B, hc, generator=g) * 0.8 + 0.1
    w = (torch.rand(d, generator=g) + 0.5).to(torch.bfloat16)
    r = fused2.hc_pre_norm_quant2(x.to(DEV), pre.to(DEV), w.to(DEV), 1e-6, want_f32=True, want_perm=want_perm)
    y, yq, yf = r[0], r[1], r[2]
    f = lambda t: O.bf16_bits_to_f32(u16(t.contiguous()))
    ref_y, _ = O.hc_pre_norm_quant(f(x.reshape(B, hc, d)), pre.numpy(), f(w), 1e-6)
    got = f(y)
    assert np.all(np.abs(got - ref_y) <= np.abs(ref_y) * 2.0 ** -7 + 1e-30) and (got == ref_y).mean() > 0.99
    assert np.array_equal(f(yq), O.fake_quant_fp8(got))
    assert np.array_equal(yf.cpu().numpy(), got)
    if want_perm:
        assert np.array_equal(f(r[3]), O.permute_x(f(yq)))


@pytest.mark.parametrize("mode", ["x", "y2", "y2_sum_first"])
def test_hc_post(mode):
    """The in-place hyper-connection post mix against the oracle (one rounding; fp32 FMA order within one bf16 ulp), with
    x given, or from the MoE pieces y2 [B, nsum, d] (or [nsum, B, d]) + ys."""
    from dsv41_amd import fused2
    rng = np.random.default_rng(70)
    B, d, nsum = 3, 7168, 8
    res0 = O.bf16_round(rng.standard_normal((B, 1, 4, d)).astype(np.float32))
    post = rng.standard_normal((B, 4)).astype(np.float32)
    comb = rng.standard_normal((B, 4, 4)).astype(np.float32)
    to_bf16 = lambda a: torch.from_numpy(O.f32_to_bf16_bits(a).view(np.int16)).view(torch.bfloat16).to(DEV)
    res = to_bf16(res0)
    if mode == "x":
        xv = O.bf16_round(rng.standard_normal((B, d)).astype(np.float32))
        fused2.hc_post2_(to_bf16(xv), res, torch.from_numpy(post).to(DEV), torch.from_numpy(comb).to(DEV))
    else:
        y2 = rng.standard_normal((B, nsum, d)).astype(np.float32)
        ys = O.bf16_round(rng.standard_normal((B, d)).astype(np.float32))
        xv = O.hc_post_input(y2, ys)
        y2d = torch.from_numpy(y2 if mode == "y2" else np.ascontiguousarray(y2.transpose(1, 0, 2))).to(DEV)
        fused2.hc_post2_(None, res, torch.from_numpy(post).to(DEV), torch.from_numpy(comb).to(DEV), y2=y2d, ys=to_bf16(ys),
                         y2_sum_first=(mode == "y2_sum_first"))
    ref = O.hc_post(xv, res0.reshape(B, 4, d), post, comb)
    got = O.bf16_bits_to_f32(u16(res.contiguous())).reshape(B, 4, d)
    tol = np.maximum(np.abs(ref), np.abs(got)) * 2.0 ** -7 + 1e-5
    assert np.all(np.abs(got - ref) <= tol) and (got == ref).mean() > 0.99
