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


def test_moe_dispatch_drops_invalid_ids():
    """Ids outside [0, E) are dropped: brute force on a tiny case (the placed pairs in expert order, ascending pair
    order inside an expert; dropped pairs have inv -1; padding starts at the number of placed pairs)."""
    E, k = 8, 3
    eid = np.array([[3, -1, 5], [700, 3, 1], [8, 0, 3]], np.int32)
    wt = np.arange(9, dtype=np.float32).reshape(3, 3) + 1
    tok, wts, inv, ge, gs, G = O.moe_dispatch(eid, wt, k, E, 2)
    flat = eid.reshape(-1)
    kept = [p for p in range(9) if 0 <= flat[p] < E]
    order = sorted(kept, key=lambda p: (flat[p], p))
    assert len(order) == 6
    assert tok[:6].tolist() == [p // k for p in order] and tok[6:].tolist() == [0, 0, 0]
    assert wts[:6].tolist() == [float(wt.reshape(-1)[p]) for p in order] and wts[6:].tolist() == [0.0, 0.0, 0.0]
    assert [inv[p] for p in range(9)] == [order.index(p) if p in order else -1 for p in range(9)]
    # experts 0, 1, 3 (3 pairs -> groups of 2 + 1), 5
    assert G == 5 and ge[:5].tolist() == [0, 1, 3, 3, 5] and gs[:5].tolist() == [0, 1, 2, 4, 5]
    assert np.all(ge[5:] == -1) and np.all(gs[5:] == 6)


def test_linear_bf16_matches_torch_linear():
    """linear_bf16 against torch's F.linear on bf16 CPU tensors (the op linear_w runs for a bf16 weight,
    w8.py:102-103): one bf16 rounding of an fp32-accumulated product. fp32 summation order may move a value across a
    rounding boundary, so almost all outputs are bit-equal and none is more than one bf16 ulp away; without the
    rounding step no output would be bf16."""
    import torch
    g = torch.Generator().manual_seed(21)
    x = O.fake_quant_fp8(torch.randn(3, 1024, generator=g).to(torch.bfloat16).float().numpy())
    W = (torch.randn(256, 1024, generator=g) / 32).to(torch.bfloat16)
    got = O.linear_bf16(x, W.view(torch.int16).numpy().view(np.uint16))
    ref = torch.nn.functional.linear(torch.from_numpy(x).to(torch.bfloat16), W).float().numpy()
    assert np.array_equal(got, O.bf16_round(got))
    assert (got == ref).mean() > 0.98
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)


def _one_hot_x(dim, k0, v):
    x = np.zeros((1, dim), np.float32)
    x[0, k0] = v
    return x


def test_shared_expert_structure_against_routed_expert():
    """With the shared expert's weights equal to the dequantised FP4 weights of one routed expert (bf16-exact) and a
    one-hot activation (every gu value is one product of <= 6 significant bits, so the bf16 rounding of gu is exact),
    shared_expert must equal the library-pinned moe_layer_routed of that expert with weight 1, rounded to bf16: this
    pins the w1 / w3 halves, the SwiGLU limit, the absent routing weight and the final bf16 rounding."""
    rng = np.random.default_rng(31)
    E, inter, dim = 3, 128, 256
    w13 = rng.integers(0, 256, (E, 2 * inter, dim // 2), dtype=np.uint8)
    s13 = rng.integers(124, 130, (E, 2 * inter, dim // 32), dtype=np.uint8)
    w2 = rng.integers(0, 256, (E, dim, inter // 2), dtype=np.uint8)
    s2 = rng.integers(118, 124, (E, dim, inter // 32), dtype=np.uint8)
    e = 1
    Ws13 = O.dequant_fp4(w13[e], s13[e])
    Ws2 = O.dequant_fp4(w2[e], s2[e])
    for limit, (k0, v) in [(10.0, (37, 2.5)), (0.0, (200, -1.75)), (10.0, (5, 6.0))]:
        xq = O.fake_quant_fp8(_one_hot_x(dim, k0, v))
        ys = O.shared_expert(xq, Ws13, Ws2, inter, limit)
        routed = O.moe_layer_routed(xq, np.array([[e]]), np.array([[1.0]], np.float32), w13, s13, w2, s2, inter, limit)
        assert np.abs(routed).max() > 0
        assert np.array_equal(ys, O.bf16_round(routed))
    # swapping the halves changes the result (the check above is sensitive to it)
    xq = O.fake_quant_fp8(_one_hot_x(dim, 37, 2.5))
    swapped = np.concatenate([Ws13[inter:], Ws13[:inter]])
    assert not np.array_equal(O.shared_expert(xq, swapped, Ws2, inter, 10.0), O.shared_expert(xq, Ws13, Ws2, inter, 10.0))


def test_moe_layer_composition():
    """moe_layer = bf16(routed sum + shared), with x FP8-fake-quantised first (model.py:565-591). With the shared
    expert equal to routed expert e' and an off-grid one-hot x (fq8 moves it), it must equal
    bf16(moe_layer_routed(fq8 x) + bf16(moe_layer_routed row of e' with weight 1))."""
    rng = np.random.default_rng(33)
    E, inter, dim = 6, 128, 256
    w13 = rng.integers(0, 256, (E, 2 * inter, dim // 2), dtype=np.uint8)
    s13 = rng.integers(124, 130, (E, 2 * inter, dim // 32), dtype=np.uint8)
    w2 = rng.integers(0, 256, (E, dim, inter // 2), dtype=np.uint8)
    s2 = rng.integers(118, 124, (E, dim, inter // 32), dtype=np.uint8)
    x = _one_hot_x(dim, 77, 3.3)
    xq = O.fake_quant_fp8(x)
    assert not np.array_equal(xq, x)
    eid = np.array([[0, 2, 4]])
    wt = np.array([[0.5, 0.3, 0.2]], np.float32)
    es = 5
    got = O.moe_layer(x, eid, wt, w13, s13, w2, s2, O.dequant_fp4(w13[es], s13[es]), O.dequant_fp4(w2[es], s2[es]), inter, 10.0)
    routed = O.moe_layer_routed(xq, eid, wt, w13, s13, w2, s2, inter, 10.0)
    shared = O.bf16_round(O.moe_layer_routed(xq, np.array([[es]]), np.array([[1.0]], np.float32), w13, s13, w2, s2, inter, 10.0))
    assert np.array_equal(got, O.bf16_round(routed + shared))


def test_gemv_pairs_pins():
    """gemv_pairs = wt x grouped_gemm on singleton groups (the textbook-pinned function), and a scalar brute-force
    sum on a tiny case (cukern.py:60-77: out[p] = wt[p] * x[row_in[p]] . deq(W[expert[p]]))."""
    rng = np.random.default_rng(41)
    E, N, K = 4, 32, 128
    w = rng.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    s = rng.integers(120, 130, (E, N, K // 32), dtype=np.uint8)
    x = O.fake_quant_fp8(rng.standard_normal((3, K)).astype(np.float32))
    row_in = np.array([2, 0, 2, 1], np.int32)
    expert = np.array([3, 3, 0, 1], np.int32)
    wt = np.array([0.5, -1.25, 2.0, 1.0], np.float32)
    got = O.gemv_pairs(x, w, s, row_in, expert, wt)
    single = O.grouped_gemm(x, w, s, expert, np.arange(5, dtype=np.int32), row_in, 4)
    assert np.allclose(got, wt[:, None] * single, rtol=1e-6, atol=1e-6)
    for p in range(4):
        for n in (0, 13, 31):
            acc = 0.0
            for kk in range(K):
                code = (int(w[expert[p], n, kk // 2]) >> (4 * (kk % 2))) & 15
                acc += float(x[row_in[p], kk]) * float(O.FP4_TABLE[code]) * 2.0 ** (int(s[expert[p], n, kk // 32]) - 127)
            assert abs(got[p, n] - wt[p] * acc) <= 1e-5 * max(1.0, abs(wt[p] * acc))


def test_every_oracle_function_has_a_pin():
    """Every public function of the oracle that computes a result is listed in PINS (helpers excepted)."""
    import inspect
    helpers = {"f32_bits", "bits_f32", "f32_to_bf16_bits", "bf16_bits_to_f32", "bf16_round", "e4m3_encode", "e4m3_decode", "unpack_fp4",
               "dequant_fp4_f32", "dequant_fp4_values", "untile_fp4", "untile_fp4_scales", "quant_fp8_e8m0", "pow2_scale", "unpermute_x",
               "sigmoid_f32", "dense_weights", "expert_pair", "deq64", "rel_l2", "max_abs_over_rms", "fp8_split_values"}
    fns = {n for n, f in inspect.getmembers(O, inspect.isfunction) if f.__module__ == O.__name__ and not n.startswith("_")}
    missing = fns - helpers - set(O.PINS)
    assert not missing, f"oracle functions without a pin: {sorted(missing)}"
    assert set(O.PINS) <= fns, f"PINS names functions the oracle lacks: {sorted(set(O.PINS) - fns)}"


def test_hc_pre_norm_quant_pins():
    """One-hot pre weights reduce the pre-mix to a copy of one stream: rmsnorm of it (torch rms_norm, fp32 CPU) and the
    golden-pinned fq8; splitting that stream's weight over two equal streams gives the same result."""
    import torch
    g = torch.Generator().manual_seed(7)
    B, hc, d = 3, 4, 512
    x = (torch.randn(B, hc, d, generator=g) * 2).to(torch.bfloat16)
    w = (torch.rand(d, generator=g) + 0.5).to(torch.bfloat16)
    pre = np.zeros((B, hc), np.float32)
    pre[:, 2] = 1.0
    y, yq = O.hc_pre_norm_quant(x.float().numpy(), pre, w.float().numpy(), 1e-6)
    ref = torch.nn.functional.rms_norm(x[:, 2].float(), (d,), w.float(), eps=1e-6).to(torch.bfloat16).float().numpy()
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30) and (y == ref).mean() > 0.99
    assert np.array_equal(yq, O.fake_quant_fp8(y))
    x2 = x.clone()
    x2[:, 1] = x2[:, 2]
    pre2 = np.zeros((B, hc), np.float32)
    pre2[:, 1] = pre2[:, 2] = 0.5
    y2, _ = O.hc_pre_norm_quant(x2.float().numpy(), pre2, w.float().numpy(), 1e-6)
    assert np.array_equal(y2, y)


def test_hc_post_pins():
    import torch
    rng = np.random.default_rng(8)
    B, d = 2, 256
    res = O.bf16_round(rng.standard_normal((B, 4, d)).astype(np.float32))
    x = O.bf16_round(rng.standard_normal((B, d)).astype(np.float32))
    # post 0 and comb = identity: the streams are unchanged; comb 0 and post one-hot: stream i takes x, the rest 0
    assert np.array_equal(O.hc_post(x, res, np.zeros((B, 4)), np.tile(np.eye(4), (B, 1, 1))), res)
    oh = np.zeros((B, 4))
    oh[:, 3] = 1.0
    out = O.hc_post(x, res, oh, np.zeros((B, 4, 4)))
    assert np.array_equal(out[:, 3], x) and np.all(out[:, :3] == 0)
    # general mix against torch's einsum in float64
    post = rng.standard_normal((B, 4))
    comb = rng.standard_normal((B, 4, 4))
    t = torch.einsum("bji,bjn->bin", torch.from_numpy(comb), torch.from_numpy(res.astype(np.float64))) + \
        torch.from_numpy(post)[:, :, None] * torch.from_numpy(x.astype(np.float64))[:, None, :]
    assert np.array_equal(O.hc_post(x, res, post, comb), O.bf16_round(t.numpy().astype(np.float32)))
    # the MoE pieces: small integers times powers of two sum exactly
    y2 = rng.integers(-64, 64, (B, 6, d)).astype(np.float32) * 0.25
    ys = rng.integers(-8, 8, (B, d)).astype(np.float32)
    assert np.array_equal(O.hc_post_input(y2, ys), O.bf16_round((y2.sum(1) + ys).astype(np.float32)))


def _torch_dequant_fp8(w, s):
    """quant.dequant_fp8_block built from torch's own float8_e4m3fn cast and ldexp (not the oracle's decode)."""
    import torch
    wt = torch.from_numpy(np.ascontiguousarray(w)).view(torch.float8_e4m3fn).float()
    e = torch.from_numpy(np.ascontiguousarray(s).astype(np.int32)) - 127
    N, K = w.shape
    e = e.repeat_interleave(32, 0)[:N].repeat_interleave(32, 1)[:, :K]
    return torch.ldexp(wt, e.float())


def test_dequant_fp8_every_code_and_scale():
    """Every E4M3 code times every scale byte 1..254 against torch's float8_e4m3fn cast times ldexp (the reference's
    w.float() * s), fp32 bit-exact and after the bf16 cast (NaN codes compared as NaN)."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    w = np.tile(codes, (32, 1))                                          # every row holds all 256 codes
    for b0 in range(1, 255, 8):
        sc = np.arange(b0, b0 + 8).clip(1, 254).astype(np.uint8).reshape(1, 8)
        got = O.dequant_fp8_block_f32(w, sc)
        ref = _torch_dequant_fp8(w, sc).numpy()
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(O.f32_bits(got)[~nan], O.f32_bits(ref)[~nan]), f"scale bytes {b0}.."
        gb = O.dequant_fp8_block(w, sc)
        rb = torch.from_numpy(ref).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(gb[~nan], rb[~nan])


def test_dequant_fp8_block_structure():
    """A scale byte changed in one block moves exactly that 32 x 32 block, by a factor of 2 (ragged N and K)."""
    rng = np.random.default_rng(5)
    w = rng.integers(0, 256, (70, 100), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0
    s = rng.integers(110, 130, (3, 4), dtype=np.uint8)
    a = O.dequant_fp8_block_f32(w, s)
    s2 = s.copy()
    s2[1, 2] += 1
    b = O.dequant_fp8_block_f32(w, s2)
    mask = np.zeros_like(a, dtype=bool)
    mask[32:64, 64:96] = True
    assert np.array_equal(a[~mask], b[~mask])
    assert np.array_equal(b[mask], a[mask] * 2)


def test_linear_fp8w_pins():
    """One-hot rows pick dequantised columns exactly; random x against torch F.linear in float64 on the torch-built
    dequant; the block-diagonal form against a scalar loop."""
    import torch
    rng = np.random.default_rng(6)
    N, K = 96, 128
    w = rng.integers(0, 256, (N, K), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0
    s = rng.integers(115, 135, (3, 4), dtype=np.uint8)
    deq = torch.from_numpy(_torch_dequant_fp8(w, s).numpy()).to(torch.bfloat16).float()
    x = np.zeros((3, K), np.float32)
    x[0, 5] = 1.0
    x[1, 77] = -2.0
    x[2, 127] = 0.5
    got = O.linear_fp8w(x, w, s)
    assert np.array_equal(got[0], deq[:, 5].numpy())
    assert np.array_equal(got[1], -2 * deq[:, 77].numpy())
    assert np.array_equal(got[2], 0.5 * deq[:, 127].numpy())
    xr = torch.randn(4, K, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).float().numpy()
    ref = torch.nn.functional.linear(torch.from_numpy(xr).double(), deq.double()).float().numpy()
    assert np.array_equal(O.linear_fp8w(xr, w, s), ref)
    gc = 32
    G = N // gc
    xg = torch.randn(2 * G, K, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).float().numpy()
    got = O.linear_fp8w(xg, w, s, group_cols=gc)
    d = deq.double().numpy()
    for b in range(2):
        for n in range(N):
            v = float(np.dot(xg[b * G + n // gc].astype(np.float64), d[n]))
            assert got[b, n] == np.float32(v)


def test_lo_exponent_brute_force():
    """lo_exponent(a) is the smallest e >= -126 with a <= 448 * 2^e, found by scanning e; on random magnitudes over the
    whole fp32 range, on powers of two and on the 448 * 2^k boundaries and their fp32 neighbours."""
    rng = np.random.default_rng(7)
    a = np.concatenate([np.exp(rng.uniform(-100, 88, 3000)).astype(np.float32),
                        np.ldexp(np.float32(1.0), np.arange(-149, 127)).astype(np.float32),
                        np.ldexp(np.float32(448.0), np.arange(-140, 118)).astype(np.float32)])
    a = np.concatenate([a, np.nextafter(a, np.float32(np.inf)), np.nextafter(a, np.float32(0)), [0.0, 1e-45]]).astype(np.float32)
    got = O.lo_exponent(a)
    for ai, g in zip(a.astype(np.float64), got):
        e = -126
        while ai > 448.0 * 2.0 ** e:
            e += 1
        assert g == e, (ai, g, e)


def test_fp8_split_pins():
    """hi is the golden-pinned quant_fp8 encoding; lo is torch's float8_e4m3fn cast of the residual at its scale; hi + lo
    reconstructs bf16 x exactly except residuals below lo's normal range (then within 2^-21 of the block amax); an
    FP8-grid x gives all-zero lo codes."""
    import torch
    rng = np.random.default_rng(11)
    for scale in (1.0, 1e-3, 300.0):
        x = torch.from_numpy((rng.standard_normal((64, 256)) * scale).astype(np.float32)).to(torch.bfloat16).float().numpy()
        x[0, :32] = 0.0
        x[1, :32] = torch.tensor(1e-6).to(torch.bfloat16).float().item()   # a block under the hi rule's 1e-4 floor
        hc, hs, lc, ls = O.fp8_split(x)
        qc, qs = O.quant_fp8_e8m0(x)
        assert np.array_equal(hc, qc) and np.array_equal(hs, qs)
        hv = O.e4m3_decode(hc).astype(np.float64) * np.ldexp(1.0, np.repeat(hs.astype(np.int32) - 127, 32, axis=-1))
        r = (x.astype(np.float64) - hv).astype(np.float32)
        e2 = ls.astype(np.int32) - 127
        want = torch.from_numpy((r / np.ldexp(1.0, np.repeat(e2, 32, axis=-1))).astype(np.float32)).to(torch.float8_e4m3fn)
        assert np.array_equal(lc, want.view(torch.uint8).numpy())
        v = O.fp8_split_values(hc, hs, lc, ls)
        amax = np.repeat(np.abs(x.reshape(-1, 32)).max(-1), 32).reshape(x.shape).astype(np.float64)
        err = np.abs(v - x)
        assert np.all(err <= amax * 2.0 ** -21)
        assert np.mean(err == 0) > 0.9999
    fq = O.fake_quant_fp8(x)
    _, _, lc0, _ = O.fp8_split(fq)
    assert not np.any(lc0 & 0x7F)
