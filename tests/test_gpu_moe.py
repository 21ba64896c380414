"""Parity of the HIP expert path with the CPU oracle (tolerance from the benchmark spec: relative L2 <= 2e-3 and
max-abs <= 1e-2 x output RMS, fp32 accumulation), bit-exact tables for the integer routing work, and
size-independent properties at the full configs[1..2] shapes (batched decode == single-token runs)."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
RTOL_L2, MAXABS_RMS = 2e-3, 1e-2


def close(got, ref, what=""):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    r, m = O.rel_l2(got, ref), O.max_abs_over_rms(got, ref)
    print(f"{what}: rel L2 {r:.2e}, max-abs/RMS {m:.2e}")
    assert r <= RTOL_L2 and m <= MAXABS_RMS, f"{what}: rel L2 {r:.3e}, max-abs/RMS {m:.3e}"


def bf16_vals(t):
    return O.bf16_bits_to_f32(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))


def make_experts(E, H, I, seed, device=DEV):
    g = torch.Generator(device=device).manual_seed(seed)
    w13 = torch.randint(0, 256, (E, 2 * I, H // 2), generator=g, dtype=torch.uint8, device=device)
    s13 = torch.randint(119, 124, (E, 2 * I, H // 32), generator=g, dtype=torch.uint8, device=device)
    w2 = torch.randint(0, 256, (E, H, I // 2), generator=g, dtype=torch.uint8, device=device)
    s2 = torch.randint(119, 124, (E, H, I // 32), generator=g, dtype=torch.uint8, device=device)
    return w13, s13, w2, s2


def to_ex(w13, s13, w2, s2, tiled):
    from dsv41_amd import moe, quant
    if tiled:
        return moe.ExpertWeights(quant.tile_fp4(w13), quant.tile_fp4_scales(s13), quant.tile_fp4(w2), quant.tile_fp4_scales(s2), True)
    return moe.ExpertWeights(w13, s13, w2, s2, False)


def host_subset(ws, ids):
    """The selected experts' row-major weights on the host, indexed by global id."""
    idx = torch.tensor(sorted(ids), device=DEV)
    sub = [w.index_select(0, idx).cpu().numpy() for w in ws]
    pos = {e: i for i, e in enumerate(sorted(ids))}

    class View:
        def __init__(self, a):
            self.a = a
            self.shape = (None,) + a.shape[1:]

        def __getitem__(self, e):
            return self.a[pos[int(e)]]
    return [View(a) for a in sub]


def rand_routing(M, E, k, seed):
    rng = np.random.default_rng(seed)
    eid = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    logits = rng.standard_normal((M, E)).astype(np.float32)
    w = np.take_along_axis(logits, eid, 1)
    w = np.exp(w - w.max(1, keepdims=True))
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return eid, w


def rand_x(M, H, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, H, generator=g) * scale).to(torch.bfloat16)


# ------------------------------------------------------------------------------------------ grouped GEMM
@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("sizes", [[1, 1, 1, 1, 1, 1, 1, 1], [3, 16, 1, 7], [17, 33, 64], [130, 5]])
def test_grouped_gemm_matches_textbook(tiled, sizes):
    from dsv41_amd import hipkern, quant
    E, N, K = 12, 96, 512
    w13, s13, _, _ = make_experts(E, K, N // 2, 7)
    wk = quant.tile_fp4(w13) if tiled else w13
    sk = quant.tile_fp4_scales(s13) if tiled else s13
    rng = np.random.default_rng(sum(sizes))
    R = 40
    x = quant.fake_quant_fp8(rand_x(R, K, 5).to(DEV))
    ge = rng.choice(E, len(sizes), replace=False).astype(np.int32)
    gs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    P = int(gs[-1])
    tok = rng.integers(0, R, P).astype(np.int32)
    xc, xs = quant.quant_fp8_e8m0(x)
    out = torch.full((P, N), float("nan"), device=DEV)
    t = lambda a: torch.from_numpy(a).to(DEV)
    hipkern.grouped_gemm_codes(xc, xs, wk, sk, t(ge), t(gs), t(tok), out, max(sizes), tiled)
    ref = O.grouped_gemm(bf16_vals(x), w13.cpu().numpy(), s13.cpu().numpy(), ge, gs, tok, len(sizes))
    close(out.cpu().numpy(), ref, f"grouped gemm tiled={tiled} sizes={sizes}")


def test_fp4_gemv_pairs_and_gemm_tc_drop_in():
    from dsv41_amd import hipkern, quant
    E, N, K = 10, 128, 768
    w, s, _, _ = make_experts(E, K, N // 2, 11)
    x = quant.fake_quant_fp8(rand_x(6, K, 12, 2.0).to(DEV))
    row_in = torch.tensor([0, 1, 5, 5, 2, 3], dtype=torch.int32, device=DEV)
    expert = torch.tensor([9, 0, 4, 4, 7, 2], dtype=torch.int32, device=DEV)
    wt = torch.tensor([0.5, 1.0, -2.0, 0.25, 1.5, 3.0], device=DEV)
    out = hipkern.fp4_gemv_pairs(x, w, s, row_in, expert, wt, 6)
    ref = O.gemv_pairs(bf16_vals(x), w.cpu().numpy(), s.cpu().numpy(), row_in.cpu().numpy(), expert.cpu().numpy(), wt.cpu().numpy())
    close(out.cpu().numpy(), ref, "fp4_gemv_pairs")
    # fp4_gemm_tc: permuted x, tiled weights, shard masking with zero_out, out_col into a wider buffer
    wtl, stl = quant.tile_fp4(w), quant.tile_fp4_scales(s)
    xp = hipkern.permute_x(x)
    ge = torch.tensor([2, 4, 7], dtype=torch.int32, device=DEV)
    gs = torch.tensor([0, 2, 5, 6], dtype=torch.int32, device=DEV)
    tok = torch.tensor([0, 3, 1, 2, 4, 5], dtype=torch.int32, device=DEV)
    full = hipkern.fp4_gemm_tc(xp, wtl, stl, ge, gs, tok, 6, 4)
    ref2 = O.grouped_gemm(bf16_vals(x), w.cpu().numpy(), s.cpu().numpy(), ge.cpu().numpy(), gs.cpu().numpy(), tok.cpu().numpy(), 3)
    close(full.cpu().numpy(), ref2, "fp4_gemm_tc")
    wide = torch.full((6, N + 64), 7.0, device=DEV)
    # this shard holds experts [3, 8): its weight tensors are the shard's own experts (ep.py shard layout)
    hipkern.fp4_gemm_tc(xp, wtl[3:8], stl[3:8], ge, gs, tok, 6, 4, shard_start=3, shard_n=5, zero_out=True, out=wide, out_col=64)
    got = wide.cpu().numpy()
    assert np.all(got[:, :64] == 7.0)
    assert np.all(got[0:2, 64:] == 0.0)              # expert 2 is outside [3, 8): rows zeroed
    close(got[2:6, 64:], ref2[2:6], "fp4_gemm_tc shard")


@pytest.mark.parametrize("block_m", [16, 64])
def test_grouped_fp4_gemm_atomic_rows(block_m):
    """N = 64 (not a multiple of 256): the 16-pair grouped kernel, over block_m's own tables (block_m 64: built on
    demand by a second dispatch over the same stable pair order), repeated output rows summed atomically."""
    from dsv41_amd import moe_kernels, quant
    E, N, K = 8, 64, 256
    w, s, _, _ = make_experts(E, K, N // 2, 13)
    a = quant.fake_quant_fp8(rand_x(5, K, 14).to(DEV))
    rng = np.random.default_rng(15)
    P = 40
    eid = torch.from_numpy(rng.integers(0, E, P).astype(np.int32)).to(DEV)
    rin = torch.from_numpy(rng.integers(0, 5, P).astype(np.int32)).to(DEV)
    rout = torch.from_numpy(rng.integers(0, 3, P).astype(np.int32)).to(DEV)   # repeated rows: atomic sums
    wgt = torch.from_numpy(rng.random(P).astype(np.float32)).to(DEV)
    pairs = moe_kernels.GroupedPairs(eid, rin, rout, wgt, block_m, n_experts=E)
    out = moe_kernels.grouped_fp4_gemm(a, w, s, pairs, 3)
    ref = np.zeros((3, N), np.float64)
    ev = eid.cpu().numpy()
    for p in range(P):
        ref[rout[p].item()] += O.gemv_pairs(bf16_vals(a), w.cpu().numpy(), s.cpu().numpy(), [rin[p].item()], [ev[p]], [wgt[p].item()])[0]
    close(out.cpu().numpy(), ref, f"grouped_fp4_gemm atomic block_m={block_m}")


def test_big_groups_on_the_128_pair_tile_kernel():
    """Groups of more than 16 pairs: cukern.fp4_gemm_tc (max_tokens 64, cukern.FP4_W_MAX) and moe_kernels.grouped_fp4_gemm
    (block_m 64, the reference's prefill call, model.py:584-589) run on the 128-pair tile kernel; results equal the
    textbook oracle, with repeated output rows (atomic sums), a group over the 64-pair cap split by the dispatch, and
    dropped (out-of-range) expert ids."""
    from dsv41_amd import hipkern, moe_kernels, quant
    E, N, K = 6, 512, 768
    w, s, _, _ = make_experts(E, K, N // 2, 21)
    wtl, stl = quant.tile_fp4(w), quant.tile_fp4_scales(s)
    X = 90
    x = quant.fake_quant_fp8(rand_x(X, K, 22, 2.0).to(DEV))
    rng = np.random.default_rng(23)
    # fp4_gemm_tc: groups of 64, 40, 17 and 3 pairs over arbitrary token rows
    sizes = [64, 40, 17, 3]
    ge = torch.tensor([4, 0, 5, 2], dtype=torch.int32, device=DEV)
    gs = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), device=DEV)
    P = int(sum(sizes))
    tok = torch.from_numpy(rng.integers(0, X, P).astype(np.int32)).to(DEV)
    assert hipkern.t128_ok(N, K, 64)
    got = hipkern.fp4_gemm_tc(hipkern.permute_x(x), wtl, stl, ge, gs, tok, P, 64)
    ref = O.grouped_gemm(bf16_vals(x), w.cpu().numpy(), s.cpu().numpy(), ge.cpu().numpy(), gs.cpu().numpy(), tok.cpu().numpy(), 4)
    close(got.cpu().numpy(), ref, "fp4_gemm_tc 64-pair groups")
    # grouped_fp4_gemm: 300 pairs, a popular expert (> 64 pairs: split into tiles), repeated output rows, ids out of range
    P2 = 300
    eid = rng.choice(E, P2, p=[0.5, 0.1, 0.1, 0.1, 0.1, 0.1]).astype(np.int32)
    eid[[7, 100]] = [-1, E]                                                 # dropped by the dispatch
    rin = rng.integers(0, X, P2).astype(np.int32)
    rout = rng.integers(0, 50, P2).astype(np.int32)
    wgt = rng.random(P2).astype(np.float32)
    pairs = moe_kernels.GroupedPairs(torch.from_numpy(eid).to(DEV), torch.from_numpy(rin).to(DEV), torch.from_numpy(rout).to(DEV),
                                     torch.from_numpy(wgt).to(DEV), 64, n_experts=E)
    out = moe_kernels.grouped_fp4_gemm(x, wtl, stl, pairs, 50, tiled=True)
    ref = np.zeros((50, N), np.float64)
    xv, wn, sn = bf16_vals(x), w.cpu().numpy(), s.cpu().numpy()
    for p in range(P2):
        if 0 <= eid[p] < E:
            ref[rout[p]] += O.gemv_pairs(xv, wn, sn, [rin[p]], [eid[p]], [wgt[p]])[0]
    close(out.cpu().numpy(), ref, "grouped_fp4_gemm block_m 64")


@pytest.mark.parametrize("K", [768, 4096])
def test_grouped_fp4_gemm_scatter_forms(K):
    """grouped_fp4_gemm through dsv41_fp4_grouped_gemm_scatter (tile kernel into per-pair rows, then the weighted add
    into the output rows), in the reference's prefill call pattern (one output row per pair, model.py:584-589), with a
    popular expert of more than 128 pairs (a 256-pair tile) and ids out of range dropped: with out new the rows are
    stored, with out given they are read, added and written; both equal fl(w_p * y_p) (+ out) bit for bit, y_p the
    unweighted pair rows of the 128-pair tile entry on the same sorted pairs, and the oracle within tolerance. Rows
    shared by pairs take the atomic form, equal to the oracle's sums within tolerance. K = 4096: one column block per
    workgroup (long k-loops)."""
    from dsv41_amd import hipkern, moe_kernels, quant
    E, N = 6, 512
    w, s, _, _ = make_experts(E, K, N // 2, 41)
    wtl, stl = quant.tile_fp4(w), quant.tile_fp4_scales(s)
    X, P, R = 120, 400, 410
    x = quant.fake_quant_fp8(rand_x(X, K, 42, 2.0).to(DEV))
    rng = np.random.default_rng(43)
    eid = rng.choice(E, P, p=[0.5, 0.1, 0.1, 0.1, 0.1, 0.1]).astype(np.int32)
    eid[[3, 250]] = [-1, E + 2]
    rin = rng.integers(0, X, P).astype(np.int32)
    rout = rng.permutation(R)[:P].astype(np.int32)
    wgt = rng.random(P).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(DEV)
    pairs = moe_kernels.GroupedPairs(t(eid), t(rin), t(rout), t(wgt), 64, n_experts=E)
    assert int(pairs.distinct_rows(R)) == 1
    ge, gs = pairs.tables(moe_kernels.TILE_GROUP)
    sizes = np.diff(gs.cpu().numpy())[: int(np.count_nonzero(ge.cpu().numpy() >= 0))]
    assert sizes.max() > 128                                                 # a 256-pair tile
    out = moe_kernels.grouped_fp4_gemm(x, wtl, stl, pairs, R, tiled=True)   # stores
    xc, xs = quant.quant_fp8_e8m0(x)
    g128, s128 = pairs.tables(128)
    y2 = torch.zeros(P, N, device=DEV)
    hipkern.grouped_gemm_t128(xc, xs, wtl, stl, g128, s128, pairs.s_row_in, y2, P, True)
    n = int(gs[-1])
    assert n == P - 2
    rs = pairs.s_row_out[:n].long()
    exp = torch.zeros(R, N, device=DEV)
    exp[rs] = y2[:n] * pairs.s_weight[:n, None]
    assert torch.equal(out, exp)
    out0 = torch.randn(R, N, device=DEV)
    out1 = moe_kernels.grouped_fp4_gemm(x, wtl, stl, pairs, R, out=out0.clone(), tiled=True)   # read, add, write
    exp1 = out0.clone()
    exp1[rs] = out0[rs] + y2[:n] * pairs.s_weight[:n, None]
    assert torch.equal(out1, exp1)
    ref = np.zeros((R, N), np.float64)
    xv, wn, sn = bf16_vals(x).astype(np.float64), w.cpu().numpy(), s.cpu().numpy()
    dense = [O.dense_weights(wn[e], sn[e]).astype(np.float64) for e in range(E)]
    pair_row = lambda p: wgt[p] * (dense[eid[p]] @ xv[rin[p]])
    for p in range(P):
        if 0 <= eid[p] < E:
            ref[rout[p]] += pair_row(p)
    close(out.cpu().numpy(), ref, f"grouped_fp4_gemm distinct rows K={K}")
    # shared output rows: fp32 atomics
    rout2 = (rout % 37).astype(np.int32)
    pairs2 = moe_kernels.GroupedPairs(t(eid), t(rin), t(rout2), t(wgt), 64, n_experts=E)
    assert int(pairs2.distinct_rows(37)) == 0
    out2 = moe_kernels.grouped_fp4_gemm(x, wtl, stl, pairs2, 37, tiled=True)
    ref2 = np.zeros((37, N), np.float64)
    for p in range(P):
        if 0 <= eid[p] < E:
            ref2[rout2[p]] += pair_row(p)
    close(out2.cpu().numpy(), ref2, f"grouped_fp4_gemm shared rows (atomic) K={K}")


def test_rows_distinct_flag():
    """dsv41_rows_distinct: 1 exactly when no two counted entries (the first n_placed, inside [0, out_rows)) repeat a
    row; 0 unchecked past its 2^20-row bitmap."""
    from dsv41_amd import hipkern
    t = lambda a: torch.tensor(np.asarray(a), dtype=torch.int32, device=DEV)

    def f(rows, n_out, placed=None):
        return int(hipkern.rows_distinct(t(rows), len(rows), None if placed is None else t([placed]), n_out))
    assert f([3, 1, 2, 0], 4) == 1
    assert f([3, 1, 3, 0], 4) == 0
    assert f([3, 1, 7, 7], 4) == 1                    # the repeated row lies outside [0, out_rows): never written
    assert f([3, 1, -1, -1], 4) == 1
    assert f([3, 1, 0, 0], 4, placed=3) == 1          # the repeat is past the placed pairs
    assert f([3, 1, 0, 0], 4, placed=4) == 0
    rows = np.random.default_rng(3).permutation(300000)[:50000]
    assert f(rows, 300000) == 1
    rows[49999] = rows[123]
    assert f(rows, 300000) == 0
    assert f([0, 1], (1 << 20) + 1) == 0              # past the bitmap: unchecked, the atomic form


def test_t128_entry_bounds():
    """dsv41_fp4_grouped_gemm_t128: group ranges are clamped to n_pairs, input rows outside [0, x_rows) read zeros (rows of
    y for them are 0), rows of pairs outside every group are left untouched; shape errors return -1 before any launch."""
    from dsv41_amd import _lib, quant
    E, N, K = 3, 256, 384
    w, s, _, _ = make_experts(E, K, N // 2, 31)
    x = quant.fake_quant_fp8(rand_x(8, K, 32).to(DEV))
    xc, xs = quant.quant_fp8_e8m0(x)
    ge = torch.tensor([1, 2], dtype=torch.int32, device=DEV)
    gs = torch.tensor([0, 5, 400], dtype=torch.int32, device=DEV)            # the second range runs past n_pairs
    rows = torch.tensor([0, 3, -4, 8, 7, 1, 2, 100000], dtype=torch.int32, device=DEV)
    y = torch.full((9, N), 5.0, device=DEV)
    # the one-term call, then a raw (off-grid) x with its second term: the MODE 2 pass keeps the same bounds
    xr = rand_x(8, K, 33).to(DEV)
    hc, hs, lc, ls, flag = quant.quant_fp8_split(xr)
    for xv, (c, sc, lo) in ((bf16_vals(x), (xc, xs, (None, None, None))), (bf16_vals(xr), (hc, hs, (_lib.ptr(lc), _lib.ptr(ls), _lib.ptr(flag))))):
        y = torch.full((9, N), 5.0, device=DEV)
        _lib.call("dsv41_fp4_grouped_gemm_t128", _lib.ptr(c), c.stride(0), _lib.ptr(sc), sc.stride(0), 8, *lo, _lib.ptr(rows), _lib.ptr(w),
                  w.stride(0), _lib.ptr(s), s.stride(0), 0, E, N, K, _lib.ptr(ge), _lib.ptr(gs), 2, 8, _lib.ptr(y), N, _lib.stream(DEV))
        got = y.cpu().numpy()
        wn, sn = w.cpu().numpy(), s.cpu().numpy()
        for p in range(8):
            e = 1 if p < 5 else 2
            r = int(rows[p])
            if 0 <= r < 8:
                close(got[p], O.gemv_pairs(xv, wn, sn, [r], [e], [1.0])[0], f"t128 pair {p}")
            else:
                assert np.all(got[p] == 0.0), f"pair {p}: row {r} outside the input must read zeros"
        assert np.all(got[8] == 5.0), "a row past n_pairs is not written"
    bad = lambda **kw: _lib.lib().dsv41_fp4_grouped_gemm_t128(_lib.ptr(xc), xc.stride(0), _lib.ptr(xs), xs.stride(0), 8, None, None, None,
                                                              _lib.ptr(rows),
                                                              _lib.ptr(w), w.stride(0), _lib.ptr(s), s.stride(0), 0, E, kw.get("N", N),
                                                              kw.get("K", K), _lib.ptr(ge), _lib.ptr(gs), 2, 8, _lib.ptr(y), N, _lib.stream(DEV))
    assert bad(N=128) == -1 and bad(K=256) == -1


# ------------------------------------------------------------------------------------------ routing
@pytest.mark.parametrize("M,k,E,gmax", [(1, 8, 384, 64), (4, 8, 384, 64), (16, 8, 384, 64), (16, 8, 16, 4), (129, 8, 384, 64),
                                       (2048, 8, 384, 64), (4096, 8, 384, 64), (300, 6, 48, 16)])
def test_dispatch_tables_exact(M, k, E, gmax):
    from dsv41_amd import hipkern
    eid, wt = rand_routing(M, E, k, M * 7 + E)
    n_groups = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = hipkern.moe_dispatch(torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), k, E, gmax, DEV, n_groups=n_groups)
    tok, wts, inv, ge, gs, G = O.moe_dispatch(eid, wt, k, E, gmax)
    for a, b in zip(got, (tok, wts, inv, ge, gs)):
        assert np.array_equal(a.cpu().numpy(), b)
    assert n_groups.item() == G


@pytest.mark.parametrize("func", ["softmax", "sigmoid", "sqrtsoftplus"])
def test_gate_topk(func):
    from dsv41_amd import fused2
    rng = np.random.default_rng(21)
    sc = (rng.standard_normal((16, 384)) * 2).astype(np.float32)
    bias = (rng.standard_normal(384) * 0.1).astype(np.float32)
    eid, wt = fused2.gate_topk(torch.from_numpy(sc).to(DEV), torch.from_numpy(bias).to(DEV), 1.0, 8, 2.5, func, True)
    ref_i, ref_w = O.gate_topk(sc, bias, 1.0, 8, 2.5, func, True)
    assert np.array_equal(eid.cpu().numpy(), ref_i)
    assert np.allclose(wt.cpu().numpy(), ref_w, rtol=2e-6, atol=0)
    # without renormalisation the raw scores (softmax denominators included) are checked too
    eid2, wt2 = fused2.gate_topk(torch.from_numpy(sc).to(DEV), torch.from_numpy(bias).to(DEV), 1.3, 8, 1.0, func, False)
    ref_i2, ref_w2 = O.gate_topk(sc, bias, 1.3, 8, 1.0, func, False)
    assert np.array_equal(eid2.cpu().numpy(), ref_i2)
    assert np.allclose(wt2.cpu().numpy(), ref_w2, rtol=4e-6, atol=0)
    tied = torch.zeros(1, 64, device=DEV)
    e1, _ = fused2.gate_topk(tied, None, 1.0, 4, 1.0, "softmax", True)
    assert e1.tolist() == [0, 1, 2, 3]
    # NaN scores never win and no index is ever out of range
    nanrow = torch.full((1, 384), float("nan"), device=DEV)
    nanrow[0, 7] = 1.0
    e2, _ = fused2.gate_topk(nanrow, None, 1.0, 8, 1.0, "sigmoid", True)
    assert e2[0].item() == 7 and int(e2.max()) < 384 and int(e2.min()) >= 0


# ------------------------------------------------------------------------------------------ decode experts
@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("M", [1, 2, 4, 16])
@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_decode_experts_small(tiled, M, limit):
    from dsv41_amd import moe, quant
    E, H, I, k = 24, 1024, 256, 8
    ws = make_experts(E, H, I, 100 + M)
    ex = to_ex(*ws, tiled)
    eid, wt = rand_routing(M, E, k, M)
    x = rand_x(M, H, M)
    xq = quant.fake_quant_fp8(x.to(DEV))
    y = moe.moe_experts(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, limit)
    ref = O.moe_layer_routed(bf16_vals(xq), eid, wt, *[w.cpu().numpy() for w in ws], I, limit)
    close(y.cpu().numpy(), ref, f"decode small M={M} tiled={tiled} L={limit}")


@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("M", [1, 3])
def test_decode_experts_wide_hidden(tiled, M):
    """Hidden 8448: a wave's weight stream has 33 k-chunks, more than the up kernel stages scales for in LDS, and
    one token no longer fits the one-token path, so both take the member-pass path with per-tile scale loads."""
    from dsv41_amd import moe, quant
    E, H, I, k = 12, 8448, 256, 4
    ws = make_experts(E, H, I, 500 + M)
    ex = to_ex(*ws, tiled)
    eid, wt = rand_routing(M, E, k, 600 + M)
    xq = quant.fake_quant_fp8(rand_x(M, H, 700 + M).to(DEV))
    y = moe.moe_experts(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, 10.0)
    ref = O.moe_layer_routed(bf16_vals(xq), eid, wt, *[w.cpu().numpy() for w in ws], I, 10.0)
    close(y.cpu().numpy(), ref, f"decode hidden 8448 M={M} tiled={tiled}")


@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("M,I", [(16, 640), (16, 512), (8, 1024), (16, 2048), (16, 2560)])
def test_decode_down_h_rows_global(tiled, M, I):
    """Pair rows too large for LDS (M * 8 + 1 rows of I + I / 32 bytes > 60 KiB): the down projection reads h from
    global memory. I <= 2048 takes the per-group scale loads (I = 640: 20 scale bytes per row, so the 16-byte h scale
    loads of a row overlap; I = 512: exactly 16); I = 2560 (20 k-chunks) the per-tile scale bytes. Checked against the
    oracle's w2 on the kernel's own h (the up projection's FP8 rounding is covered by the tests above), and bit for bit
    against the per-tile scale path on the same h (forced by a 4-byte-misaligned h scale row stride). The one-launch
    kernel (dsv41_moe_down_sum) throughout: at these sizes the default is the run-split form, tested below."""
    import copy
    from dsv41_amd import moe, quant
    E, H, k = 24, 1024, 8
    P, Ks = M * k, I // 32
    w = make_experts(E, H, I, 700 + I + M)
    ex = to_ex(*w, tiled)
    eid, wt = rand_routing(M, E, k, 7 * M)
    xq = quant.fake_quant_fp8(rand_x(M, H, 7 * M).to(DEV))
    ws = moe.decode_up(xq, ex, 10.0, k, eid=torch.from_numpy(eid).to(DEV), wt=torch.from_numpy(wt).to(DEV))
    y = moe.decode_down(ws, ex, split=False).clone()
    ge, gs, tok = ws.grp_expert.cpu().numpy(), ws.grp_start.cpu().numpy(), ws.tok_sorted.cpu().numpy()
    h = _e4m3_values(ws.hc[:P], ws.hs[:P])
    y2 = O.grouped_gemm(h, w[2].cpu().numpy(), w[3].cpu().numpy(), ge, gs, np.arange(P, dtype=np.int32), int(np.count_nonzero(ge >= 0)))
    ref = np.zeros((M, H), np.float64)
    np.add.at(ref, tok[:P], y2)
    close(y.cpu().numpy(), ref, f"decode down, h rows from global, M={M} I={I} tiled={tiled}")
    hs_wide = torch.zeros(P + 1, Ks + 1, dtype=torch.uint8, device=DEV)
    hs_wide[:, :Ks] = ws.hs
    ws2 = copy.copy(ws)
    ws2.hs = hs_wide[:, :Ks]
    y_tile = torch.empty(M, H, dtype=torch.float32, device=DEV)
    moe.decode_down(ws2, ex, y32=y_tile, split=False)
    assert torch.equal(y, y_tile), f"per-group vs per-tile scale loads differ: max {float((y - y_tile).abs().max())}"


@pytest.mark.parametrize("M,I,tiled", [(5, 2048, True), (8, 1024, False), (16, 1024, True)])
def test_decode_down_split_drops_ids_and_post_mix(M, I, tiled):
    """The run-split down projection (dsv41_moe_down_sum_split; taken by default when M > 4 tokens' h rows overflow the
    one-launch kernel's LDS) with ids outside [0, E) (the offload dummy slot E, E + 7, -1): those pairs are dropped and
    the layer matches the oracle with their weights zeroed; it agrees with the one-launch kernel on the same h to fp32
    rounding (its runs' partial sums add in another order); bf16(y + ys) equals the rounding of its own fp32 y bit for
    bit, and its hyper-connection post mix equals hc_post2_ on its own bf16 output bit for bit."""
    from dsv41_amd import fused2, moe, quant
    E, H, k = 32, 1024, 8
    w = make_experts(E, H, I, 880 + M)
    ex = to_ex(*w, tiled)
    eid, wt = rand_routing(M, E, k, 881 + M)
    eid[0, 2], eid[M - 1, 5], eid[M // 2, 0] = E, -1, E + 7
    xq = quant.fake_quant_fp8(rand_x(M, H, 882 + M).to(DEV))
    ws = moe.decode_up(xq, ex, 10.0, k, eid=torch.from_numpy(eid).to(DEV), wt=torch.from_numpy(wt).to(DEV))
    assert moe._down_split(ws, ex)
    y = moe.decode_down(ws, ex).clone()
    valid = (eid >= 0) & (eid < E)
    ref = O.moe_layer_routed(bf16_vals(xq), np.where(valid, eid, 0), np.where(valid, wt, 0).astype(np.float32),
                             *[t.cpu().numpy() for t in w], I, 10.0)
    close(y.cpu().numpy(), ref, f"split down M={M} I={I} tiled={tiled}, dropped ids")
    y1 = torch.empty_like(y)
    moe.decode_down(ws, ex, y32=y1, split=False)
    yn, y1n = y.cpu().numpy(), y1.cpu().numpy()
    rms = float(np.sqrt(np.mean(y1n.astype(np.float64) ** 2)))
    assert np.all(np.abs(yn - y1n) <= 1e-5 * (np.abs(y1n) + rms)), f"split vs one launch: max {np.abs(yn - y1n).max():.3e}"
    rng = np.random.default_rng(883 + M)
    ys = torch.from_numpy(O.f32_to_bf16_bits(rng.standard_normal((M, H)).astype(np.float32)).view(np.int16)).view(torch.bfloat16).to(DEV)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    moe.decode_down(ws, ex, ys=ys, out=out)
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(u16(out), O.f32_to_bf16_bits((yn + bf16_vals(ys)).astype(np.float32)))
    res0 = torch.from_numpy(O.f32_to_bf16_bits(rng.standard_normal((M, 1, 4, H)).astype(np.float32)).view(np.int16)).view(torch.bfloat16).to(DEV)
    post = torch.from_numpy(rng.standard_normal((M, 4)).astype(np.float32)).to(DEV)
    comb = torch.from_numpy(rng.standard_normal((M, 4, 4)).astype(np.float32)).to(DEV)
    res_ref = res0.clone()
    fused2.hc_post2_(out, res_ref, post, comb)
    res = res0.clone()
    moe.decode_down(ws, ex, ys=ys, hc=(res, post, comb))
    torch.cuda.synchronize()
    assert torch.equal(res, res_ref)


@pytest.mark.parametrize("M,func,norm", [(1, "softmax", True), (3, "sigmoid", True), (16, "sqrtsoftplus", True), (5, "softmax", False)])
def test_decode_up_routing_and_tables(M, func, norm):
    """The fused decode entry routes from the logits: its ids / weights equal the standalone gate kernel's (the
    same device code) and the oracle's, its bucketing tables equal moe_dispatch's exactly (one group per
    expert), and the layer output matches the oracle."""
    from dsv41_amd import fused2, moe, quant
    E, H, I, k = 384, 512, 128, 8
    ws = make_experts(E, H, I, 300 + M)
    ex = to_ex(*ws, True)
    rng = np.random.default_rng(M)
    logits = (rng.standard_normal((M, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    lg, bs = torch.from_numpy(logits).to(DEV), torch.from_numpy(bias).to(DEV)
    xq = quant.fake_quant_fp8(rand_x(M, H, 7 + M).to(DEV))
    eo = torch.full((M, k), -7, dtype=torch.int32, device=DEV)
    wo = torch.empty(M, k, device=DEV)
    y = moe.moe_route_experts(xq, lg, bs, 1.0, k, 2.5, func, norm, ex, 10.0, eid_out=eo, wt_out=wo)
    ge_i, ge_w = fused2.gate_topk(lg, bs, 1.0, k, 2.5, func, norm, eid=torch.empty_like(eo), wt=torch.empty_like(wo))
    assert torch.equal(eo, ge_i) and torch.equal(wo, ge_w)
    eid, wt = O.gate_topk(logits, bias, 1.0, k, 2.5, func, norm)
    assert np.array_equal(eo.cpu().numpy(), eid)
    assert np.allclose(wo.cpu().numpy(), wt, rtol=4e-6, atol=0)
    w_dev = wo.cpu().numpy()
    tok, wts, _, g_e, g_s, _ = O.moe_dispatch(eid, w_dev, k, E, 16)
    wsp = moe._WS[(DEV, M, k, H, I)]
    if 1 < M <= moe.PAIRS_MAX_M:
        # routed pair by pair: group p = pair p alone (token p // k, its pick p % k)
        P = M * k
        pair_tables = ((wsp.tok_sorted, np.arange(P) // k), (wsp.wt_sorted, w_dev.reshape(-1)), (wsp.grp_expert, eid.reshape(-1)),
                       (wsp.grp_start, np.arange(P + 1)))
        for got, ref_p in pair_tables:
            assert np.array_equal(got.cpu().numpy(), ref_p)
    else:
        for got, ref in ((wsp.tok_sorted, tok), (wsp.wt_sorted, wts), (wsp.grp_expert, g_e), (wsp.grp_start, g_s)):
            assert np.array_equal(got.cpu().numpy(), ref)
    ref = O.moe_layer_routed(bf16_vals(xq), eid, w_dev, *[w.cpu().numpy() for w in ws], I, 10.0)
    close(y.cpu().numpy(), ref, f"decode routed from logits M={M} {func}")
    # the up-projection launch routing all M tokens itself (moe_route_experts uses it at M = 1 only)
    eo2, wo2 = torch.full_like(eo, -7), torch.empty_like(wo)
    wsp2 = moe.decode_up(xq, ex, 10.0, k, logits=lg, gate=(bs, 1.0, 2.5, func, norm), eid_out=eo2, wt_out=wo2)
    assert torch.equal(eo2, eo) and torch.equal(wo2, wo)
    for got, ref_t in ((wsp2.tok_sorted, tok), (wsp2.wt_sorted, wts), (wsp2.grp_expert, g_e), (wsp2.grp_start, g_s)):
        assert np.array_equal(got.cpu().numpy(), ref_t)
    y2 = moe.decode_down(wsp2, ex)
    if 1 < M <= moe.PAIRS_MAX_M:   # pairs sum a token's experts in pick order, the bucketed form in expert order
        assert O.rel_l2(y2.cpu().numpy(), y.cpu().numpy()) < 1e-5
    else:
        assert torch.equal(y2, y)


@pytest.mark.parametrize("M", [2, 3, 8, 16])
@pytest.mark.parametrize("given", [False, True])
def test_decode_up_pairs(M, given):
    """dsv41_moe_decode_up_pairs: routing from the logits (or given ids / weights), one group per (token, pick) pair with
    its h row p; ids and weights equal the gate kernel's exactly, tables are the pair identity, the layer equals the
    bucketed launch's (sums in pick order instead of expert order) and the oracle's. Tokens that share experts (here
    many, E = 24) read them once per pair."""
    from dsv41_amd import fused2, moe, quant
    E, H, I, k = 24, 512, 128, 6
    ws = make_experts(E, H, I, 500 + M)
    ex = to_ex(*ws, True)
    rng = np.random.default_rng(600 + M)
    lg = torch.from_numpy((rng.standard_normal((M, E)) * 2).astype(np.float32)).to(DEV)
    xq = quant.fake_quant_fp8(rand_x(M, H, 9 + M).to(DEV))
    gate = (None, 1.0, 1.0, "softmax", True)
    ei, wi = fused2.gate_topk(lg, None, 1.0, k, 1.0, "softmax", True, eid=torch.empty(M, k, dtype=torch.int32, device=DEV),
                              wt=torch.empty(M, k, device=DEV))
    eo, wo = torch.full((M, k), -7, dtype=torch.int32, device=DEV), torch.empty(M, k, device=DEV)
    if given:
        wsp = moe.decode_up(xq, ex, 10.0, k, eid=ei, wt=wi, pairs=True)
    else:
        wsp = moe.decode_up(xq, ex, 10.0, k, logits=lg, gate=gate, eid_out=eo, wt_out=wo, pairs=True)
        assert torch.equal(eo, ei) and torch.equal(wo, wi)
    P = M * k
    e_np, w_np = ei.cpu().numpy(), wi.cpu().numpy()
    assert np.array_equal(wsp.grp_expert.cpu().numpy(), e_np.reshape(-1))
    assert np.array_equal(wsp.grp_start.cpu().numpy(), np.arange(P + 1))
    assert np.array_equal(wsp.tok_sorted.cpu().numpy(), np.arange(P) // k)
    assert np.array_equal(wsp.wt_sorted.cpu().numpy(), w_np.reshape(-1))
    y = moe.decode_down(wsp, ex).clone()
    yb = moe.moe_experts(xq, ei, wi, ex, 10.0)
    assert O.rel_l2(y.cpu().numpy(), yb.cpu().numpy()) < 1e-5
    ref = O.moe_layer_routed(bf16_vals(xq), e_np, w_np, *[w.cpu().numpy() for w in ws], I, 10.0)
    close(y.cpu().numpy(), ref, f"decode pairs M={M} given={given}")


@pytest.fixture(scope="module")
def full_layer():
    """configs[1..2] expert shapes: 384 experts, hidden 7168, intermediate 1664 (7.3 GB packed, tiled)."""
    E, H, I = 384, 7168, 1664
    ws = make_experts(E, H, I, 2024)
    ex = to_ex(*ws, True)
    yield E, H, I, ws, ex
    del ex


@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_decode_full_m1_vs_oracle(full_layer, limit):
    from dsv41_amd import moe, quant
    E, H, I, ws, ex = full_layer
    eid, wt = rand_routing(1, E, 8, 5)
    eid[0, 0] = 383                                    # the last expert: > 4 GiB offsets into the weights
    x = rand_x(1, H, 6)
    xq = quant.fake_quant_fp8(x.to(DEV))
    y = moe.moe_experts(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, limit)
    W13, S13, W2, S2 = host_subset(ws, set(eid.reshape(-1).tolist()))
    ref = O.moe_layer_routed(bf16_vals(xq), eid, wt, W13, S13, W2, S2, I, limit)
    close(y.cpu().numpy(), ref, f"decode configs[1] M=1 L={limit}")


@pytest.mark.parametrize("M", [4, 8, 16])
def test_decode_full_batched_equals_single(full_layer, M):
    """a batched step equals M single-token steps (the reference's test_rows.py strategy), and one
    token is checked against the oracle."""
    from dsv41_amd import moe, quant
    E, H, I, ws, ex = full_layer
    eid, wt = rand_routing(M, E, 8, 40 + M)
    xq = quant.fake_quant_fp8(rand_x(M, H, 50 + M).to(DEV))
    ed, wd = torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)
    yb = moe.moe_experts(xq, ed, wd, ex, 10.0).clone()
    for t in range(M):
        ys = moe.moe_experts(xq[t:t + 1].contiguous(), ed[t:t + 1].contiguous(), wd[t:t + 1].contiguous(), ex, 10.0)
        assert O.rel_l2(yb[t].cpu().numpy(), ys[0].cpu().numpy()) < 1e-5
    t = M - 1
    W13, S13, W2, S2 = host_subset(ws, set(eid[t].tolist()))
    ref = O.moe_layer_routed(bf16_vals(xq[t:t + 1]), eid[t:t + 1], wt[t:t + 1], W13, S13, W2, S2, I, 10.0)
    close(yb[t:t + 1].cpu().numpy(), ref, f"decode configs[2] M={M} token {t}")


def test_decode_full_shared_experts_multipass(full_layer):
    """Every token of a 16-token step picks the same 8 experts: each group holds 16 members, more than the LDS rows
    the up kernel stages at hidden 7168, so it streams each expert in several passes (and the down kernel takes
    its unstaged path). Batched equals single-token steps, and one token matches the oracle."""
    from dsv41_amd import moe, quant
    E, H, I, ws, ex = full_layer
    M = 16
    eid1, _ = rand_routing(1, E, 8, 77)
    eid = np.repeat(eid1, M, axis=0)
    wt = np.random.default_rng(78).random((M, 8)).astype(np.float32)
    xq = quant.fake_quant_fp8(rand_x(M, H, 79).to(DEV))
    ed, wd = torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)
    yb = moe.moe_experts(xq, ed, wd, ex, 10.0).clone()
    for t in (0, 7, 15):
        ys = moe.moe_experts(xq[t:t + 1].contiguous(), ed[t:t + 1].contiguous(), wd[t:t + 1].contiguous(), ex, 10.0)
        assert O.rel_l2(yb[t].cpu().numpy(), ys[0].cpu().numpy()) < 1e-5
    W13, S13, W2, S2 = host_subset(ws, set(eid1[0].tolist()))
    ref = O.moe_layer_routed(bf16_vals(xq[9:10]), eid[9:10], wt[9:10], W13, S13, W2, S2, I, 10.0)
    close(yb[9:10].cpu().numpy(), ref, "decode configs[2] shape, 16 members per group, token 9")


def test_decode_layer_with_shared_expert_and_router(full_layer):
    """Whole layer: router GEMV (bf16 [384, 7168]) -> softmax top-8 -> shared bf16 SwiGLU + routed experts ->
    bf16(sum + ys). Each stage against the oracle in fp32 (the tolerance is defined on fp32 outputs), and the
    final bf16 rounding bit-exactly against the composition of the stages."""
    from dsv41_amd import moe
    E, H, I, ws, ex = full_layer
    g = torch.Generator(device=DEV).manual_seed(77)
    Ws13 = (torch.randn(2 * I, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16)
    Ws2 = (torch.randn(H, I, generator=g, device=DEV) / I ** 0.5).to(torch.bfloat16)
    G = (torch.randn(E, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16)
    layer = moe.MoEDecodeLayer(ex, Ws13, Ws2, 10.0, topk=8, score_func="softmax", router=G)
    x = rand_x(1, H, 78).to(DEV)
    y = layer(x).clone()
    b = layer._bufs[1]
    # routing
    logits = (x.float().cpu() @ G.float().cpu().T).numpy()
    assert np.allclose(b["logits"].cpu().numpy(), logits, rtol=1e-4, atol=1e-4)
    eid, wt = O.gate_topk(logits, None, 1.0, 8, 1.0, "softmax", True)
    assert np.array_equal(b["eid"].cpu().numpy(), eid)
    assert np.allclose(b["wt"].cpu().numpy(), wt, rtol=1e-4)
    # shared expert (bf16 output)
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    xq = bf16_vals(b["xq"])
    assert np.array_equal(xq, O.fake_quant_fp8(bf16_vals(x)))
    ys_ref = O.shared_expert(xq, u16(Ws13), u16(Ws2), I, 10.0)
    close(bf16_vals(b["ys"]), ys_ref, "shared expert")
    # routed experts in fp32
    y32 = torch.empty(1, H, device=DEV)
    out = torch.empty(1, H, dtype=torch.bfloat16, device=DEV)
    moe.moe_experts(b["xq"], b["eid"], b["wt"], ex, 10.0, ys=b["ys"], out=out, y32=y32)
    W13, S13, W2, S2 = host_subset(ws, set(eid.reshape(-1).tolist()))
    routed_ref = O.moe_layer_routed(xq, eid, b["wt"].cpu().numpy(), W13, S13, W2, S2, I, 10.0)
    close(y32.cpu().numpy(), routed_ref, "routed experts fp32")
    close(y32.cpu().numpy() + bf16_vals(b["ys"]), routed_ref + ys_ref, "layer fp32 (routed + shared)")
    # final rounding: out = bf16(y32 + ys) exactly, and the layer call produced the same bits
    comp = O.f32_to_bf16_bits((y32.cpu().numpy() + bf16_vals(b["ys"])).astype(np.float32))
    assert np.array_equal(u16(out), comp) and torch.equal(out, y)


def test_graph_capture_replay(full_layer):
    """The decode layer captured in a graph replays correctly several times, with eager work in between."""
    from dsv41_amd import moe, quant
    E, H, I, ws, ex = full_layer
    M = 4
    eid, wt = rand_routing(M, E, 8, 91)
    xq = quant.fake_quant_fp8(rand_x(M, H, 92).to(DEV))
    ed, wd = torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())           # inputs were produced on the current stream
    with torch.cuda.stream(s):
        moe.moe_experts(xq, ed, wd, ex, 10.0, out=out)   # warm-up (workspaces allocated outside capture)
    torch.cuda.synchronize()
    eager = out.clone()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        moe.moe_experts(xq, ed, wd, ex, 10.0, out=out)
    for i in range(3):
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        moe.moe_experts(xq, ed, wd, ex, 0.0)            # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("M,with_y", [(1, True), (1, False), (5, True)])
def test_router_logits_fused_step(M, with_y):
    """The stack's fused router launch: xn / xq against the oracle's layer-to-layer step, the split-K logits
    against a dense matmul of the kernel's own xn, and the gate over the partial sums (added in part order)
    against the oracle gate on the same sums."""
    from dsv41_amd import fused2, moe
    E, H, k = 384, 7168, 8
    g = torch.Generator(device=DEV).manual_seed(300 + M)
    G = (torch.randn(E, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16)
    x = (torch.randn(M, H, generator=g, device=DEV) * 2).to(torch.bfloat16)
    y = torch.randn(M, H, generator=g, device=DEV).to(torch.bfloat16) if with_y else None
    part, xn, xq = moe.router_logits(x, y, G)
    yv = bf16_vals(y) if with_y else np.zeros((M, H), np.float32)
    ref_n, _ = O.residual_rmsnorm_quant(bf16_vals(x), yv, None, 1e-6)
    got_n = bf16_vals(xn)
    assert np.all(np.abs(got_n - ref_n) <= np.abs(ref_n) * 2.0 ** -7 + 1e-30) and (got_n == ref_n).mean() > 0.99
    assert np.array_equal(bf16_vals(xq), O.fake_quant_fp8(got_n))
    parts = part.cpu().numpy()
    summed = np.zeros((M, E), np.float32)
    for p in range(parts.shape[0]):
        summed = (summed + parts[p]).astype(np.float32)
    dense = got_n.astype(np.float64) @ bf16_vals(G).astype(np.float64).T
    assert np.allclose(summed, dense, rtol=1e-4, atol=1e-4)
    eid, wt = fused2.gate_topk(part, None, 1.0, k, 1.0, "softmax", True, eid=torch.empty(M, k, dtype=torch.int32, device=DEV),
                               wt=torch.empty(M, k, device=DEV))
    ref_i, ref_w = O.gate_topk(summed, None, 1.0, k, 1.0, "softmax", True)
    assert np.array_equal(eid.cpu().numpy(), ref_i)
    assert np.allclose(wt.cpu().numpy(), ref_w, rtol=4e-6, atol=0)


# ------------------------------------------------------------------------------------------ prefill
def _skewed_routing(T, E, k, hot, seed):
    """Every token routes to expert `hot` plus k - 1 others (so `hot` spans several 128-pair groups)."""
    rng = np.random.default_rng(seed)
    eid = np.stack([rng.permutation(np.concatenate([[hot], rng.choice([e for e in range(E) if e != hot], k - 1, replace=False)]))
                    for _ in range(T)]).astype(np.int32)
    lg = rng.standard_normal((T, k)).astype(np.float32)
    wt = (np.exp(lg) / np.exp(lg).sum(1, keepdims=True)).astype(np.float32)
    return eid, wt


def _e4m3_values(codes, scales):
    c = codes.cpu().numpy()
    s = O.e8m0_to_f32(scales.cpu().numpy())
    return O.e4m3_decode(c) * np.repeat(s, 32, axis=1)


def test_prefill_group_order_changes_nothing_but_the_order():
    """dsv41_group_order: a permutation of the groups by pair count, largest first (padding and dropped groups last). Both
    prefill launches write the same h codes, E8M0 bytes and y2 rows bit for bit with it as in table order (each item writes
    its own rows), here with groups of a few pairs up to full 256-pair ones on both tile kernels."""
    from dsv41_amd import _lib, moe, quant
    E, I, H, k, T = 64, 384, 512, 6, 700
    ws = make_experts(E, H, I, 611)
    ex = to_ex(*ws, True)
    rng = np.random.default_rng(13)   # Zipf(1.1) popularity: groups from a few pairs up to full 256-pair ones
    pop = 1.0 / np.arange(1, E + 1) ** 1.1
    pop = pop[rng.permutation(E)] / pop.sum()
    eid = np.stack([rng.choice(E, k, replace=False, p=pop) for _ in range(T)]).astype(np.int32)
    wt = rng.random((T, k)).astype(np.float32)
    xq = quant.fake_quant_fp8(rand_x(T, H, 12).to(DEV))
    st = moe.prefill_up(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, 10.0)   # w13 in size order
    moe.prefill_down(st, ex)                                                                         # w2 in table order
    P, G, dev = T * k, st.G, xq.device
    order = torch.empty(G, dtype=torch.int32, device=dev)
    _lib.call("dsv41_group_order", _lib.ptr(st.grp_expert), _lib.ptr(st.grp_start), G, P, _lib.ptr(order), _lib.stream(dev))
    o = order.cpu().numpy()
    ge, gs = st.grp_expert.cpu().numpy()[:G], st.grp_start.cpu().numpy()
    cnt = np.where(ge >= 0, np.clip(gs[1:G + 1], 0, P) - np.clip(gs[:G], 0, P), 0)
    assert sorted(o.tolist()) == list(range(G))
    assert np.all(np.diff(np.minimum(cnt[o], 256)) <= 0), "not largest first"
    assert cnt.max() > 128 and (cnt[cnt > 0] <= 16).any()
    hc, hs, y2 = st.hc.clone(), st.hs.clone(), st.y2.clone()
    xc, xs = quant.quant_fp8_e8m0(xq)

    def up(order_ptr):
        st.hc.zero_(); st.hs.zero_()
        _lib.call("dsv41_prefill_up", _lib.ptr(xc), xc.stride(0), _lib.ptr(xs), xs.stride(0), T, _lib.ptr(ex.w13), ex.w13.stride(0),
                  _lib.ptr(ex.s13), ex.s13.stride(0), 1, E, H, I, _lib.ptr(st.grp_expert), _lib.ptr(st.grp_start), G, _lib.ptr(st.tok_sorted),
                  _lib.ptr(st.wt_sorted), 10.0, _lib.ptr(st.hc), st.hc.stride(0), _lib.ptr(st.hs), st.hs.stride(0), order_ptr, _lib.stream(dev))

    def down(order_ptr):
        st.y2.zero_()
        _lib.call("dsv41_prefill_down", _lib.ptr(st.hc), st.hc.stride(0), _lib.ptr(st.hs), st.hs.stride(0), P, _lib.ptr(ex.w2), ex.w2.stride(0),
                  _lib.ptr(ex.s2), ex.s2.stride(0), 1, E, H, I, _lib.ptr(st.grp_expert), _lib.ptr(st.grp_start), G, _lib.ptr(st.y2),
                  st.y2.stride(0), order_ptr, _lib.stream(dev))

    up(None)                                                  # table order
    assert torch.equal(st.hc, hc) and torch.equal(st.hs, hs)
    down(_lib.ptr(order))                                     # size order
    assert torch.equal(st.y2, y2)


@pytest.mark.parametrize("tiled", [True, False])
@pytest.mark.parametrize("limit", [10.0, 0.0])
@pytest.mark.parametrize("H", [512, 768])
def test_prefill_stages_vs_oracle(tiled, limit, H):
    """Prefill stage by stage (T = 300 tokens, top-4 of 16 experts, expert 3 in every token: 300 pairs = several
    groups, the last one partial). h: the oracle's SwiGLU + fq8 of gu = x . deq(W13)^T, element for element, except where fp32
    summation order moves a value across an E4M3 rounding boundary (one code step, rare). y2: fp64 product of the
    kernel's own h with deq(W2), tolerance of the spec. Combine: slot-ordered sum, bit-exact. H = 768: three 256-row
    column blocks in w2, so a workgroup taking two column blocks also meets one with a single block."""
    from dsv41_amd import moe, quant
    E, I, k, T = 16, 384, 4, 300
    ws = make_experts(E, H, I, 500 + int(tiled))
    ex = to_ex(*ws, tiled)
    eid, wt = _skewed_routing(T, E, k, 3, 7)
    xq = quant.fake_quant_fp8(rand_x(T, H, 8).to(DEV))
    st = moe.prefill_up(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, limit)
    tok = st.tok_sorted.cpu().numpy()
    ge, gs = st.grp_expert.cpu().numpy(), st.grp_start.cpu().numpy()
    assert np.count_nonzero(ge == 3) == -(-T // moe.PREFILL_GROUP) > 1
    W13, S13, W2, S2 = [w.cpu().numpy() for w in ws]
    x = bf16_vals(xq)
    gu = O.grouped_gemm(x, W13, S13, ge, gs, tok, int(np.count_nonzero(ge >= 0))).astype(np.float32)
    h_ref = O.swiglu_quant(gu, st.wt_sorted.cpu().numpy(), I, limit)
    h = _e4m3_values(st.hc, st.hs)
    diff = h != h_ref
    assert diff.mean() < 2e-3, f"{diff.mean():.2e} of h differs"
    assert np.all(np.abs(h - h_ref)[diff] <= np.abs(h_ref)[diff] * 0.25 + 2.0 ** -9 * np.abs(h_ref).max())
    y = moe.prefill_down(st, ex)
    y2_ref = O.grouped_gemm(h, W2, S2, ge, gs, np.arange(T * k, dtype=np.int32), int(np.count_nonzero(ge >= 0)))
    close(st.y2.cpu().numpy(), y2_ref, f"prefill w2 tiled={tiled} L={limit}")
    inv = st.inv.cpu().numpy().reshape(T, k)
    y2 = st.y2.cpu().numpy()
    comb = np.zeros((T, H), np.float32)
    for j in range(k):
        comb = (comb + y2[inv[:, j]]).astype(np.float32)
    assert np.array_equal(y.cpu().numpy(), comb)
    # bf16 output with a shared-expert term equals bf16(y32 + ys)
    ys = rand_x(T, H, 9).to(DEV)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    y32 = torch.empty(T, H, device=DEV)
    moe.prefill_experts(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, limit, ys=ys, out=out, y32=y32)
    assert torch.equal(y32, y)
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), O.f32_to_bf16_bits((y32.cpu().numpy() + bf16_vals(ys)).astype(np.float32)))


def test_prefill_layer_vs_oracle():
    """End to end at the benchmark's intermediate size (I = 1664, hidden 512, 16 experts, 300 tokens, top-8)."""
    from dsv41_amd import moe, quant
    E, H, I, k, T = 16, 512, 1664, 8, 300
    ws = make_experts(E, H, I, 600)
    ex = to_ex(*ws, True)
    eid, wt = _skewed_routing(T, E, k, 5, 11)
    xq = quant.fake_quant_fp8(rand_x(T, H, 12).to(DEV))
    y = moe.prefill_experts(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, 10.0)
    ref = O.moe_layer_routed(bf16_vals(xq), eid, wt, *[w.cpu().numpy() for w in ws], I, 10.0)
    close(y.cpu().numpy(), ref, "prefill layer I=1664")


# ------------------------------------------------------------------------------------------ benchmark configs at full shape
def test_configs0_single_gemv_full_shape():
    """one FP4 GEMV, W [2048 x 4096] E2M1 (uniform nibbles), E8M0 scale bytes 119..123, x [1 x 4096] N(0,1)
    bf16 -> fq8, fp32 accumulation -> bf16 output, through the reference's fp4_gemv_pairs surface (one pair), both
    weight layouts."""
    from dsv41_amd import hipkern, quant
    N, K = 2048, 4096
    g = torch.Generator(device=DEV).manual_seed(2048)
    w = torch.randint(0, 256, (1, N, K // 2), generator=g, dtype=torch.uint8, device=DEV)
    s = torch.randint(119, 124, (1, N, K // 32), generator=g, dtype=torch.uint8, device=DEV)
    x = quant.fake_quant_fp8(rand_x(1, K, 4096).to(DEV))
    one = torch.zeros(1, dtype=torch.int32, device=DEV)
    ref = O.gemv_pairs(bf16_vals(x), w.cpu().numpy(), s.cpu().numpy(), [0], [0], [1.0])
    for tiled in (False, True):
        wk = quant.tile_fp4(w) if tiled else w
        sk = quant.tile_fp4_scales(s) if tiled else s
        out = hipkern.fp4_gemv_pairs(x, wk, sk, one, one, torch.ones(1, device=DEV), 1, tiled=tiled)
        close(out.cpu().numpy(), ref, f"configs[0] GEMV tiled={tiled}")
        # the bf16 output: fp32 summation order may move a value across a rounding boundary, so outputs agree
        # bit for bit except for rare differences of one bf16 ulp plus the fp32 error (which dominates near zero)
        ob, rb = O.bf16_round(out.cpu().numpy()), O.bf16_round(ref)
        tol = np.maximum(np.abs(ob), np.abs(rb)) * 2.0 ** -7 + 1e-4 * np.sqrt(np.mean(ref.astype(np.float64) ** 2))
        assert (ob == rb).mean() > 0.99 and np.all(np.abs(ob - rb) <= tol)


def test_configs3_prefill_full_shape(full_layer):
    """2048 tokens x top-8 over 384 experts with Zipf(1.1) popularity (the benchmark's own routing),
    hidden 7168, intermediate 1664, tiled weights: every expert touched, the busiest spread over many 128-pair groups
    (56-step k-loops). Sampled tokens (including tokens of the busiest expert) against the oracle, and against the
    decode path on the same token."""
    from bench import zipf_routing
    from dsv41_amd import moe, quant
    E, H, I, ws, ex = full_layer
    T, k = 2048, 8
    eid, wt = zipf_routing(T, 31)
    counts = np.bincount(eid.reshape(-1), minlength=E)
    hot = int(counts.argmax())
    assert counts[hot] > 1000 and (counts > 0).sum() == E
    xq = quant.fake_quant_fp8(rand_x(T, H, 3100).to(DEV))
    ed, wd = torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)
    y = moe.prefill_experts(xq, ed, wd, ex, 10.0).cpu().numpy()
    hot_toks = np.nonzero((eid == hot).any(1))[0]
    sample = sorted(set([int(hot_toks[0]), int(hot_toks[len(hot_toks) // 2]), int(hot_toks[-1]), 0, 777, T - 1]))
    ids = set(eid[sample].reshape(-1).tolist())
    W13, S13, W2, S2 = host_subset(ws, ids)
    xv = bf16_vals(xq[sample])
    ref = O.moe_layer_routed(xv, eid[sample], wt[sample], W13, S13, W2, S2, I, 10.0)
    for i, t in enumerate(sample):
        close(y[t], ref[i], f"configs[3] prefill token {t}")
    # the decode path (M <= 16) on the sampled tokens agrees within the same tolerance
    yd = moe.moe_experts(xq[sample].contiguous(), ed[sample].contiguous(), wd[sample].contiguous(), ex, 10.0).cpu().numpy()
    close(y[sample], yd, "configs[3] prefill vs decode on the sampled tokens")


def test_configs4_stack_graph_equals_eager():
    """configs[4] shape (4 independent 384-expert layers here; the benchmark runs 20): per layer the fused router
    launch (residual + RMSNorm + FP8 quant + split-K logits, 7 partial sums) then the routed experts with the routing
    done inside the up launch from those partial sums (the M = 1 early path). The captured graph equals eager
    layer-by-layer on every replay; layer 0's routing equals the oracle gate on the summed parts and its output the
    oracle layer."""
    from dsv41_amd import moe
    E, H, I, L, k = 384, 7168, 1664, 4, 8
    layers, raw0 = [], None
    for l in range(L):
        w = make_experts(E, H, I, 4000 + l)
        if l == 0:
            raw0 = w
        layers.append(to_ex(*w, True))
    g = torch.Generator(device=DEV).manual_seed(4100)
    routers = [(torch.randn(E, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16) for _ in range(L)]
    x0 = rand_x(1, H, 4101).to(DEV)
    xs = [x0.clone(), torch.empty_like(x0)]
    xq = torch.empty_like(x0)
    y = torch.zeros_like(x0)
    part = torch.empty(H // 1024, 1, E, dtype=torch.float32, device=DEV)
    eids = torch.empty(L, 1, k, dtype=torch.int32, device=DEV)
    wts = torch.empty(L, 1, k, dtype=torch.float32, device=DEV)
    parts0 = torch.empty_like(part)
    xq0 = torch.empty_like(x0)
    y0_32 = torch.empty(1, H, device=DEV)
    outs = torch.empty(L, 1, H, dtype=torch.bfloat16, device=DEV)

    def run():
        xs[0].copy_(x0)
        y.zero_()
        for l in range(L):
            moe.router_logits(xs[l % 2], y, routers[l], None, 1e-6, part=part, xn=xs[(l + 1) % 2], xq=xq)
            if l == 0:
                parts0.copy_(part)
                xq0.copy_(xq)
            moe.moe_route_experts(xq, part, None, 1.0, k, 1.0, "softmax", True, layers[l], 10.0, out=y, eid_out=eids[l], wt_out=wts[l],
                                  y32=y0_32 if l == 0 else None)
            outs[l].copy_(y)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.synchronize()
    eager = (outs.clone(), eids.clone(), wts.clone())
    # layer 0 routing: the up launch's gate over the 7 partial sums equals the oracle gate on the summed parts
    pp = parts0.cpu().numpy()
    summed = np.zeros((1, E), np.float32)
    for p in range(pp.shape[0]):
        summed = (summed + pp[p]).astype(np.float32)
    ref_i, ref_w = O.gate_topk(summed, None, 1.0, k, 1.0, "softmax", True)
    assert np.array_equal(eids[0].cpu().numpy(), ref_i)
    assert np.allclose(wts[0].cpu().numpy(), ref_w, rtol=4e-6, atol=0)
    W13, S13, W2, S2 = host_subset(raw0, set(ref_i.reshape(-1).tolist()))
    ref0 = O.moe_layer_routed(bf16_vals(xq0), ref_i, wts[0].cpu().numpy(), W13, S13, W2, S2, I, 10.0)
    close(y0_32.cpu().numpy(), ref0, "configs[4] layer 0")   # the spec tolerance is on the fp32 output
    assert np.array_equal(bf16_vals(outs[0]), O.bf16_round(y0_32.cpu().numpy()))
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        run()
    for i in range(3):
        outs.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs, eager[0]) and torch.equal(eids, eager[1]) and torch.equal(wts, eager[2]), f"replay {i}"
        moe.router_logits(x0, None, routers[0], None, 1e-6)   # eager work between replays
        torch.cuda.synchronize()
    del layers


def test_dispatch_drops_invalid_ids_and_combine_skips_them():
    """Ids outside [0, E) are dropped by the dispatch: tables equal the oracle's (inv = -1, padding at the placed
    count), and the combine leaves dropped pairs out of a token's sum."""
    from dsv41_amd import _lib, hipkern
    E, k, T = 16, 4, 300
    rng = np.random.default_rng(5)
    eid = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    eid[3, 1] = -1
    eid[10, 0] = E
    eid[299, 3] = 1 << 20
    wt = rng.random((T, k)).astype(np.float32)
    got = hipkern.moe_dispatch(torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), k, E, 64, DEV)
    ref = O.moe_dispatch(eid, wt, k, E, 64)
    for a, b in zip(got, ref[:5]):
        assert np.array_equal(a.cpu().numpy(), b)
    tok, wts, inv, ge, gs = got
    H = 64
    y2 = torch.randn(T * k, H, device=DEV)
    y = torch.empty(T, H, device=DEV)
    _lib.call("dsv41_combine_pairs", _lib.ptr(y2), H, _lib.ptr(inv), k, T, H, None, H, None, H, _lib.ptr(y), H, _lib.stream(DEV))
    invn, y2n = inv.cpu().numpy().reshape(T, k), y2.cpu().numpy()
    ref_y = np.zeros((T, H), np.float32)
    for j in range(k):
        ref_y = (ref_y + np.where(invn[:, j:j + 1] >= 0, y2n[np.maximum(invn[:, j], 0)], 0)).astype(np.float32)
    assert np.array_equal(y.cpu().numpy(), ref_y)


def test_grouped_gemm_bounds():
    """The generic grouped GEMM's bounds: a pair whose token row is outside [0, x_rows) gives zeros, a group whose
    expert is outside the shard is skipped (rows untouched without zero_out), ranges past n_pairs are clamped."""
    from dsv41_amd import hipkern, quant
    E, N, K = 6, 64, 256
    w, s, _, _ = make_experts(E, K, N // 2, 13)
    x = quant.fake_quant_fp8(rand_x(4, K, 14).to(DEV))
    xc, xs = quant.quant_fp8_e8m0(x)
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=DEV)
    ge, gs, tok = t([1, 9, 3]), t([0, 2, 3, 100]), t([0, 7, 2, 3, 1])
    out = torch.full((5, N), 5.0, device=DEV)
    hipkern.grouped_gemm_codes(xc, xs, w, s, ge, gs, tok, out, 16, False)
    ref = O.grouped_gemm(bf16_vals(x), w.cpu().numpy(), s.cpu().numpy(), np.array([1, 1, 3]), np.array([0, 2, 3, 5]),
                         np.array([0, 0, 2, 3, 1]), 3)
    got = out.cpu().numpy()
    close(got[0], ref[0], "in-range pair")
    assert np.all(got[1] == 0.0)          # token 7 of 4 rows: zeros
    assert np.all(got[2] == 5.0)          # expert 9 of 6: skipped, untouched
    close(got[3:5], ref[3:5], "range clamped to n_pairs")


@pytest.mark.parametrize("M,tiled", [(1, True), (2, True), (1, False)])
def test_decode_fused_shared_expert(full_layer, M, tiled):
    """The bf16 shared expert riding in the two decode launches (its gate/up row blocks in the up launch, its down
    projection in each down-launch workgroup): ys against the oracle's shared expert (bf16 gate/up, model.py:409-412),
    the routed part unchanged bit for bit, out = bf16(routed + ys) exactly, and ys close to the standalone launches'."""
    from dsv41_amd import moe, quant
    E, H, I, ws, ex = full_layer
    assert moe.fused_shared_ok(M, 8, I)
    g = torch.Generator(device=DEV).manual_seed(880 + M)
    Ws13 = (torch.randn(2 * I, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16)
    Ws2 = (torch.randn(H, I, generator=g, device=DEV) / I ** 0.5).to(torch.bfloat16)
    eid, wt = rand_routing(M, E, 8, 881 + M)
    xq = quant.fake_quant_fp8(rand_x(M, H, 882 + M).to(DEV))
    ed, wd = torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    y32 = torch.empty(M, H, device=DEV)
    ys = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    sh = moe.SharedExpert.prepare(Ws13, Ws2, tiled=tiled)
    moe.moe_experts(xq, ed, wd, ex, 10.0, out=out, y32=y32, shared=sh, ys_out=ys)
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    ys_ref = O.shared_expert(bf16_vals(xq), u16(Ws13), u16(Ws2), I, 10.0)
    close(bf16_vals(ys), ys_ref, f"fused shared expert M={M}")
    y_plain = moe.moe_experts(xq, ed, wd, ex, 10.0).clone()
    assert torch.equal(y32, y_plain), "the routed sum changed with the shared expert fused in"
    comp = O.f32_to_bf16_bits((y32.cpu().numpy() + bf16_vals(ys)).astype(np.float32))
    assert np.array_equal(u16(out), comp)
    ys_alone = moe.shared_expert(xq, sh.w13, sh.w2, 10.0, tiled=tiled).clone()
    close(bf16_vals(ys), bf16_vals(ys_alone), f"fused vs standalone shared expert M={M}")
    close(bf16_vals(ys_alone), ys_ref, f"standalone shared expert (tiled={tiled}) M={M}")
    W13, S13, W2, S2 = host_subset(ws, set(eid.reshape(-1).tolist()))
    ref = O.moe_layer_routed(bf16_vals(xq), eid, wt, W13, S13, W2, S2, I, 10.0)
    close(y32.cpu().numpy(), ref, f"routed part with the shared expert fused M={M}")


@pytest.mark.parametrize("M", [1, 2])
def test_decode_fused_fp8_shared_expert(full_layer, M):
    """The FP8 shared expert (w8.W8 weights, the checkpoint's format) in the two decode launches: its gate/up row blocks
    decode E4M3 tiles with their block scales into bf16 MFMA operands, its down projection likewise in every down
    workgroup. ys against the oracle's shared expert on the dequantised weights (the decode is exact, so only the fp32
    summation order differs), the routed part unchanged bit for bit, out = bf16(routed + ys) exactly, and ys close to
    the W8 linear_w path's (two FP8 GEMM launches + SwiGLU)."""
    from dsv41_amd import moe, quant, w8
    E, H, I, ws, ex = full_layer
    assert moe.fused_shared_ok(M, 8, I, fp8=True)
    g = torch.Generator().manual_seed(890 + M)

    def fp8_weight(n, k):
        c = torch.randint(0, 256, (n, k), generator=g, dtype=torch.uint8)
        c[(c & 0x7F) == 0x7F] = 0
        c[(c & 0x78) >= 0x60] &= 0xA7            # moderate magnitudes (exponent field < 12)
        return c, torch.randint(116, 122, ((n + 31) // 32, k // 32), generator=g, dtype=torch.uint8)
    c13, s13 = fp8_weight(2 * I, H)
    c2, s2 = fp8_weight(H, I)
    W13, W2 = w8.W8(c13.to(DEV), s13.to(DEV)), w8.W8(c2.to(DEV), s2.to(DEV))
    sh = moe.SharedExpert.of((W13, W2))
    assert sh.fp8
    eid, wt = rand_routing(M, E, 8, 891 + M)
    xq = quant.fake_quant_fp8(rand_x(M, H, 892 + M).to(DEV))
    ed, wd = torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    y32 = torch.empty(M, H, device=DEV)
    ys = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    moe.moe_experts(xq, ed, wd, ex, 10.0, out=out, y32=y32, shared=sh, ys_out=ys)
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    ys_ref = O.shared_expert(bf16_vals(xq), O.dequant_fp8_block(c13.numpy(), s13.numpy()), O.dequant_fp8_block(c2.numpy(), s2.numpy()),
                             I, 10.0)
    close(bf16_vals(ys), ys_ref, f"fused FP8 shared expert M={M}")
    y_plain = moe.moe_experts(xq, ed, wd, ex, 10.0).clone()
    assert torch.equal(y32, y_plain), "the routed sum changed with the FP8 shared expert fused in"
    comp = O.f32_to_bf16_bits((y32.cpu().numpy() + bf16_vals(ys)).astype(np.float32))
    assert np.array_equal(u16(out), comp)
    ys_w8 = moe.shared_expert_rows(xq, W13, W2, I, 10.0)
    close(bf16_vals(ys), bf16_vals(ys_w8), f"fused vs linear_w FP8 shared expert M={M}")


@pytest.mark.parametrize("T", [1, 3, 40])
def test_moe_layer_class(T):
    """model.MoE.__call__'s surface (moe.MoE): fp32 router weights, sigmoid gate with bias and route scale, FP8 x, routed
    experts, bf16 shared expert, bf16 output, for one token (shared expert fused into the decode launches), three tokens
    (decode, shared expert as its own launches) and 40 tokens (prefill path). Routing against the oracle gate on fp64
    logits; the output against the oracle layer on the same routing (bf16 output: the spec tolerance plus one bf16
    rounding step)."""
    from dsv41_amd import moe
    E, H, I, k = 32, 1024, 384, 4
    ws = make_experts(E, H, I, 1200 + T)
    ex = to_ex(*ws, True)
    g = torch.Generator(device=DEV).manual_seed(1300 + T)
    gate_w = torch.randn(E, H, generator=g, device=DEV) / H ** 0.5
    bias = torch.randn(E, generator=g, device=DEV) * 0.05
    Ws13 = (torch.randn(2 * I, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16)
    Ws2 = (torch.randn(H, I, generator=g, device=DEV) / I ** 0.5).to(torch.bfloat16)
    layer = moe.MoE(ex, gate_w, bias, topk=k, score_func="sigmoid", route_scale=2.5, swiglu_limit=10.0, sh_w13=Ws13, sh_w2=Ws2)
    x = (rand_x(T, H, 1400 + T) * 2).to(DEV)
    y = layer(x).clone()
    eid, wt = [t.cpu().numpy() for t in layer.last_routing]
    logits = (bf16_vals(x).astype(np.float64) @ gate_w.cpu().double().numpy().T).astype(np.float32)
    ref_i, ref_w = O.gate_topk(logits, bias.cpu().numpy(), 1.0, k, 2.5, "sigmoid", True)
    assert np.array_equal(eid, ref_i)
    assert np.allclose(wt, ref_w, rtol=1e-4, atol=1e-6)
    u16 = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    ids = set(eid.reshape(-1).tolist())
    W13, S13, W2, S2 = host_subset(ws, ids)
    ref = O.moe_layer(bf16_vals(x), eid, wt, W13, S13, W2, S2, u16(Ws13), u16(Ws2), I, 10.0)
    got = bf16_vals(y)
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    print(f"MoE T={T}: rel L2 {O.rel_l2(got, ref):.2e}")
    assert O.rel_l2(got, ref) <= RTOL_L2
    assert np.all(np.abs(got - ref) <= MAXABS_RMS * rms + np.abs(ref) * 2.0 ** -7)
    xs = O.fake_quant_fp8(bf16_vals(x))
    close(layer.shared_expert(x).cpu().numpy(), O.shared_expert(xs, u16(Ws13), u16(Ws2), I, 10.0), f"MoE.shared_expert T={T}")
    # the gate entry point on its own
    w2_, i2_ = layer.gate(x)
    assert np.array_equal(i2_.cpu().numpy(), ref_i)


@pytest.mark.parametrize("M,with_shared", [(1, True), (3, False)])
def test_decode_hc_post_fused(full_layer, M, with_shared):
    """The hyper-connection post mix in the down launch's epilogue equals the standalone hc_post2_ on the layer's bf16
    output, bit for bit (same x = bf16(y + ys), same multiply-add order), in place on the 4 residual streams."""
    from dsv41_amd import fused2, moe, quant
    E, H, I, ws, ex = full_layer
    rng = np.random.default_rng(990 + M)
    eid, wt = rand_routing(M, E, 8, 991 + M)
    xq = quant.fake_quant_fp8(rand_x(M, H, 992 + M).to(DEV))
    ed, wd = torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV)
    shared = None
    if with_shared:
        g = torch.Generator(device=DEV).manual_seed(993)
        shared = moe.SharedExpert.prepare((torch.randn(2 * I, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16),
                                          (torch.randn(H, I, generator=g, device=DEV) / I ** 0.5).to(torch.bfloat16))
    res0 = torch.from_numpy(O.f32_to_bf16_bits(rng.standard_normal((M, 1, 4, H)).astype(np.float32)).view(np.int16)).view(torch.bfloat16).to(DEV)
    post = torch.from_numpy(rng.standard_normal((M, 4)).astype(np.float32)).to(DEV)
    comb = torch.from_numpy(rng.standard_normal((M, 4, 4)).astype(np.float32)).to(DEV)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    moe.moe_experts(xq, ed, wd, ex, 10.0, out=out, shared=shared)
    res_ref = res0.clone()
    fused2.hc_post2_(out, res_ref, post, comb)
    res = res0.clone()
    moe.moe_experts(xq, ed, wd, ex, 10.0, shared=shared, hc=(res, post, comb))
    torch.cuda.synchronize()
    assert torch.equal(res, res_ref)


@pytest.mark.parametrize("M", [2, 3, 4])
def test_decode_pairs_duplicate_ids(M):
    """moe_experts at 2-4 tokens runs pair by pair, so a token may name one expert twice (each pair is its own group and
    h row): the layer equals the oracle's sum over the pairs, duplicates included."""
    from dsv41_amd import moe, quant
    E, H, I, k = 24, 512, 128, 6
    ws = make_experts(E, H, I, 700 + M)
    ex = to_ex(*ws, True)
    rng = np.random.default_rng(710 + M)
    eid = rng.integers(0, E, (M, k)).astype(np.int32)
    eid[:, 1] = eid[:, 0]                        # every token names its first expert twice
    wt = rng.random((M, k)).astype(np.float32)
    xq = quant.fake_quant_fp8(rand_x(M, H, 720 + M).to(DEV))
    y = moe.moe_experts(xq, torch.from_numpy(eid).to(DEV), torch.from_numpy(wt).to(DEV), ex, 10.0)
    ref = O.moe_layer_routed(bf16_vals(xq), eid, wt, *[w.cpu().numpy() for w in ws], I, 10.0)
    close(y.cpu().numpy(), ref, f"decode pairs M={M} with duplicate ids")


@pytest.mark.parametrize("M", [2, 4])   # M = 2: the shared expert in the two launches; M = 4 (M I > 4096): its own launches
def test_decode_pairs_shared_and_hc(full_layer, M):
    """moe_route_experts at 2-4 tokens routes pair by pair (dsv41_moe_decode_up_pairs) with the bf16 shared expert (in
    the two launches, or its own when it does not fit them) and the hyper-connection post mix in the down launch: the
    shared expert's output equals the
    bucketed launches' bit for bit, the routed sums match theirs (pick order instead of expert order), out is
    bf16(routed + ys) exactly, the post mix equals the standalone hc_post2_ on out, and token 0's routed sum matches
    the oracle."""
    from dsv41_amd import fused2, moe, quant
    E, H, I, ws, ex = full_layer
    assert 1 < M <= moe.PAIRS_MAX_M and moe.fused_shared_ok(M, 8, I) == (M == 2)
    rng = np.random.default_rng(1200 + M)
    lg = torch.from_numpy(rng.standard_normal((M, E)).astype(np.float32)).to(DEV)
    xq = quant.fake_quant_fp8(rand_x(M, H, 1201 + M).to(DEV))
    g = torch.Generator(device=DEV).manual_seed(1202 + M)
    shared = moe.SharedExpert.prepare((torch.randn(2 * I, H, generator=g, device=DEV) / H ** 0.5).to(torch.bfloat16),
                                      (torch.randn(H, I, generator=g, device=DEV) / I ** 0.5).to(torch.bfloat16))
    eo, wo = torch.empty(M, 8, dtype=torch.int32, device=DEV), torch.empty(M, 8, device=DEV)
    out, ys = torch.empty(M, H, dtype=torch.bfloat16, device=DEV), torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    y32 = torch.empty(M, H, device=DEV)
    route = (xq, lg, None, 1.0, 8, 1.0, "softmax", True, ex, 10.0)
    moe.moe_route_experts(*route, out=out, y32=y32, eid_out=eo, wt_out=wo, shared=shared, ys_out=ys)
    out_b, ys_b, y32_b = torch.empty_like(out), torch.empty_like(ys), torch.empty_like(y32)
    moe.moe_experts(xq, eo, wo, ex, 10.0, out=out_b, y32=y32_b, shared=shared, ys_out=ys_b)
    torch.cuda.synchronize()
    assert torch.equal(ys, ys_b)
    assert O.rel_l2(y32.cpu().numpy(), y32_b.cpu().numpy()) < 1e-5   # the routed sums, in pick order vs expert order
    # out = bf16(routed + ys) exactly (model.py:590-591)
    ref_out = O.bf16_round(y32.cpu().numpy() + ys.float().cpu().numpy())
    assert np.array_equal(out.float().cpu().numpy(), ref_out)
    res0 = torch.from_numpy(O.f32_to_bf16_bits(rng.standard_normal((M, 1, 4, H)).astype(np.float32)).view(np.int16)).view(torch.bfloat16).to(DEV)
    post = torch.from_numpy(rng.standard_normal((M, 4)).astype(np.float32)).to(DEV)
    comb = torch.from_numpy(rng.standard_normal((M, 4, 4)).astype(np.float32)).to(DEV)
    res, res_ref = res0.clone(), res0.clone()
    moe.moe_route_experts(*route, shared=shared, hc=(res, post, comb))
    fused2.hc_post2_(out, res_ref, post, comb)
    torch.cuda.synchronize()
    assert torch.equal(res, res_ref)
    eid, wt = eo.cpu().numpy(), wo.cpu().numpy()
    W13, S13, W2, S2 = host_subset(ws, set(eid[0].tolist()))
    y0 = O.moe_layer_routed(bf16_vals(xq[0:1]), eid[0:1], wt[0:1], W13, S13, W2, S2, I, 10.0)
    close(y32[0:1].cpu().numpy(), y0, f"pairs M={M} token 0 routed layer")
