"""The FP8 dense-weight family (w8.W8 / linear_w / oproj_a, hipkern.fp8_gemm_tc / fp8_gemv, quant.dequant_fp8_block)
against the oracle: dequantisation bit-exact over every E4M3 code and scale byte; the GEMM's in-register decode
bit-exact through one-hot activations; the reference test's shapes (test_fp8_tc.py:19, test_fp8_tcw.py:38) within
the floating-point tolerance (the kernel and the oracle differ only in fp32 summation order)."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def rand_fp8(N, K, seed, lo=110, hi=130):
    """E4M3 bytes without NaN codes and E8M0 scales in [lo, hi) (test_fp8_tc.py:12-16)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(0, 256, (N, K), generator=g, dtype=torch.uint8)
    w[(w & 0x7F) == 0x7F] = 0
    s = torch.randint(lo, hi, ((N + 31) // 32, K // 32), generator=g, dtype=torch.uint8)
    return w, s


def check_close(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref ** 2)) + 1e-30
    rel = np.linalg.norm(got - ref) / (np.linalg.norm(ref) + 1e-30)
    mx = np.abs(got - ref).max()
    # fp32 accumulation in another order: rel L2 <= 2e-3 and max-abs <= 1e-2 RMS (far looser than what is seen)
    assert rel <= 2e-3 and mx <= 1e-2 * rms, f"{what}: rel L2 {rel:.3e}, max-abs {mx:.3e} (rms {rms:.3e})"


def check_bf16(got, ref32, what):
    """bf16 outputs against the oracle's fp32 result rounded to bf16 (as the reference rounds its fp32 accumulator):
    at most one bf16 ulp apart (summation order can move a value across a rounding boundary) plus 1e-4 RMS (fp32
    summation-order error on results that cancel to near zero), >= 99% bit-equal, and rel L2 <= 2e-3 against the
    unrounded fp32 result."""
    got = np.asarray(got, np.float32)
    ref32 = np.asarray(ref32, np.float32)
    refb = O.bf16_round(ref32)
    rms = float(np.sqrt(np.mean(ref32.astype(np.float64) ** 2)))
    tol = np.maximum(np.abs(got), np.abs(refb)) * 2.0 ** -7 + 1e-4 * rms
    bad = np.abs(got - refb) > tol
    assert not bad.any(), f"{what}: {bad.sum()} outputs more than one bf16 ulp off, e.g. {got[bad][:4]} vs {ref32[bad][:4]}"
    assert (got == refb).mean() >= 0.99, f"{what}: only {(got == refb).mean():.3f} bit-equal"
    assert O.rel_l2(got, ref32) <= 2e-3, f"{what}: rel L2 {O.rel_l2(got, ref32):.3e}"


@pytest.mark.parametrize("tiled", [False, True])
def test_dequant_fp8_every_code_and_scale(tiled):
    from dsv41_amd import quant, w8
    codes = torch.arange(256, dtype=torch.uint8)
    w = codes.repeat(32, 1)                                   # [32, 256]: every row holds all codes
    for b0 in range(0, 256, 8):
        s = torch.arange(b0, b0 + 8, dtype=torch.int32).clamp(0, 255).to(torch.uint8).view(1, 8)
        wd = (w8.tile(w) if tiled else w).to(DEV)
        got = u16(quant.dequant_fp8_block(wd, s.to(DEV), tiled=tiled))
        ref = O.dequant_fp8_block(w.numpy(), s.numpy())
        nan = np.isnan(O.bf16_bits_to_f32(ref))
        assert np.array_equal(np.isnan(O.bf16_bits_to_f32(got)), nan)
        assert np.array_equal(got[~nan], ref[~nan]), f"scale bytes {b0}..{b0 + 7}"


@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("rows,N", [(4, 256), (16, 256), (64, 256), (16, 4112)])
def test_fp8_gemm_decode_one_hot_exact(tiled, rows, N):
    """One-hot activation rows make each output one product: out[t, n] = x[t, k_t] * deq[n, k_t] exactly. Launches of
    `rows` tokens (4: the LDS-staged kernel; 16 and 64: one and four token tiles; 16 over 257 row blocks: two row
    blocks per workgroup, the last one alone) cover every k position of the first 256 (every lane group and both MFMA
    halves) and a spread beyond, over rows holding every E4M3 code, with scale bytes 90..160 (products normal in bf16)."""
    from dsv41_amd import hipkern, w8
    K = 1024
    g = torch.Generator().manual_seed(11)
    w = torch.stack([torch.cat([torch.randperm(256, generator=g) for _ in range(K // 256)]) for _ in range(N)]).to(torch.uint8)
    w[(w & 0x7F) == 0x7F] = 0
    s = torch.randint(90, 161, ((N + 31) // 32, K // 32), generator=g, dtype=torch.uint8)
    deq = O.bf16_bits_to_f32(O.dequant_fp8_block(w.numpy(), s.numpy()))
    wd = (w8.tile(w) if tiled else w).to(DEV)
    sd = s.to(DEV)
    ks = list(range(256)) + list(range(256, K, 7))
    for b in range(0, len(ks), rows):
        kk = ks[b:b + rows]
        x = torch.zeros(len(kk), K, dtype=torch.bfloat16)
        for t, k in enumerate(kk):
            x[t, k] = 1.0 if t % 3 else -0.5
        y = hipkern.fp8_gemm_tc(x.to(DEV), wd, sd, out_dtype=torch.float32, tiled=tiled).cpu().numpy()
        ref = np.stack([deq[:, k] * (1.0 if t % 3 else -0.5) for t, k in enumerate(kk)])
        assert np.array_equal(y, ref.astype(np.float32)), f"k {kk[0]}.."   # values (a zero product may carry either sign)


# the reference's test shapes (M, N, K, group_cols): test_fp8_tc.py:19 and the 17-64-row kernel's test_fp8_tcw.py:38
SHAPES = [(1, 512, 5120, 0), (1, 1280, 5120, 0), (1, 32768, 1280, 0), (6, 5120, 8192, 0), (16, 4608, 5120, 0),
          (8, 8192, 4096, 1024), (1, 5120, 2304, 0), (32, 5120, 8192, 0), (48, 1280, 5120, 0), (64, 5120, 8192, 0)]

# every launch shape of the <= 4-token LDS kernel: 2 waves (>= 256 row blocks, K <= 1536), 4 waves with 4 tiles in
# flight (>= 256 row blocks), 4 waves with 10 (fewer), and the 8- and 16-wave fallbacks for 4 tokens at K = 8192
SHAPES += [(2, 32768, 1280, 0), (1, 4608, 5120, 0), (3, 512, 5120, 0), (4, 5120, 8192, 0), (4, 1280, 8192, 0)]
# and of the 5-16-row kernel with 3 tiles in flight (fewer than 6 chunks per wave): 8 and 16 waves per workgroup
SHAPES += [(12, 32768, 1280, 0), (16, 5120, 2304, 0), (16, 1280, 5120, 0)]
# the 5-16-row kernel's two-row-block workgroups: an odd row-block count (the last workgroup's second block past the
# end), 8-wave workgroups (K < 4096), column groups of 32 rows (both blocks share one x offset) and of 16 (one block
# per workgroup)
SHAPES += [(16, 4112, 4096, 0), (5, 4112, 1280, 0), (9, 4096, 1024, 32), (7, 4096, 1024, 16)]


@pytest.mark.parametrize("M,N,K,gc", SHAPES)
def test_fp8_gemm_reference_shapes(M, N, K, gc):
    from dsv41_amd import fused, hipkern, w8
    print(f"fp8_gemm M={M} N={N} K={K} gc={gc}", flush=True)
    w, s = rand_fp8(N, K, seed=N + K + M)
    Mx = M * (N // gc) if gc else M
    g = torch.Generator().manual_seed(M)
    x = fused.fake_quant_fp8((torch.randn(Mx, K, generator=g) * 2).to(torch.bfloat16).to(DEV))
    ref = O.linear_fp8w(O.bf16_bits_to_f32(u16(x)), w.numpy(), s.numpy(), group_cols=gc)
    wd = w8.tile(w).to(DEV)
    sd = s.to(DEV)
    y32 = hipkern.fp8_gemm_tc(x, wd, sd, group_cols=gc, out_dtype=torch.float32, tiled=True)
    yb = hipkern.fp8_gemm_tc(x, wd, sd, group_cols=gc, tiled=True)
    check_close(y32.cpu().numpy(), ref, "tiled")
    assert np.array_equal(u16(yb), O.f32_to_bf16_bits(y32.cpu().numpy())), "bf16 output is not bf16(fp32 output)"
    # natural row-major layout: the same sums in the same order
    yn = hipkern.fp8_gemm_tc(x, w.to(DEV), sd, group_cols=gc, out_dtype=torch.float32, tiled=False)
    assert torch.equal(yn, y32)


@pytest.mark.parametrize("M,N,K", [(16, 4104, 2048), (6, 4136, 4096), (16, 1000, 2048)])
def test_fp8_gemm_natural_rows_not_a_multiple_of_16(M, N, K):
    """Natural layout with N % 16 != 0 on the 5-16-row kernel: the last row block's rows past N are read clamped and
    never stored, and a two-block workgroup's second block past the last one stores nothing."""
    from dsv41_amd import hipkern
    w, s = rand_fp8(N, K, seed=N + K)
    x = (torch.randn(M, K, generator=torch.Generator().manual_seed(3)) * 2).to(torch.bfloat16).to(DEV)
    ref = O.linear_fp8w(O.bf16_bits_to_f32(u16(x)), w.numpy(), s.numpy())
    y = hipkern.fp8_gemm_tc(x, w.to(DEV), s.to(DEV), out_dtype=torch.float32, tiled=False)
    check_close(y.cpu().numpy(), ref, f"M={M} N={N} K={K}")
    assert y.shape == (M, N)


def test_fp8_gemm_rejects_short_scales():
    """A scale tensor with fewer than ceil(N / 32) rows or K / 32 columns is refused on the host, before any launch
    (the kernels read scale row n // 32 of every weight row)."""
    from dsv41_amd import hipkern
    N, K = 4112, 1024
    w, s = rand_fp8(N, K, seed=5)
    x = torch.randn(16, K).to(torch.bfloat16).to(DEV)
    with pytest.raises(ValueError):
        hipkern.fp8_gemm_tc(x, w.to(DEV), s[: N // 32].contiguous().to(DEV), out_dtype=torch.float32)
    with pytest.raises(ValueError):
        hipkern.fp8_gemm_tc(x, w.to(DEV), s[:, :-1].contiguous().to(DEV), out_dtype=torch.float32)


def test_fp8_gemm_deterministic_wide_and_narrow():
    """Repeated calls give bit-identical results, for a grid of few row blocks (16-wave workgroups) and of many."""
    from dsv41_amd import hipkern, w8
    for (M, N, K) in [(4, 1280, 5120), (3, 5120, 2304)]:
        w, s = rand_fp8(N, K, seed=7)
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(DEV)
        wd, sd = w8.tile(w).to(DEV), s.to(DEV)
        a = hipkern.fp8_gemm_tc(x, wd, sd, out_dtype=torch.float32, tiled=True)
        b = hipkern.fp8_gemm_tc(x, wd, sd, out_dtype=torch.float32, tiled=True)
        assert torch.equal(a, b)
        ref = O.linear_fp8w(O.bf16_bits_to_f32(u16(x)), w.numpy(), s.numpy())
        check_close(a.cpu().numpy(), ref, f"M={M} N={N} K={K}")


def test_w8_surface():
    """W8 / linear_w / linear_fp8 / oproj_a / fp8_gemv with the reference's call shapes."""
    from dsv41_amd import fused, hipkern, quant, w8
    N, K = 1024, 2048
    w, s = rand_fp8(N, K, seed=21)
    W = w8.W8(w.to(DEV), s.to(DEV))
    assert W.tiled and W.shape == (N, K) and W.dtype == torch.bfloat16
    assert torch.equal(W.natural().cpu(), w)
    assert np.array_equal(u16(W.bf16()), O.dequant_fp8_block(w.numpy(), s.numpy()))
    g = torch.Generator().manual_seed(22)
    for rows in (1, 3, 16, 40, 64, 100):
        x = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(DEV)
        y = w8.linear_w(x.view(1, rows, K), W)
        assert y.shape == (1, rows, N) and y.dtype == torch.bfloat16
        ref = O.linear_fp8w(O.bf16_bits_to_f32(u16(x)), w.numpy(), s.numpy())
        check_bf16(y.float().view(rows, N).cpu().numpy(), ref, f"linear_w rows={rows}")
    # linear_fp8 rounds the activations to FP8 first (model.py:55-58)
    x = torch.randn(2, K, generator=g).to(torch.bfloat16).to(DEV)
    assert torch.equal(w8.linear_fp8(x, W), w8.linear_w(fused.fake_quant_fp8(x), W))
    # the kept bf16 copy serves large row counts
    W.keep_bf16()
    assert W.bf16w is not None and np.array_equal(u16(W.bf16w), O.dequant_fp8_block(w.numpy(), s.numpy()))
    # concatenation along N keeps tiles and scale blocks whole
    w2, s2 = rand_fp8(512, K, seed=23)
    C = w8.W8.cat([w8.W8(w.to(DEV), s.to(DEV)), w8.W8(w2.to(DEV), s2.to(DEV))])
    assert torch.equal(C.natural().cpu(), torch.cat([w, w2]))
    # block-diagonal o-projection: o [b, s, g, d], rank columns per group
    gN, rank, d = 8, 128, 512
    wo, so = rand_fp8(gN * rank, d, seed=24)
    Wo = w8.W8(wo.to(DEV), so.to(DEV))
    o = torch.randn(2, 3, gN, d, generator=g).to(torch.bfloat16).to(DEV)
    y = w8.oproj_a(o, Wo, gN, rank)
    assert y.shape == (2, 3, gN * rank)
    ref = O.linear_fp8w(O.bf16_bits_to_f32(u16(o.reshape(-1, d))), wo.numpy(), so.numpy(), group_cols=rank)
    check_bf16(y.float().reshape(6, -1).cpu().numpy(), ref, "oproj_a")
    # fp8_gemv: natural layout, any N, K % 32 == 0 (K % 64 == 32 padded)
    for (Nn, Kk) in [(1000, 1280), (96, 1312)]:
        wv, sv = rand_fp8(Nn, Kk, seed=Nn)
        xv = torch.randn(1, Kk, generator=g).to(torch.bfloat16).to(DEV)
        out = hipkern.fp8_gemv(xv, wv.view(torch.float8_e4m3fn).to(DEV), sv.to(DEV))
        ref = O.linear_fp8w(O.bf16_bits_to_f32(u16(xv)), wv.numpy(), sv.numpy())
        check_close(out.cpu().numpy(), ref, f"fp8_gemv N={Nn} K={Kk}")
    _ = quant


def test_fp8_gemm_graph_replay():
    """Captured in a graph and replayed: every replay equals the eager result."""
    from dsv41_amd import hipkern, w8
    M, N, K = 2, 1280, 5120
    w, s = rand_fp8(N, K, seed=31)
    wd, sd = w8.tile(w).to(DEV), s.to(DEV)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(32)).to(torch.bfloat16).to(DEV)
    eager = hipkern.fp8_gemm_tc(x, wd, sd, tiled=True)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        hipkern.fp8_gemm_tc(x, wd, sd, tiled=True)
    torch.cuda.current_stream().wait_stream(st)
    gph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gph):
        y = hipkern.fp8_gemm_tc(x, wd, sd, tiled=True)
    for _ in range(3):
        gph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        _ = hipkern.fp8_gemm_tc(x, wd, sd, tiled=True)   # eager work between replays
        torch.cuda.synchronize()
