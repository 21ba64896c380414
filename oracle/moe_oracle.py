"""CPU oracle for the FP4 MoE expert path: a numpy restatement of the reference's algorithm.

THIS IS TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import it, and only as the checker. The product path (the HIP library) never calls it.

Each function cites the reference file:line it restates (paths relative to the reference repo).
How each one is pinned (golden vectors written by the reference's own quant.py, the compiled
reference CPU library in oracle/_ref, closed forms, brute force) is listed in PINS below and
checked by tests/test_oracle.py. A function marked "parity unpinned" there has no such check.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32

# quant.py:22-24
FP8_MAX = 448.0
FP4_MAX = 6.0
FP4_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=F32)

PINS = {
    "e8m0_to_f32": "golden deq_all (every scale byte) + exp2 identity",
    "dequant_fp4": "golden deq_all (16 codes x 256 scale bytes) + golden rand_deq",
    "tile_fp4": "golden rand_w_tiled + round trip",
    "tile_fp4_scales": "golden rand_s_tiled + round trip",
    "ceil_log2": "golden cl2 + brute force against log2 on powers of two",
    "round_e4m3": "torch float8_e4m3fn cast on 2^20 samples (test_fused.py:17 twin) + exhaustive code grid",
    "fake_quant_fp8": "golden fq8 (bf16 and fp32 inputs, edge groups)",
    "quant_fp8": "golden qfp8 codes and scales",
    "lo_exponent": "brute force: the smallest e >= -126 with a <= 448 2^e by scanning e, on random, power-of-two and "
                   "448 2^k boundary amax values",
    "fp8_split": "hi = the golden-pinned quant_fp8 codes/scales; hi + lo reconstructs bf16 x exactly wherever the residual "
                 "is in lo's normal range and within 2^-21 of the block amax elsewhere (closed form); lo codes = torch "
                 "float8_e4m3fn cast of residual / 2^e2; FP8-grid x gives lo = 0",
    "permute_x": "closed form: inverse permutation round trip",
    "swiglu_quant": "compiled reference CPU library (oracle/_ref) layer output + closed form",
    "gate_topk": "brute force (sort) on random and tied inputs",
    "moe_dispatch": "invariants + brute force on tiny inputs",
    "grouped_gemm": "textbook matmul against dense fp64 on tiny inputs",
    "moe_layer_routed": "compiled reference CPU library (oracle/_ref, bf16 mode) on I = 256",
    "moe_layer": "composition check: with the shared expert equal to a routed expert (one-hot off-grid x), "
                 "bf16(moe_layer_routed(fq8 x) + bf16(the expert's moe_layer_routed row)), the reference's order "
                 "(model.py:565-591)",
    "linear_bf16": "torch F.linear on bf16 CPU tensors (the op linear_w runs for bf16 weights, w8.py:102-103)",
    "shared_expert": "torch F.linear (bf16) for both GEMVs + golden/library-pinned swiglu_quant; structure (w1/w3 "
                     "halves, no routing weight, limit) against moe_layer_routed with the expert's dequantised weights "
                     "and a one-hot x (gu exact in bf16)",
    "gemv_pairs": "wt x grouped_gemm on singleton groups + scalar brute force on a tiny case",
    "hc_pre_norm_quant": "one-hot pre weights reduce it to rmsnorm: torch.nn.functional.rms_norm (fp32, CPU) + golden-pinned "
                         "fake_quant_fp8; an equal split of one stream over two weights gives the same",
    "hc_post": "special cases (post 0, comb identity: unchanged; comb 0, post one-hot: the stream takes x) + torch.einsum "
               "of the 4 x 4 mix in float64",
    "hc_post_input": "closed form on exactly representable sums (small integers times powers of two)",
    "residual_rmsnorm_quant": "torch.nn.functional.rms_norm (fp32, CPU) + golden-pinned fake_quant_fp8",
    "int8_quant_blocks": "closed form (|v - q s| <= s / 2, q range, zero block) + compiled reference CPU library (int8 mode) layer output",
    "w4a8_gemv": "brute force on tiny inputs (integer dot by hand) + compiled reference CPU library (int8 mode) layer output",
    "swiglu_quant_host": "compiled reference CPU library stage-2 output h (inter a multiple of 256) + golden-pinned fake_quant_fp8",
    "host_layer": "compiled reference CPU library (oracle/_ref) gu, h and out, int8 and bf16 modes, inter a multiple of 256",
    "dequant_fp8_block_f32": "torch float8_e4m3fn -> float32 cast of all 256 codes (the reference's w.float()) times torch.ldexp "
                             "over 256 scale bytes; one scale byte changed moves exactly its 32 x 32 block",
    "dequant_fp8_block": "bf16 of dequant_fp8_block_f32 = torch .to(torch.bfloat16) of the torch-built product",
    "linear_fp8w": "one-hot x rows give dequantised weight columns exactly; torch F.linear in float64 on the torch-built "
                   "dequant; block-diagonal form against a scalar loop over (b, n) on a tiny case",
}


# --------------------------------------------------------------------------- scalar formats
def f32_bits(a) -> np.ndarray:
    return np.asarray(a, dtype=F32).view(np.uint32)


def bits_f32(u) -> np.ndarray:
    return np.asarray(u, dtype=np.uint32).view(F32)


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit pattern (torch's `.to(torch.bfloat16)`).
    Every NaN becomes 0xFFFF, as torch's vectorised CPU conversion writes it."""
    u = f32_bits(a).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(np.asarray(a, dtype=F32))
    r = np.where(nan, np.uint32(0xFFFF), r)
    return (r & 0xFFFF).astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return bits_f32(np.asarray(b, dtype=np.uint32) << 16)


def bf16_round(a) -> np.ndarray:
    """fp32 -> bf16 -> fp32 (the `.to(torch.bfloat16)` rounding point)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def e8m0_to_f32(b) -> np.ndarray:
    """E8M0 byte -> fp32 2^(b-127); byte 0 is the subnormal 2^-127 and 255 is +inf (quant.py:27-31)."""
    b = np.asarray(b, dtype=np.uint32)
    return np.where(b == 0, bits_f32(np.uint32(0x00400000)), bits_f32(b << 23)).astype(F32)


def ceil_log2(a) -> np.ndarray:
    """ceil(log2(a)) for a > 0 exactly, via frexp (quant.py:34-37)."""
    m, e = np.frexp(np.asarray(a, dtype=F32))
    return (e - (m == 0.5)).astype(np.int32)


def pow2_scale(amax, qmax: float) -> np.ndarray:
    """2^ceil(log2(amax / qmax)) (quant.py:40-42); the division is an fp32 RNE division."""
    return np.ldexp(F32(1.0), ceil_log2(np.asarray(amax, dtype=F32) / F32(qmax))).astype(F32)


def round_e4m3(v) -> np.ndarray:
    """Round fp32 |v| <= 448 to the nearest float8_e4m3fn value, ties to even (fused.py:24-34, the formula
    test_fused.py:17 checks against torch's float8_e4m3fn cast)."""
    v = np.asarray(v, dtype=F32)
    a = np.abs(v)
    e = ((f32_bits(a) >> 23) & 0xFF).astype(np.int32) - 127
    e = np.maximum(e, -6)
    ulp = np.ldexp(F32(1.0), e - 3).astype(F32)
    r = (np.rint(a / ulp) * ulp).astype(F32)
    r = np.minimum(r, F32(448.0))
    # sign from the sign bit: -0.0 stays -0.0 as in torch's cast (quant.py:53); fused.py:34's
    # `where(v < 0, -r, r)` would give +0.0 there, which quant.py (the spec) does not
    return np.copysign(r, v).astype(F32)


def e4m3_encode(q) -> np.ndarray:
    """float8_e4m3fn bit pattern of values already on the E4M3 grid (|q| <= 448)."""
    q = np.asarray(q, dtype=F32)
    a = np.abs(q)
    sign = (f32_bits(q) >> 31).astype(np.uint32)
    ex = ((f32_bits(a) >> 23) & 0xFF).astype(np.int32) - 127
    normal = a >= F32(2.0 ** -6)
    man_n = ((f32_bits(a) >> 20) & 7).astype(np.uint32)
    code_n = (((ex + 7).clip(0, 15).astype(np.uint32)) << 3) | man_n
    code_s = np.rint(a * F32(512.0)).astype(np.uint32)  # subnormal: multiples of 2^-9
    code = np.where(normal, code_n, code_s)
    return ((sign << 7) | code).astype(np.uint8)


def e4m3_decode(c) -> np.ndarray:
    c = np.asarray(c, dtype=np.uint32)
    s = np.where((c >> 7) & 1, F32(-1.0), F32(1.0))
    e = ((c >> 3) & 15).astype(np.int32)
    m = (c & 7).astype(F32)
    val = np.where(e == 0, m * F32(2.0 ** -9), np.ldexp(F32(1.0) + m / F32(8.0), e - 7)).astype(F32)
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(F32)


# --------------------------------------------------------------------------- FP4 weights
def unpack_fp4(packed) -> np.ndarray:
    """uint8 [..., K/2] -> fp32 [..., K] E2M1 values, low nibble = even k (quant.py:98-103)."""
    p = np.asarray(packed, dtype=np.uint8)
    lo, hi = p & 0x0F, p >> 4
    return np.stack([FP4_TABLE[lo], FP4_TABLE[hi]], axis=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)


def dequant_fp4_f32(packed, scale, block: int = 32) -> np.ndarray:
    """fp32 product E2M1 x 2^(S-127) before the bf16 cast (quant.py:106-110)."""
    v = unpack_fp4(packed)
    s = np.repeat(e8m0_to_f32(scale), block, axis=-1)
    with np.errstate(invalid="ignore", over="ignore"):
        return (v * s).astype(F32)


def dequant_fp4(packed, scale, block: int = 32) -> np.ndarray:
    """-> bf16 bit patterns [..., K] (quant.py:106-110)."""
    return f32_to_bf16_bits(dequant_fp4_f32(packed, scale, block))


def dequant_fp4_values(packed, scale) -> np.ndarray:
    """fp32 values of the bf16 dequant (what the reference's torch oracles multiply with). When every scale
    byte is in [2, 250] the fp32 product already has <= 2 significant bits inside bf16's exponent range, so the
    bf16 rounding is the identity and is skipped (test_oracle checks this shortcut against the full path)."""
    sc = np.asarray(scale)
    if sc.size and sc.min() >= 2 and sc.max() <= 250:
        return dequant_fp4_f32(packed, scale)
    return bf16_bits_to_f32(dequant_fp4(packed, scale))


def tile_fp4(w) -> np.ndarray:
    """[E, N, K/2] row-major -> [E][N/16][K/128][16 rows][64 B] (quant.py:118-122)."""
    E, N, Kh = w.shape
    assert N % 16 == 0 and Kh % 64 == 0
    return np.ascontiguousarray(w.reshape(E, N // 16, 16, Kh // 64, 64).transpose(0, 1, 3, 2, 4).reshape(E, N, Kh))


def untile_fp4(w) -> np.ndarray:
    """inverse of tile_fp4 (quant.py:125-127)."""
    E, N, Kh = w.shape
    return np.ascontiguousarray(w.reshape(E, N // 16, Kh // 64, 16, 64).transpose(0, 1, 3, 2, 4).reshape(E, N, Kh))


def tile_fp4_scales(s) -> np.ndarray:
    """[E, N, K/32] -> [E][N/16][K/128][16][4] (quant.py:130-134)."""
    E, N, Ks = s.shape
    assert N % 16 == 0 and Ks % 4 == 0
    return np.ascontiguousarray(s.reshape(E, N // 16, 16, Ks // 4, 4).transpose(0, 1, 3, 2, 4).reshape(E, N, Ks))


def untile_fp4_scales(s) -> np.ndarray:
    """inverse of tile_fp4_scales (quant.py:137-139)."""
    E, N, Ks = s.shape
    return np.ascontiguousarray(s.reshape(E, N // 16, Ks // 4, 16, 4).transpose(0, 1, 3, 2, 4).reshape(E, N, Ks))


# --------------------------------------------------------------------------- FP8 activations
def _groups(x, block):
    x = np.asarray(x, dtype=F32)
    return x.reshape(-1, block)


def quant_fp8_e8m0(x, block: int = 32):
    """Per-`block` FP8 quantisation (quant.py:57-64) returned as (E4M3 codes uint8 [..., K],
    E8M0 bytes uint8 [..., K/block]) -- the operand format of the scaled MFMA."""
    shape = np.shape(x)
    xg = _groups(x, block)
    amax = np.maximum(np.abs(xg).max(axis=-1, keepdims=True), F32(1e-4))
    e = ceil_log2(amax / F32(FP8_MAX))
    s = np.ldexp(F32(1.0), e).astype(F32)
    q = round_e4m3(np.clip(xg / s, -FP8_MAX, FP8_MAX))
    codes = e4m3_encode(q).reshape(shape)
    scales = (e + 127).astype(np.uint8).reshape(*shape[:-1], shape[-1] // block)
    return codes, scales


def lo_exponent(amax) -> np.ndarray:
    """Smallest integer e >= -126 with amax / 2^e <= 448 (no 1e-4 floor): the scale exponent of the split's second
    term. This build's own rule (the reference has no FP8 activation operand); brute-force pinned."""
    a = np.asarray(amax, dtype=np.float64)
    e = np.full(a.shape, -126, dtype=np.int32)
    pos = a > 0
    m, ex = np.frexp(a[pos])                      # a = m 2^ex, m in [0.5, 1)
    need = np.ceil(np.log2(a[pos] / 448.0)).astype(np.int32)
    # log2 can be off by an ulp at exact powers of two: settle the integer with the exact comparison a <= 448 2^e
    need = np.where(np.ldexp(448.0, need - 1) >= a[pos], need - 1, need)
    need = np.where(np.ldexp(448.0, need) < a[pos], need + 1, need)
    e[pos] = np.maximum(need, -126)
    return e


def fp8_split(x, block: int = 32):
    """bf16-valued x [..., K] as two FP8 operand terms (dsv41_quant_fp8_split): (hi codes, hi scales, lo codes, lo
    scales). hi = quant_fp8_e8m0(x) (quant.py:57-64); lo = the residual x - hi (exact in fp32), quantised per block
    with 2^lo_exponent(amax of the residual) and E4M3 round-to-nearest-even. The reference multiplies bf16 x directly
    (fp4_gemv.cu:15-66, moe_kernels.py:154-200); hi + lo is that x to within 2^-21 of the block's amax."""
    shape = np.shape(x)
    xg = _groups(x, block)
    hc, hs = quant_fp8_e8m0(xg, block)
    hv = e4m3_decode(hc).astype(np.float64) * np.ldexp(1.0, hs.astype(np.int32) - 127)
    r = (xg.astype(np.float64) - hv).astype(F32)            # exact: both are short fp32 values within 24 bits
    e2 = lo_exponent(np.abs(r).max(axis=-1, keepdims=True))
    q2 = round_e4m3(np.clip(r / np.ldexp(F32(1.0), e2).astype(F32), -FP8_MAX, FP8_MAX))
    lc = e4m3_encode(q2)
    ls = (e2 + 127).astype(np.uint8)
    return hc.reshape(shape), hs.reshape(*shape[:-1], shape[-1] // block), lc.reshape(shape), ls.reshape(*shape[:-1], shape[-1] // block)


def fp8_split_values(hc, hs, lc, ls, block: int = 32) -> np.ndarray:
    """float64 value of hi + lo, per element."""
    shape = np.shape(hc)
    v = lambda c, s: e4m3_decode(np.asarray(c).reshape(-1, block)).astype(np.float64) * \
        np.ldexp(1.0, np.asarray(s).reshape(-1, 1).astype(np.int32) - 127)
    return (v(hc, hs) + v(lc, ls)).reshape(shape)


def quant_fp8(x, block: int = 32):
    """(E4M3 values as fp32, fp32 scales [..., K/block]) exactly as quant.quant_fp8 (quant.py:57-64)."""
    shape = np.shape(x)
    xg = _groups(x, block)
    amax = np.maximum(np.abs(xg).max(axis=-1, keepdims=True), F32(1e-4))
    s = pow2_scale(amax, FP8_MAX)
    q = round_e4m3(np.clip(xg / s, -FP8_MAX, FP8_MAX))
    return q.reshape(shape), s.reshape(*shape[:-1], shape[-1] // block)


def fake_quant_fp8(x, block: int = 32) -> np.ndarray:
    """Quantise-dequantise per `block` along the last dim, fp32 result (quant.py:45-54). A bf16 caller
    casts the result back to bf16, which is exact (4 significant bits times a power of two)."""
    shape = np.shape(x)
    q, s = quant_fp8(x, block)
    return (q.reshape(-1, block) * s.reshape(-1, 1)).astype(F32).reshape(shape)


def residual_rmsnorm_quant(x, y, w, eps: float):
    """The stack's layer-to-layer step: r = bf16(x + y); xn = bf16(r * (1 / sqrt(mean(r^2) + eps)) * w)
    (fused.py:92-110: fp32 statistics, one rounding); xq = fake_quant_fp8(xn) (quant.py:45-54).
    Inputs are bf16 values held in fp32; returns (xn, xq) as fp32 arrays of bf16 values."""
    r = bf16_round(np.asarray(x, F32) + np.asarray(y, F32))
    var = (r.astype(np.float64) ** 2).sum(axis=-1, keepdims=True) / r.shape[-1]
    inv = (1.0 / np.sqrt(var.astype(F32) + F32(eps))).astype(F32)
    wv = np.ones(r.shape[-1], F32) if w is None else np.asarray(w, F32)
    xn = bf16_round((r * inv * wv).astype(F32))
    return xn, fake_quant_fp8(xn).astype(F32)


_PERM8 = np.array([0, 4, 2, 6, 1, 5, 3, 7])


def permute_x(x) -> np.ndarray:
    """Within every 8 k: order 0,4,2,6,1,5,3,7 (cukern.py:221-227)."""
    M, K = x.shape
    return np.ascontiguousarray(x.reshape(M, K // 8, 8)[:, :, _PERM8].reshape(M, K))


def unpermute_x(xp) -> np.ndarray:
    M, K = xp.shape
    inv = np.argsort(_PERM8)
    return np.ascontiguousarray(xp.reshape(M, K // 8, 8)[:, :, inv].reshape(M, K))


# --------------------------------------------------------------------------- SwiGLU + quant
def sigmoid_f32(g) -> np.ndarray:
    g = np.asarray(g, dtype=F32)
    with np.errstate(over="ignore"):
        return (F32(1.0) / (F32(1.0) + np.exp(-g))).astype(F32)


def swiglu_quant(gu, weights, inter: int, limit: float, permute: bool = False) -> np.ndarray:
    """h = fq8(bf16(w * silu(min(g, L)) * clamp(u, +-L))) per 32 (fused.py:284-306, 334-345; torch twin
    model._swiglu model.py:608-613 + quant.fake_quant_fp8, equality test_fused.py:81-88). Returns fp32
    values of the bf16 output [rows, inter]; permute=True stores the 8-k permuted order (fused.py:303-305)."""
    gu = np.asarray(gu, dtype=F32)
    gate, up = gu[:, :inter].copy(), gu[:, inter:2 * inter].copy()
    if limit > 0:
        up = np.clip(up, F32(-limit), F32(limit))
        gate = np.minimum(gate, F32(limit))
    h = ((gate * sigmoid_f32(gate)).astype(F32) * up).astype(F32)
    if weights is not None:
        h = (h * np.asarray(weights, dtype=F32).reshape(-1, 1)).astype(F32)
    h = bf16_round(h)
    h = fake_quant_fp8(h, 32)
    if permute:
        h = permute_x(h)
    return h


# --------------------------------------------------------------------------- routing
def gate_topk(scores, bias, temp: float, topk: int, route_scale: float, score_func: str, norm: bool):
    """MoE gate on precomputed logits (model.py:391-404; fused2.py:419-452): scoring function, + bias for
    the selection only, top-k with the lowest index winning ties, weights renormalised (+1e-20) and scaled."""
    s = np.asarray(scores, dtype=F32) / F32(temp)
    if score_func == "softmax":
        mx = s.max(axis=-1, keepdims=True)
        ex = np.exp(s - mx).astype(F32)
        s = (ex / ex.sum(axis=-1, keepdims=True)).astype(F32)
    elif score_func == "sigmoid":
        s = sigmoid_f32(s)
    else:
        with np.errstate(over="ignore"):
            sp = np.where(s > 20.0, s, np.log1p(np.exp(s))).astype(F32)
        s = np.sqrt(sp).astype(F32)
    b = (s + (np.zeros(s.shape[-1], F32) if bias is None else np.asarray(bias, F32))).astype(F32)
    # stable sort of -b: equal values keep ascending index order -> lowest index first
    idx = np.argsort(-b, axis=-1, kind="stable")[:, :topk].astype(np.int32)
    w = np.take_along_axis(s, idx, axis=-1).astype(F32)
    if norm:
        w = (w / (w.sum(axis=-1, keepdims=True) + F32(1e-20))).astype(F32)
    w = (w * F32(route_scale)).astype(F32)
    return idx, w


def moe_dispatch(eid, wt, topk: int, n_experts: int, gmax: int):
    """Expert bucketing (p2p.cu:90-132, cukern.py:323-337) with a deterministic within-expert order
    (ascending pair index). The reference's order within an expert is arbitrary (atomic cursors,
    p2p.cu:91-93): tests compare against this through order-free invariants."""
    eid = np.asarray(eid, dtype=np.int64).reshape(-1)
    wt = np.asarray(wt, dtype=F32).reshape(-1)
    n = eid.size
    # ids outside [0, n_experts) are dropped (the reference indexes its histogram with them, p2p.cu:106: undefined);
    # a dropped pair has inv = -1, and the slots past the placed pairs hold token 0 / weight 0
    keep = (eid >= 0) & (eid < n_experts)
    order = np.argsort(np.where(keep, eid, n_experts), kind="stable")[: int(keep.sum())]
    placed = order.size
    tok_sorted = np.zeros(n, np.int32)
    wt_sorted = np.zeros(n, F32)
    tok_sorted[:placed] = order // topk
    wt_sorted[:placed] = wt[order]
    inv = np.full(n, -1, np.int32)
    inv[order] = np.arange(placed, dtype=np.int32)
    counts = np.bincount(eid[keep], minlength=n_experts)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    ge, gs = [], []
    for e in range(n_experts):
        for t in range(0, counts[e], gmax):
            ge.append(e)
            gs.append(starts[e] + t)
    G = len(ge)
    grp_expert = np.full(n, -1, np.int32)
    grp_start = np.full(n + 1, placed, np.int32)
    grp_expert[:G] = ge
    grp_start[:G] = gs
    return tok_sorted, wt_sorted, inv, grp_expert, grp_start, G


# --------------------------------------------------------------------------- GEMMs and the layer
def dense_weights(w, s) -> np.ndarray:
    """fp32 values of dequant_fp4 (bf16-exact) for [N, K/2] / [N, K/32] (row-major layout)."""
    return dequant_fp4_values(w, s)


def grouped_gemm(x, w, s, grp_expert, grp_start, pair_tok, G: int) -> np.ndarray:
    """out[p, n] = sum_k x[pair_tok[p], k] * deq(W[grp_expert[g]])[n, k] for the pairs p of group g
    (cukern.py:238-276 fp4_gemm_tc; test_fp4_tcw.py:55-58), fp32 accumulation (done in fp64 here)."""
    x = np.asarray(x, dtype=np.float64)
    n_pairs = int(grp_start[G])
    N = w.shape[1]
    out = np.zeros((n_pairs, N), np.float64)
    cache = {}
    for g in range(G):
        e = int(grp_expert[g])
        if e not in cache:
            cache[e] = dense_weights(w[e], s[e]).astype(np.float64)
        a, b = int(grp_start[g]), int(grp_start[g + 1])
        out[a:b] = x[np.asarray(pair_tok[a:b], dtype=np.int64)] @ cache[e].T
    return out.astype(F32)


def gemv_pairs(x, w, s, row_in, expert, wt) -> np.ndarray:
    """out[p, n] = wt[p] * x[row_in[p]] . deq(W[expert[p]])[n] (cukern.py:60-77, fp4_gemv.cu:15-66)."""
    x = np.asarray(x, dtype=np.float64)
    P = len(row_in)
    out = np.zeros((P, w.shape[1]), np.float64)
    for p in range(P):
        W = dense_weights(w[int(expert[p])], s[int(expert[p])]).astype(np.float64)
        out[p] = float(wt[p]) * (W @ x[int(row_in[p])])
    return out.astype(F32)


def expert_pair(xq_row, W13, S13, W2, S2, wt: float, inter: int, limit: float):
    """One (token, expert) pair of the layer (test_cpumoe.py:19-25, fused.py:284-306, decode.py:316-335):
    gu = xq . deq(W13)^T ; h = swiglu_quant(gu, w) ; y2 = h . deq(W2)^T. fp32 [H], fp32 accumulation."""
    gu = (dense_weights(W13, S13) @ np.asarray(xq_row, F32)).astype(F32)
    h = swiglu_quant(gu.reshape(1, -1), np.array([wt], F32), inter, limit)[0]
    return (dense_weights(W2, S2) @ h.astype(F32)).astype(F32)


def deq64(w, s):
    return dense_weights(w, s).astype(np.float64)


def linear_bf16(x, W_bits) -> np.ndarray:
    """F.linear of bf16 x and bf16 W (W given as bf16 bit patterns [N, K]) with a bf16 result: fp32 accumulation,
    one rounding (what linear_w does for a bf16 weight, w8.py:102-103). Returns fp32 values of the bf16 result."""
    W = bf16_bits_to_f32(W_bits)
    return bf16_round((np.asarray(x, F32) @ W.T).astype(F32))


# --------------------------------------------------------------------------- FP8 dense weights (W8)
def dequant_fp8_block_f32(w, scale, block: int = 32) -> np.ndarray:
    """fp32 product e4m3(w) x 2^(S-127), one E8M0 byte per 32 x 32 block, before the bf16 cast (quant.py:90-95).
    w: uint8 E4M3 bytes [N, K]; scale: uint8 [ceil(N/32), ceil(K/32)]."""
    w = np.asarray(w, dtype=np.uint8)
    N, K = w.shape
    s = e8m0_to_f32(np.asarray(scale, dtype=np.uint8))[: -(-N // block), : -(-K // block)]
    s = np.repeat(np.repeat(s, block, axis=0)[:N], block, axis=1)[:, :K]
    with np.errstate(invalid="ignore", over="ignore"):
        return (e4m3_decode(w) * s).astype(F32)


def dequant_fp8_block(w, scale, block: int = 32) -> np.ndarray:
    """-> bf16 bit patterns [N, K] (quant.py:90-95: (w.float() * s).to(torch.bfloat16))."""
    return f32_to_bf16_bits(dequant_fp8_block_f32(w, scale, block))


def linear_fp8w(x, w, scale, group_cols: int = 0) -> np.ndarray:
    """x @ dequant_fp8_block(w, scale)^T with fp32 accumulation of exact products (w8.linear_w, w8.py:102-113;
    cukern.fp8_gemm_tc, cukern.py:114-173), summed in float64 here and rounded to fp32. group_cols > 0: block-diagonal
    use (cukern.py:119-121): x has B * (N / group_cols) rows and output [b, n] uses x row b * (N / group_cols) +
    n // group_cols. Returns fp32 [rows, N] before the bf16 output rounding."""
    W = bf16_bits_to_f32(dequant_fp8_block(w, scale)).astype(np.float64)
    x = np.asarray(x, dtype=np.float64)
    if not group_cols:
        return (x @ W.T).astype(F32)
    N, K = W.shape
    G = N // group_cols
    xg = x.reshape(-1, G, K)
    out = np.empty((xg.shape[0], N), dtype=np.float64)
    for g in range(G):
        cols = slice(g * group_cols, (g + 1) * group_cols)
        out[:, cols] = xg[:, g, :] @ W[cols].T
    return out.astype(F32)


def shared_expert(xq, Ws13, Ws2, inter: int, limit: float) -> np.ndarray:
    """Shared expert with bf16 weights (model.py:409-412, decode.py:368-370): gu = linear_w(xq, Ws13) is a bf16
    tensor (F.linear on bf16), h = swiglu_quant(gu, no weight) (bf16 on the FP8 grid), ys = linear_w(h, Ws2),
    bf16. Ws13 = [w1; w3] and Ws2 as bf16 bit patterns. Returns fp32 values of the bf16 ys [M, H]."""
    gu = linear_bf16(xq, Ws13)
    h = swiglu_quant(gu, None, inter, limit)
    return linear_bf16(h, Ws2)


def moe_layer_routed(xq, eid, wt, W13, S13, W2, S2, inter: int, limit: float) -> np.ndarray:
    """Routed part of one MoE layer for M tokens (model.py:578-581; decode.py:316-335): fp32 [M, H] =
    sum over j (fixed order) of the pair outputs, routing weight folded into h before rounding
    (fused.py:297-302)."""
    xq = np.asarray(xq, F32)
    M, k = np.shape(eid)
    H = W2.shape[1]
    y = np.zeros((M, H), F32)
    # fp32 BLAS products (fp32 accumulation, as the reference's kernels); experts dequantised once each
    experts = sorted({int(e) for e in np.asarray(eid).reshape(-1)})
    gu_all = {}
    for e in experts:
        A13 = dense_weights(W13[e], S13[e])
        toks = [t for t in range(M) if e in [int(v) for v in eid[t]]]
        gu_all[e] = {t: (A13 @ xq[t]).astype(F32) for t in toks}
        del A13
    y2 = {}
    for e in experts:
        A2 = dense_weights(W2[e], S2[e])
        for t, gu in gu_all[e].items():
            for j in [jj for jj, v in enumerate(eid[t]) if int(v) == e]:   # every pair of t naming e (ids may repeat)
                h = swiglu_quant(gu.reshape(1, -1), np.array([wt[t][j]], F32), inter, limit)[0]
                y2[(t, j)] = (A2 @ h).astype(F32)
        del A2
    for t in range(M):
        acc = np.zeros(H, F32)
        for j in range(k):
            acc = (acc + y2[(t, j)]).astype(F32)
        y[t] = acc
    return y


def moe_layer(x_bf16_vals, eid, wt, W13, S13, W2, S2, Ws13, Ws2, inter: int, limit: float) -> np.ndarray:
    """Whole layer: y = bf16(sum_j y2_j + ys) (model.py:554-591; fused2.py:490-495). Input x is fp32
    values of a bf16 tensor; it is FP8 fake-quantised first (model.py:565). Returns fp32 values of bf16."""
    xq = fake_quant_fp8(np.asarray(x_bf16_vals, F32))
    y = moe_layer_routed(xq, eid, wt, W13, S13, W2, S2, inter, limit)
    if Ws13 is not None:
        y = (y + shared_expert(xq, Ws13, Ws2, inter, limit)).astype(F32)
    return bf16_round(y)


# --------------------------------------------------------------------------- hyper-connection steps around the experts
def hc_pre_norm_quant(x, pre, w, eps: float):
    """The decode block's hyper-connection pre-mix + rmsnorm + FP8 fake quant (fused2.py:121-151; the two-pass twin
    fused2.py:180-236): a = bf16(sum_h pre[h] x_h) (fp32), y = bf16(a * (1 / sqrt(mean(a^2) + eps)) * w),
    yq = fake_quant_fp8(y). x [B, hc, d] (values of bf16), pre [B, hc], w [d]. Returns (y, yq) as fp32 values of bf16.
    The sums are evaluated in float64 and rounded once to fp32 (the kernels' fp32 order differs by at most an ulp)."""
    x = np.asarray(x, np.float64)
    pre = np.asarray(pre, np.float64)
    a = bf16_round((pre[:, :, None] * x).sum(1).astype(F32))
    var = ((a.astype(np.float64) ** 2).sum(-1, keepdims=True) / a.shape[-1]).astype(F32)
    inv = (F32(1.0) / np.sqrt(var + F32(eps))).astype(F32)
    y = bf16_round((a * inv * np.asarray(w, F32)).astype(F32))
    return y, fake_quant_fp8(y).astype(F32)


def hc_post(x, res, post, comb):
    """In-place hyper-connection post mix (fused2.py:476-508): r_i <- bf16(post[i] x + sum_j comb[j][i] r_j) per row, the 4
    streams of res [B, 4, d] (values of bf16); x [B, d]; post [B, 4]; comb [B, 4, 4]. Evaluated in float64, rounded once."""
    x = np.asarray(x, np.float64)
    res = np.asarray(res, np.float64)
    post = np.asarray(post, np.float64)
    comb = np.asarray(comb, np.float64)
    out = post[:, :, None] * x[:, None, :] + (comb[:, :, :, None] * res[:, :, None, :]).sum(1)
    return bf16_round(out.astype(F32))


def hc_post_input(y2, ys):
    """x of the post mix from the MoE pieces (fused2.py:490-495): bf16(sum_k y2_k + ys), y2 [B, nsum, d] fp32, ys [B, d]."""
    s = np.asarray(y2, np.float64).sum(1) + (0.0 if ys is None else np.asarray(ys, np.float64))
    return bf16_round(s.astype(F32))


# --------------------------------------------------------------------------- host (CPU) int8 path
# Twice the E2M1 value of each code: the int8 weights of the CPU library's int8 mode (moe_cpu.cpp:210-216).
FP4_TABLE_X2 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], dtype=np.int64)


def int8_quant_blocks(v, block: int = 32):
    """Per-block symmetric int8 re-quantisation of an activation (quant_x_u8, moe_cpu.cpp:218-228):
    s = fp32(amax / 127) (s = 1 for an all-zero block), q = clamp(rint(fp32(v * fp32(1 / s))), -127, 127).
    Returns (q int64 [..., K], s fp32 [..., K / block])."""
    v = np.asarray(v, F32)
    g = v.reshape(*v.shape[:-1], v.shape[-1] // block, block)
    amax = np.abs(g).max(-1)
    s = np.where(amax > 0, (amax / F32(127.0)).astype(F32), F32(1.0)).astype(F32)
    inv = (F32(1.0) / s).astype(F32)
    q = np.clip(np.rint((g * inv[..., None]).astype(F32)), -127, 127).astype(np.int64)
    return q.reshape(v.shape), s


def w4a8_gemv(w, s, v) -> np.ndarray:
    """The CPU library's int8-mode GEMV (dot_row_v2 / dot_row_vnni, moe_cpu.cpp:237-301): per 32-block, the
    exact integer dot of q (int8_quant_blocks of v) with twice the E2M1 codes of w, times 2^(scale byte - 127)
    (byte 0 -> 0) * s_v / 2; blocks summed in float64. w [N, K/2] u8, s [N, K/32] u8, v [K] -> float64 [N]."""
    w = np.asarray(w, np.uint8)
    N = w.shape[0]
    K = w.shape[1] * 2
    codes = np.empty((N, K), np.int64)
    codes[:, 0::2] = FP4_TABLE_X2[w & 0x0F]
    codes[:, 1::2] = FP4_TABLE_X2[w >> 4]
    q, sv = int8_quant_blocks(np.asarray(v, F32).reshape(K))
    dots = (codes.reshape(N, K // 32, 32) * q.reshape(1, K // 32, 32)).sum(-1)
    s = np.asarray(s, np.int64)
    sw = np.where(s == 0, 0.0, np.ldexp(1.0, s - 127))
    return (dots.astype(np.float64) * sw * (sv.astype(np.float64) * 0.5)[None, :]).sum(1)


def swiglu_quant_host(gu, wt: float, inter: int, limit: float) -> np.ndarray:
    """Stage 2 of the CPU library (swiglu_quant_cols, moe_cpu.cpp:357-377) in its operation order:
    v = bf16(fp32(fp32(wt * fp32(g / (1 + exp(-g)))) * u)), then fq8 per 32 (amax floor 1e-4), over ALL inter
    columns (the reference skips the columns past the last full 256-block, moe_cpu.cpp:444; this oracle does not).
    gu [2 * inter] fp32 -> fp32 values of the bf16 h [inter]."""
    gu = np.asarray(gu, F32)
    g, u = gu[:inter].copy(), gu[inter:2 * inter].copy()
    if limit > 0:
        u = np.clip(u, F32(-limit), F32(limit))
        g = np.minimum(g, F32(limit))
    with np.errstate(over="ignore"):
        silu = (g / (F32(1.0) + np.exp(-g).astype(F32))).astype(F32)
    v = bf16_round(((F32(wt) * silu).astype(F32) * u).astype(F32))
    return fake_quant_fp8(v.reshape(1, -1), 32)[0]


def host_layer(x, ids, wts, W13, S13, W2, S2, inter: int, limit: float, int8: bool = True):
    """One token through the CPU library's three stages (cpumoe_forward, moe_cpu.cpp:386-503), with every
    column of h computed. x: fp32 values of the bf16 input [K]; W13 [E, 2I, K/2], W2 [E, H, I/2] (+ scales).
    int8=True: the int8 mode (w4a8_gemv); False: exact fp32-dequantised GEMVs (mode 0, dot_row,
    moe_cpu.cpp:177-205), both evaluated in float64. Returns (gu fp32 [n, 2I], h fp32 [n, I], out float64 [H])."""
    x = np.asarray(x, F32)
    gus, hs = [], []
    out = np.zeros(W2.shape[1], np.float64)
    for e, wt in zip(ids, wts):
        if int8:
            gu = w4a8_gemv(W13[e], S13[e], x).astype(F32)
        else:
            gu = (dense_weights(W13[e], S13[e]).astype(np.float64) @ x.astype(np.float64)).astype(F32)
        h = swiglu_quant_host(gu, float(wt), inter, limit)
        if int8:
            out += w4a8_gemv(W2[e], S2[e], h)
        else:
            out += dense_weights(W2[e], S2[e]).astype(np.float64) @ h.astype(np.float64)
        gus.append(gu)
        hs.append(h)
    return np.stack(gus), np.stack(hs), out


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs_over_rms(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    rms = float(np.sqrt(np.mean(b * b)))
    return float(np.abs(a - b).max() / max(rms, 1e-30))
