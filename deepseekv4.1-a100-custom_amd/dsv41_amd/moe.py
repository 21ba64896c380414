"""The FP4 MoE expert path of one layer on MI355X: routed experts (decode, M <= 16 tokens), the bf16 shared
expert, routing and the combine, as HIP kernels launched on torch's current stream.

Decode (decode.py:316-372 experts_tc / moe2; model.py:554-591 MoE.__call__ for <= 16 tokens), two launches:
  1. dsv41_moe_decode_up: routing from the logits (gate_topk, fused2.py:418-452) or given ids / weights, the
     (token, expert) pairs bucketed by expert (moe_dispatch order), xq (bf16 on the FP8 grid) re-encoded as
     E4M3 + E8M0 in LDS (exact), gu = x . deq(W13[e])^T for 32 SwiGLU columns per workgroup and
     h = fq8(bf16(w * silu(min(g, L)) * clamp(u, +-L))) written as FP8 codes (routing weight folded in before
     rounding, fused.py:297-302); gate/up never leave the chip
  2. dsv41_moe_down_sum: y[t] = sum over t's experts of h . deq(W2)^T in one MFMA accumulator,
     out = bf16(y + ys) (fused2.py:490-495)
Only the selected experts' weight bytes are read from HBM.

Workspaces are allocated once per (device, shape) and reused, so a captured graph replays without allocating.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .fused2 import _MODES


@dataclass
class ExpertWeights:
    """One layer's routed experts in the checkpoint format (load.py:128-148): w13 uint8 [E, 2I, H/2] (w1 rows then
    w3 rows), s13 uint8 [E, 2I, H/32], w2 uint8 [E, H, I/2], s2 uint8 [E, H, I/32]; `tiled`: tile_fp4 layout."""
    w13: torch.Tensor
    s13: torch.Tensor
    w2: torch.Tensor
    s2: torch.Tensor
    tiled: bool = True

    @property
    def E(self) -> int:
        return self.w13.shape[0]

    @property
    def H(self) -> int:
        return self.w2.shape[1]

    @property
    def I(self) -> int:
        return self.w2.shape[2] * 2

    def check(self):
        E, H, I = self.E, self.H, self.I
        assert self.w13.shape == (E, 2 * I, H // 2) and self.s13.shape == (E, 2 * I, H // 32)
        assert self.w2.shape == (E, H, I // 2) and self.s2.shape == (E, H, I // 32)
        for t in (self.w13, self.s13, self.w2, self.s2):
            assert t.dtype == torch.uint8 and t.is_contiguous() and t.is_cuda
        assert H % 128 == 0 and I % 128 == 0 and (2 * I) % 16 == 0 and H % 16 == 0

    def expert_bytes(self) -> int:
        """Packed bytes of one expert (weights + scales of w13 and w2)."""
        per = lambda t: t[0].numel() * t.element_size()
        return per(self.w13) + per(self.s13) + per(self.w2) + per(self.s2)


@dataclass
class SharedExpert:
    """The shared expert of a layer (model.py:385-387, 409-412): w13 = [w1; w3] [2I, H] (gate rows, then up rows) and
    w2 [H, I]. bf16 (s13 / s2 None): `tiled` puts both in the tile_bf16 layout (16 x 32 tiles of 1 KiB, one contiguous
    block per wave-load), which the decode kernels stream faster than row-major rows. FP8 (the checkpoint's format,
    w8.W8): w13 / w2 hold the E4M3 bytes in the w8 tile order and s13 / s2 their E8M0 block scales."""
    w13: torch.Tensor
    w2: torch.Tensor
    tiled: bool = False
    s13: torch.Tensor | None = None
    s2: torch.Tensor | None = None

    @property
    def I(self) -> int:
        return self.w2.shape[1]

    @property
    def fp8(self) -> bool:
        return self.s13 is not None

    @classmethod
    def of(cls, shared) -> "SharedExpert | None":
        """A SharedExpert from one, from a (w13, w2) row-major bf16 pair, or from a (W8, W8) pair; None stays None."""
        if shared is None or isinstance(shared, SharedExpert):
            return shared
        w13, w2 = shared
        from .w8 import W8
        if isinstance(w13, W8):
            return cls.prepare_w8(w13, w2)
        return cls(w13, w2, False)

    @classmethod
    def prepare(cls, w13: torch.Tensor, w2: torch.Tensor, tiled: bool = True) -> "SharedExpert":
        """From row-major [w1; w3] and w2 (bf16, on the GPU), repacked once into the tiled layout when `tiled`."""
        from .quant import tile_bf16
        w13, w2 = w13.to(torch.bfloat16).contiguous(), w2.to(torch.bfloat16).contiguous()
        return cls(tile_bf16(w13), tile_bf16(w2), True) if tiled else cls(w13, w2, False)

    @classmethod
    def prepare_w8(cls, w13, w2) -> "SharedExpert":
        """From W8 [w1; w3] and w2 as loaded (tiled FP8 bytes + E8M0 block scales): no copy."""
        assert w13.tiled and w2.tiled, "the fused FP8 shared expert reads the w8 tile order"
        return cls(w13.w8, w2.w8, True, w13.s8, w2.s8)

    def check(self, H: int, I: int):
        assert tuple(self.w13.shape) == (2 * I, H) and tuple(self.w2.shape) == (H, I)
        assert self.w13.stride(1) == 1 and self.w2.stride(1) == 1
        if self.fp8:
            assert self.w13.dtype == torch.uint8 and self.w2.dtype == torch.uint8 and self.tiled
            assert self.w13.is_contiguous() and self.w2.is_contiguous() and self.s13.is_contiguous() and self.s2.is_contiguous()
            assert tuple(self.s13.shape) == ((2 * I + 31) // 32, H // 32) and tuple(self.s2.shape) == ((H + 31) // 32, I // 32)
            return
        assert self.w13.dtype == torch.bfloat16 and self.w2.dtype == torch.bfloat16
        if self.tiled:
            assert self.w13.is_contiguous() and self.w2.is_contiguous()


class _Workspace:
    def __init__(self, dev, M, k, H, I):
        P = M * k
        u8, i32, f32 = torch.uint8, torch.int32, torch.float32
        self.M, self.k, self.P = M, k, P
        # row P of hc / hs stays zero: the down projection reads it for tokens a group does not contain
        self.hc = torch.zeros(P + 1, I, dtype=u8, device=dev)
        self.hs = torch.zeros(P + 1, I // 32, dtype=u8, device=dev)
        self.y = torch.empty(M, H, dtype=f32, device=dev)
        self.tok_sorted = torch.empty(P, dtype=i32, device=dev)
        self.wt_sorted = torch.empty(P, dtype=f32, device=dev)
        self.grp_expert = torch.empty(P, dtype=i32, device=dev)
        self.grp_start = torch.empty(P + 1, dtype=i32, device=dev)
        self.eid = torch.empty(M, k, dtype=i32, device=dev)       # routing, when the caller keeps none
        self.wt = torch.empty(M, k, dtype=f32, device=dev)
        self.gus = torch.empty(M, 2 * I, dtype=torch.bfloat16, device=dev)   # the fused shared expert's gate/up
        self.shared = None                                          # the SharedExpert of the last decode_up, if fused
        self.part = None                                            # run-split down projection: partial sums


def _down_split(ws: "_Workspace", ex: ExpertWeights) -> bool:
    """Whether the down projection runs split over runs of pair rows (dsv41_moe_down_sum_split): when the h rows do not
    fit the one-launch kernel's LDS (60 KiB with their E8M0 bytes), for intermediate sizes it takes."""
    I, R = ex.I, ws.P + 1
    staged = R * (I + 16 + I // 32) <= 60 * 1024 and R * (I // 16) <= 8 * 512 and R * (I // 32) <= 4 * 512
    return not staged and I % 128 == 0 and I <= 2048 and ex.H % 128 == 0


def fused_shared_ok(M: int, k: int, I: int, fp8: bool = False) -> bool:
    """Whether the shared expert can ride in the two decode launches (dsv41_moe_down_sum's limits: the h rows, their
    scales and M bf16 h_s rows in 60 KiB with at most 4 h vectors per thread, M I <= 4096; bf16: I / 32 <= 56 chunks
    per row block, FP8: I / 64 <= 40); otherwise it runs as its own launches."""
    P = M * k
    lds = (((P + 1) * (I + 16) + (P + 1) * (I // 32) + 15) & ~15) + M * (I + 8) * 2
    chunks_ok = (I % 64 == 0 and I // 64 <= 5 * 8) if fp8 else I // 32 <= 7 * 8
    return (lds <= 60 * 1024 and (P + 1) * (I // 16) <= 4 * 512 and (P + 1) * (I // 32) <= 2 * 512 and M * I <= 4096 and P <= 256
            and chunks_ok)


_WS: dict = {}


def _workspace(dev, M, k, H, I) -> _Workspace:
    key = (dev, M, k, H, I)
    ws = _WS.get(key)
    if ws is None:
        ws = _WS[key] = _Workspace(dev, M, k, H, I)
    return ws


def _as(t: torch.Tensor, dtype) -> torch.Tensor:
    t = t.reshape(-1)
    if t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def decode_up(xq, ex: ExpertWeights, limit: float, k: int, logits=None, gate=None, eid=None, wt=None, eid_out=None, wt_out=None,
              shared=None, pairs: bool = False):
    """The first of the two decode launches (dsv41_moe_decode_up): routing (from `logits` with gate = (bias,
    temp, route_scale, score_func, norm), or the given eid / wt), bucketing, up projection and SwiGLU; with
    shared (a SharedExpert or a row-major (w13, w2) pair) also the shared expert's gate/up (decode_down finishes it).
    Returns the workspace holding h (codes + E8M0, expert-sorted pair rows) and the tables for decode_down.
    pairs (M > 1): the tokens pair by pair (dsv41_moe_decode_up_pairs): every (token, pick) pair is its own group and h
    row, routed inside the launch from that token's logits (no gate launch, no bucketing)."""
    dev = _lib.require_cuda(xq, logits, eid, wt)
    M, H = xq.shape
    assert 1 <= M <= 16, "decode path: at most 16 tokens (use the prefill path beyond)"
    assert H == ex.H and xq.dtype == torch.bfloat16 and 1 <= k <= 16 and ex.E <= 512
    if xq.stride(1) != 1 or xq.stride(0) % 8 or xq.data_ptr() % 16:
        xq = xq.contiguous()
    ws = _workspace(dev, M, k, H, ex.I)
    if logits is not None:
        # logits fp32 [M, E], or [parts, M, E] partial sums (dsv41_router_logits), added in part order
        bias, temp, route_scale, score_func, norm = gate
        lg = logits if (logits.dtype == torch.float32 and logits.is_contiguous()) else logits.float().contiguous()
        parts = lg.shape[0] if lg.dim() == 3 else 1
        b = None if bias is None else _as(bias, torch.float32)
        assert lg.shape[-1] == ex.E and lg.shape[-2] == M and (b is None or b.numel() == ex.E)
        route = (_lib.ptr(lg), ex.E, parts, M * ex.E, _lib.ptr(b), float(temp), float(route_scale), _MODES[score_func], 1 if norm else 0,
                 None, None)
    else:
        eid32, wt32 = _as(eid, torch.int32), _as(wt, torch.float32)
        route = (None, ex.E, 1, 0, None, 1.0, 1.0, 0, 0, _lib.ptr(eid32), _lib.ptr(wt32))
    sh = SharedExpert.of(shared)
    Ws13 = Ss13 = None
    if sh is not None:
        sh.check(H, ex.I)
        assert fused_shared_ok(M, k, ex.I, sh.fp8)
        Ws13, Ss13 = sh.w13, sh.s13
    ws.shared = sh
    _lib.call("dsv41_moe_decode_up_pairs" if pairs else "dsv41_moe_decode_up", *route, M, k, ex.E, _lib.ptr(xq), xq.stride(0), _lib.ptr(ex.w13), ex.w13.stride(0), _lib.ptr(ex.s13),
              ex.s13.stride(0), 1 if ex.tiled else 0, H, ex.I, float(limit), _lib.ptr(ws.hc), ws.hc.stride(0), _lib.ptr(ws.hs), ws.hs.stride(0),
              _lib.ptr(eid_out), _lib.ptr(wt_out), _lib.ptr(ws.grp_expert), _lib.ptr(ws.grp_start), _lib.ptr(ws.tok_sorted),
              _lib.ptr(ws.wt_sorted), _lib.ptr(Ws13), H if Ws13 is None else Ws13.stride(0), 1 if sh is not None and sh.tiled else 0,
              _lib.ptr(ws.gus), ws.gus.stride(0), _lib.ptr(Ss13), 0 if Ss13 is None else Ss13.stride(0), _lib.stream(dev))
    return ws


def decode_down(ws: _Workspace, ex: ExpertWeights, ys=None, out=None, y32=None, limit: float = 0.0, ys_out=None, hc=None,
                split: bool | None = None):
    """The second decode launch (dsv41_moe_down_sum): y[t] = sum over t's groups of h . deq(W2[e])^T (fp32, into
    y32 or the workspace) and/or out = bf16(y + ys). When decode_up ran with the shared expert, this launch finishes it
    (SwiGLU with `limit`, Ws2) and adds its bf16 output instead of `ys` (ys_out, bf16 [M, H], receives it).
    hc = (residual bf16 [M, 1, 4, H], post fp32 [M, 4], comb fp32 [M, 4, 4]): the hyper-connection post mix
    (fused2.hc_post2_) applied to bf16(y + ys) in the same launch, in place on residual. split: run-split form
    (dsv41_moe_down_sum_split) or not; None: when the h rows do not fit the one-launch kernel's LDS."""
    dev = _lib.require_cuda(ws.hc, ys, out, y32, ys_out)
    hres = hpost = hcomb = None
    if hc is not None:
        hres, hpost, hcomb = hc
        assert hres.dtype == torch.bfloat16 and hres.is_contiguous() and hres.numel() == ws.M * 4 * ex.H
        hpost = hpost.reshape(ws.M, 4).to(torch.float32).contiguous()
        hcomb = hcomb.reshape(ws.M, 16).to(torch.float32).contiguous()
    M, H = ws.M, ex.H
    y = ws.y if y32 is None else y32
    want_y = (out is None and hc is None) or y32 is not None
    Ws2 = Ss2 = None
    if ws.shared is not None:
        Ws2, Ss2 = ws.shared.w2, ws.shared.s2
        assert ys is None
    elif _down_split(ws, ex) if split is None else split:
        q = max(1, min(32 - M, (ws.P + 7) // 8))   # pair rows per run, as dsv41_moe_down_sum_split chooses them
        runs = max(1, (ws.P + q - 1) // q)
        if ws.part is None or ws.part.numel() < runs * M * H:
            ws.part = torch.empty(runs * M * H, dtype=torch.float32, device=dev)
        _lib.call("dsv41_moe_down_sum_split", _lib.ptr(ex.w2), ex.w2.stride(0), _lib.ptr(ex.s2), ex.s2.stride(0), 1 if ex.tiled else 0, H,
                  ex.I, _lib.ptr(ws.hc), ws.hc.stride(0), _lib.ptr(ws.hs), ws.hs.stride(0), _lib.ptr(ws.grp_expert), _lib.ptr(ws.grp_start),
                  _lib.ptr(ws.tok_sorted), ws.P, M, _lib.ptr(y) if want_y else None, y.stride(0), _lib.ptr(ys), H if ys is None else ys.stride(0),
                  _lib.ptr(out), H if out is None else out.stride(0), 0, ex.E, _lib.ptr(hres), _lib.ptr(hpost), _lib.ptr(hcomb),
                  _lib.ptr(ws.part), ws.part.numel(), _lib.stream(dev))
        if hc is not None and out is None:
            return hres
        return out if out is not None else y
    _lib.call("dsv41_moe_down_sum", _lib.ptr(ex.w2), ex.w2.stride(0), _lib.ptr(ex.s2), ex.s2.stride(0), 1 if ex.tiled else 0, H, ex.I,
              _lib.ptr(ws.hc), ws.hc.stride(0), _lib.ptr(ws.hs), ws.hs.stride(0), ws.P, _lib.ptr(ws.grp_expert), _lib.ptr(ws.grp_start),
              _lib.ptr(ws.tok_sorted), ws.P, M, _lib.ptr(y) if want_y else None, y.stride(0), _lib.ptr(ys), H if ys is None else ys.stride(0),
              _lib.ptr(out), H if out is None else out.stride(0), 0, ex.E, _lib.ptr(ws.gus) if Ws2 is not None else None, ws.gus.stride(0),
              _lib.ptr(Ws2), ex.I if Ws2 is None else Ws2.stride(0), 1 if Ws2 is not None and ws.shared.tiled else 0, float(limit),
              _lib.ptr(ys_out), H if ys_out is None else ys_out.stride(0), _lib.ptr(hres), _lib.ptr(hpost), _lib.ptr(hcomb),
              _lib.ptr(Ss2), 0 if Ss2 is None else Ss2.stride(0), _lib.stream(dev))
    if hc is not None and out is None:
        return hres
    return out if out is not None else y


def _shared_plan(xq, shared, ys, k, ex, limit, ys_out):
    """(shared expert for the fused launches or None, ys): the bf16 shared expert rides in the two decode launches when
    it fits them; otherwise it runs first as its own launches and enters as ys."""
    sh = SharedExpert.of(shared)
    if sh is None:
        return None, ys
    assert ys is None, "give either the shared expert's weights or its output"
    if fused_shared_ok(xq.shape[0], k, ex.I, sh.fp8):
        return sh, None
    if sh.fp8:
        from .w8 import W8
        w13 = W8(sh.w13, sh.s13, permuted=True, tiled=True)
        w2 = W8(sh.w2, sh.s2, permuted=True, tiled=True)
        y_s = shared_expert_rows(xq, w13, w2, ex.I, limit)
        if ys_out is not None:
            ys_out.copy_(y_s)
        return None, y_s
    return None, shared_expert(xq, sh.w13, sh.w2, limit, ys=ys_out, tiled=sh.tiled)


def moe_experts(xq: torch.Tensor, eid: torch.Tensor, wt: torch.Tensor, ex: ExpertWeights, limit: float,
                ys: torch.Tensor | None = None, out: torch.Tensor | None = None, y32: torch.Tensor | None = None,
                shared: tuple | None = None, ys_out: torch.Tensor | None = None, hc: tuple | None = None) -> torch.Tensor:
    """Routed experts of one layer for M <= 16 tokens with given routing.
    xq: bf16 [M, H] on the FP8 grid (fake_quant_fp8 output); eid int [M, k] (distinct per token, except for 2 <= M <=
    PAIRS_MAX_M, which runs pair by pair); wt fp32 [M, k].
    Returns fp32 [M, H] = sum_j w_j-weighted expert outputs (routing weight folded into h, fused.py:297-302),
    or, when `out` (bf16 [M, H]) is given, writes out = bf16(y + ys) (ys: bf16 shared-expert output or None);
    y32 (fp32 [M, H]) additionally receives y. shared (a SharedExpert, or a row-major (w13, w2) bf16 pair) computes
    the shared expert too (model.py:409-412) instead of taking ys: in the same two launches when it fits them
    (fused_shared_ok), else as its own launches first; ys_out (bf16 [M, H]) receives its output. hc = (residual, post,
    comb) applies the hyper-connection post mix to bf16(y + ys) in the same launch (decode_down)."""
    k = eid.shape[-1]
    M = xq.shape[0]
    fused, ys = _shared_plan(xq, shared, ys, k, ex, limit, ys_out)
    # 2 <= M <= PAIRS_MAX_M: pair by pair (faster at these sizes, and a token may then name an expert twice)
    pairs = 1 < M <= PAIRS_MAX_M and ex.H // 16 <= 448
    ws = decode_up(xq, ex, limit, k, eid=eid, wt=wt, shared=fused, pairs=pairs)
    return decode_down(ws, ex, ys, out, y32, limit=limit, ys_out=ys_out if fused is not None else None, hc=hc)


# largest token count run pair by pair (moe_route_experts: routed inside the up launch; moe_experts: given ids): up to
# it the gate launch and the bucketing cost more than reading the few experts two tokens share twice
PAIRS_MAX_M = 4


def moe_route_experts(xq: torch.Tensor, logits: torch.Tensor, bias: torch.Tensor | None, temp: float, topk: int, route_scale: float,
                      score_func: str, norm: bool, ex: ExpertWeights, limit: float, ys: torch.Tensor | None = None,
                      out: torch.Tensor | None = None, y32: torch.Tensor | None = None, eid_out: torch.Tensor | None = None,
                      wt_out: torch.Tensor | None = None, shared: tuple | None = None, ys_out: torch.Tensor | None = None,
                      hc: tuple | None = None) -> torch.Tensor:
    """gate_topk (fused2.py:418-452) with the routed experts: logits fp32 [M, E] -> routing (written to
    eid_out int32 / wt_out fp32 [M, topk] when given) -> the same outputs as moe_experts.
    M = 1: the routing runs inside the up-projection launch (every workgroup routes the one token while its
    activations load). 1 < M <= PAIRS_MAX_M: the same, pair by pair (each (token, pick) pair's workgroups route its
    token; an expert several tokens picked is read once per pair). Larger M: one gate launch first; the up projection
    then reads the ids and streams each selected expert once for all its tokens."""
    M = xq.shape[0]
    gate = (bias, temp, route_scale, score_func, norm)
    fused, ys = _shared_plan(xq, shared, ys, topk, ex, limit, ys_out)
    if M == 1 or (M <= PAIRS_MAX_M and ex.H // 16 <= 448):
        ws = decode_up(xq, ex, limit, topk, logits=logits, gate=gate, eid_out=eid_out, wt_out=wt_out, shared=fused, pairs=M > 1)
    else:
        from .fused2 import gate_topk
        ws0 = _workspace(_lib.require_cuda(xq), M, topk, ex.H, ex.I)
        eid = ws0.eid if eid_out is None else eid_out
        wt = ws0.wt if wt_out is None else wt_out
        gate_topk(logits, bias, temp, topk, route_scale, score_func, norm, eid=eid, wt=wt)
        ws = decode_up(xq, ex, limit, topk, eid=eid, wt=wt, shared=fused)
    return decode_down(ws, ex, ys, out, y32, limit=limit, ys_out=ys_out if fused is not None else None, hc=hc)


# --------------------------------------------------------------------------- dense bf16 (shared expert, router)
def dense_gemv(W: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None, out_bf16: bool = False, tiled: bool = False) -> torch.Tensor:
    """out[t, n] = sum_k x[t, k] W[n, k] for M <= 16 rows of bf16 x and bf16 W [N, K] (fp32 accumulation; `tiled`: W in
    the tile_bf16 layout); fp32 output, or bf16 (round to nearest even) when out_bf16."""
    dev = _lib.require_cuda(W, x)
    M, K = x.shape
    N = W.shape[0]
    assert W.dtype == torch.bfloat16 and x.dtype == torch.bfloat16 and W.shape[1] == K and W.stride(1) == 1 and x.stride(1) == 1
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16 if out_bf16 else torch.float32, device=dev)
    is_b = out.dtype == torch.bfloat16
    assert not tiled or W.is_contiguous()
    _lib.call("dsv41_dense_gemv_bf16", _lib.ptr(W), W.stride(0), 1 if tiled else 0, N, K, _lib.ptr(x), x.stride(0), M,
              None if is_b else _lib.ptr(out), out.stride(0), _lib.ptr(out) if is_b else None, out.stride(0), _lib.stream(dev))
    return out


class PrefillState:
    """Intermediates of the prefill path (sorted pair order): dispatch tables, h codes + E8M0, per-pair y2."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


# pairs per group of the prefill path's dispatch: its launches take groups of up to 256 pairs (groups of more than
# 128 on a 256-pair tile), so a popular expert's weights are streamed by half as many groups
PREFILL_GROUP = 256


def prefill_up(xq: torch.Tensor, eid: torch.Tensor, wt: torch.Tensor, ex: ExpertWeights, limit: float) -> PrefillState:
    """First half of the prefill path: xq bf16 [T, H] on the FP8 grid -> E4M3 codes (exact); (token, expert) pairs
    bucketed by expert in groups of <= PREFILL_GROUP (moe_dispatch, p2p.cu:90-132); the w13 GEMM with the SwiGLU/FP8
    epilogue: h[p] = fq8(bf16(w_p * silu(min(g, L)) * clamp(u, +-L))) (model.py:584-587, fused.py:284-306). The w13
    launch takes the groups largest first (dsv41_group_order), so no long item starts near the end of it: configs[3] w13
    1149-1151 -> 1082-1087 us on one box. (The w2 launch keeps table order: its items are four times shorter, and
    largest first made it slower, 720 -> 746 us, in the same A/B.)"""
    from .hipkern import moe_dispatch
    from .quant import quant_fp8_e8m0
    dev = _lib.require_cuda(xq, eid, wt)
    T, H = xq.shape
    k = eid.shape[-1]
    P = T * k
    I = ex.I
    assert H == ex.H and xq.dtype == torch.bfloat16 and ex.E <= 512
    xc, xs = quant_fp8_e8m0(xq)
    gmax = PREFILL_GROUP
    tok_sorted, wt_sorted, inv, grp_expert, grp_start = moe_dispatch(eid, wt, k, ex.E, gmax, dev)
    G = min(P, ex.E + (P + gmax - 1) // gmax)   # groups of <= gmax pairs: at most E + P / gmax of them
    hc = torch.empty(P, I, dtype=torch.uint8, device=dev)
    hs = torch.empty(P, I // 32, dtype=torch.uint8, device=dev)
    order = torch.empty(G, dtype=torch.int32, device=dev)
    _lib.call("dsv41_group_order", _lib.ptr(grp_expert), _lib.ptr(grp_start), G, P, _lib.ptr(order), _lib.stream(dev))
    _lib.call("dsv41_prefill_up", _lib.ptr(xc), xc.stride(0), _lib.ptr(xs), xs.stride(0), T, _lib.ptr(ex.w13), ex.w13.stride(0), _lib.ptr(ex.s13),
              ex.s13.stride(0), 1 if ex.tiled else 0, ex.E, H, I, _lib.ptr(grp_expert), _lib.ptr(grp_start), G, _lib.ptr(tok_sorted),
              _lib.ptr(wt_sorted), float(limit), _lib.ptr(hc), hc.stride(0), _lib.ptr(hs), hs.stride(0), _lib.ptr(order), _lib.stream(dev))
    return PrefillState(T=T, k=k, P=P, G=G, tok_sorted=tok_sorted, wt_sorted=wt_sorted, inv=inv, grp_expert=grp_expert,
                        grp_start=grp_start, hc=hc, hs=hs, y2=None)


def prefill_down(st: PrefillState, ex: ExpertWeights, ys: torch.Tensor | None = None, out: torch.Tensor | None = None,
                 y32: torch.Tensor | None = None) -> torch.Tensor:
    """Second half: y2[p] = h[p] . deq(W2[e])^T (fp32 per pair, model.py:588), then y[t] = sum over the k slots of
    t in slot order (model.py:589, view(n, k, dim).sum(1)) -> fp32 [T, H], or out = bf16(y + ys) (model.py:590-591)."""
    dev = _lib.require_cuda(st.hc, ys, out, y32)
    H, I, T = ex.H, ex.I, st.T
    s = _lib.stream(dev)
    st.y2 = torch.empty(st.P, H, dtype=torch.float32, device=dev)
    _lib.call("dsv41_prefill_down", _lib.ptr(st.hc), st.hc.stride(0), _lib.ptr(st.hs), st.hs.stride(0), st.P, _lib.ptr(ex.w2), ex.w2.stride(0),
              _lib.ptr(ex.s2), ex.s2.stride(0), 1 if ex.tiled else 0, ex.E, H, I, _lib.ptr(st.grp_expert), _lib.ptr(st.grp_start), st.G,
              _lib.ptr(st.y2), st.y2.stride(0), None, s)
    if out is None and y32 is None:
        y32 = torch.empty(T, H, dtype=torch.float32, device=dev)
    _lib.call("dsv41_combine_pairs", _lib.ptr(st.y2), st.y2.stride(0), _lib.ptr(st.inv), st.k, T, H, _lib.ptr(ys), H if ys is None else ys.stride(0),
              _lib.ptr(out), H if out is None else out.stride(0), _lib.ptr(y32), H if y32 is None else y32.stride(0), s)
    return out if out is not None else y32


def prefill_experts(xq: torch.Tensor, eid: torch.Tensor, wt: torch.Tensor, ex: ExpertWeights, limit: float,
                    ys: torch.Tensor | None = None, out: torch.Tensor | None = None, y32: torch.Tensor | None = None) -> torch.Tensor:
    """Routed experts for many tokens (model.MoE.__call__ beyond 16 tokens, model.py:539-551, 584-591): prefill_up
    then prefill_down. Returns fp32 [T, H], or writes out = bf16(sum + ys)."""
    return prefill_down(prefill_up(xq, eid, wt, ex, limit), ex, ys, out, y32)


def residual_rmsnorm_quant(x: torch.Tensor, y: torch.Tensor, w: torch.Tensor | None = None, eps: float = 1e-6,
                           xn: torch.Tensor | None = None, xq: torch.Tensor | None = None):
    """The step between two MoE layers of the decode stack: r = bf16(x + y), xn = rmsnorm(r) * w (fused.rmsnorm,
    fused.py:92-110), xq = fake_quant_fp8(xn). x, y, w bf16; returns (xn, xq) bf16 [M, H]."""
    dev = _lib.require_cuda(x, y, w, xn, xq)
    M, H = x.shape
    assert x.dtype == y.dtype == torch.bfloat16 and y.shape == x.shape and x.stride(1) == 1 and y.stride(1) == 1
    xn = torch.empty_like(x) if xn is None else xn
    xq = torch.empty_like(x) if xq is None else xq
    wc = None if w is None else w.to(torch.bfloat16).contiguous()
    _lib.call("dsv41_residual_rmsnorm_quant", _lib.ptr(x), x.stride(0), _lib.ptr(y), y.stride(0), _lib.ptr(wc), float(eps), M, H,
              _lib.ptr(xn), xn.stride(0), _lib.ptr(xq), xq.stride(0), _lib.stream(dev))
    return xn, xq


def router_logits(x: torch.Tensor, y: torch.Tensor | None, G: torch.Tensor, w: torch.Tensor | None = None, eps: float = 1e-6,
                  part: torch.Tensor | None = None, xn: torch.Tensor | None = None, xq: torch.Tensor | None = None):
    """The next layer's router logits with the layer-to-layer step fused in (one launch): r = bf16(x + y),
    xn = rmsnorm(r) * w, logits = xn . G^T (bf16 G [E, H]; model.py:391-392). Returns (part, xn, xq): the logits
    as fp32 [H / 1024, M, E] partial sums (what moe_route_experts / gate_topk accept), xn and
    xq = fake_quant_fp8(xn) bf16 [M, H]. xn / xq must not alias x or y."""
    dev = _lib.require_cuda(x, y, G, w, part, xn, xq)
    M, H = x.shape
    E = G.shape[0]
    assert x.dtype == torch.bfloat16 and G.dtype == torch.bfloat16 and G.shape[1] == H and G.stride(1) == 1 and x.stride(1) == 1
    part = torch.empty(H // 1024, M, E, dtype=torch.float32, device=dev) if part is None else part
    xn = torch.empty_like(x) if xn is None else xn
    xq = torch.empty_like(x) if xq is None else xq
    assert part.shape == (H // 1024, M, E) and part.is_contiguous()
    wc = None if w is None else w.to(torch.bfloat16).contiguous()
    _lib.call("dsv41_router_logits", _lib.ptr(x), x.stride(0), _lib.ptr(y), H if y is None else y.stride(0), _lib.ptr(wc), float(eps),
              _lib.ptr(G), G.stride(0), E, H, M, _lib.ptr(part), _lib.ptr(xn), xn.stride(0), _lib.ptr(xq), xq.stride(0), _lib.stream(dev))
    return part, xn, xq


class _SharedWs:
    def __init__(self, dev, M, H, I):
        self.gu = torch.empty(M, 2 * I, dtype=torch.bfloat16, device=dev)
        self.h = torch.empty(M, I, dtype=torch.bfloat16, device=dev)
        self.ys = torch.empty(M, H, dtype=torch.bfloat16, device=dev)


_SWS: dict = {}


def shared_expert(xq: torch.Tensor, Ws13: torch.Tensor, Ws2: torch.Tensor, limit: float, ys: torch.Tensor | None = None,
                  tiled: bool = False) -> torch.Tensor:
    """Shared expert with bf16 weights as its own launches (model.py:409-412, decode.py:368-370): gu = linear_w(xq,
    Ws13) is bf16 (one rounding of the fp32-accumulated product), h = swiglu_quant(gu, no weight) (bf16 on the FP8
    grid), ys = bf16(h . Ws2^T). Ws13 = [w1; w3] bf16 [2I, H]; `tiled`: both in the tile_bf16 layout."""
    dev = _lib.require_cuda(xq, Ws13, Ws2)
    M, H = xq.shape
    I = Ws2.shape[1]
    key = (dev, M, H, I)
    sw = _SWS.get(key)
    if sw is None:
        sw = _SWS[key] = _SharedWs(dev, M, H, I)
    dense_gemv(Ws13, xq, out=sw.gu, tiled=tiled)
    _lib.call("dsv41_swiglu_quant", _lib.ptr(sw.gu), 1, sw.gu.stride(0), None, M, I, float(limit), None, None, _lib.ptr(sw.h), 0, _lib.stream(dev))
    out = sw.ys if ys is None else ys
    dense_gemv(Ws2, sw.h, out=out, tiled=tiled)
    return out


def shared_expert_rows(xq: torch.Tensor, sh_w13, sh_w2, inter: int, limit: float) -> torch.Tensor:
    """bf16 ys = linear_w(swiglu_quant(linear_w(xq, sh_w13)), sh_w2) (decode.py:368-371, model.py:409-412) for
    bf16 tensors or w8.W8 weights: the FP8 GEMM streams W8 weights (up to 64 rows per launch), the library GEMM takes
    bf16 weights or more rows."""
    from .fused import swiglu_quant
    from .w8 import linear_w
    gu = linear_w(xq, sh_w13)
    return linear_w(swiglu_quant(gu, None, inter, limit), sh_w2)


class MoEDecodeLayer:
    """One MoE layer at decode (M <= 16 tokens): router logits (given, or x . G^T with bf16 router weights G),
    gate_topk, the shared expert and the routed FP4 experts, combined as y = bf16(sum_j y2_j + ys)
    (model.py:554-591; decode.py:354-372; fused2.py:474-508)."""

    def __init__(self, experts: ExpertWeights, Ws13: torch.Tensor | None, Ws2: torch.Tensor | None, limit: float,
                 topk: int = 8, score_func: str = "softmax", route_scale: float = 1.0, norm: bool = True,
                 router: torch.Tensor | None = None, bias: torch.Tensor | None = None, temp: float = 1.0):
        experts.check()
        self.ex, self.Ws13, self.Ws2, self.limit = experts, Ws13, Ws2, float(limit)
        # the shared expert as the decode kernels stream it best (tile_bf16 layout, repacked once)
        self.shared = SharedExpert.prepare(Ws13, Ws2, tiled=True) if Ws13 is not None else None
        self.topk, self.score_func, self.route_scale, self.norm = topk, score_func, route_scale, norm
        self.router, self.bias, self.temp = router, bias, temp
        self._bufs: dict = {}

    def _buf(self, dev, M):
        b = self._bufs.get(M)
        if b is None:
            E, H = self.ex.E, self.ex.H
            b = self._bufs[M] = {
                "xq": torch.empty(M, H, dtype=torch.bfloat16, device=dev),
                "logits": torch.empty(M, E, dtype=torch.float32, device=dev),
                "eid": torch.empty(M, self.topk, dtype=torch.int32, device=dev),
                "wt": torch.empty(M, self.topk, dtype=torch.float32, device=dev),
                "ys": torch.empty(M, H, dtype=torch.bfloat16, device=dev),
                "out": torch.empty(M, H, dtype=torch.bfloat16, device=dev),
            }
        return b

    def __call__(self, x: torch.Tensor, logits: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        dev = _lib.require_cuda(x)
        M, H = x.shape
        b = self._buf(dev, M)
        # xq = fake_quant_fp8(x) (model.py:565): one pass writes the bf16 values; the routed path re-derives the
        # codes from them exactly
        _lib.call("dsv41_quant_fp8", _lib.ptr(x), 0, M, H, x.stride(0), 0, None, None, _lib.ptr(b["xq"]), _lib.stream(dev))
        if logits is None:
            assert self.router is not None, "router weights or logits are required"
            logits = dense_gemv(self.router, x, out=b["logits"])
        o = b["out"] if out is None else out
        shared = self.shared
        moe_route_experts(b["xq"], logits, self.bias, self.temp, self.topk, self.route_scale, self.score_func, self.norm and self.topk > 1,
                          self.ex, self.limit, out=o, eid_out=b["eid"], wt_out=b["wt"], shared=shared,
                          ys_out=b["ys"] if shared is not None else None)
        return o

    @property
    def last_routing(self):
        return {M: (v["eid"], v["wt"]) for M, v in self._bufs.items()}


# --------------------------------------------------------------------------- the whole MoE layer (eager / prefill)
def router_logits_f32w(x: torch.Tensor, G: torch.Tensor, part: torch.Tensor | None = None) -> torch.Tensor:
    """Router logits with fp32 router weights G [E, H] for M <= 16 bf16 rows x (F.linear(x.float(), gate_w),
    model.py:392): fp32 [H / 1024, M, E] partial sums over k ranges of 1024, which gate_topk / moe_route_experts add
    in part order."""
    dev = _lib.require_cuda(x, G, part)
    M, H = x.shape
    E = G.shape[0]
    assert x.dtype == torch.bfloat16 and G.dtype == torch.float32 and G.shape[1] == H and G.stride(1) == 1 and x.stride(1) == 1
    part = torch.empty(H // 1024, M, E, dtype=torch.float32, device=dev) if part is None else part
    assert part.shape == (H // 1024, M, E) and part.is_contiguous()
    _lib.call("dsv41_router_logits_f32w", _lib.ptr(x), x.stride(0), _lib.ptr(G), G.stride(0), E, H, M, _lib.ptr(part), _lib.stream(dev))
    return part


class MoE:
    """The expert compute of the reference's model.MoE (model.py:354-413, 554-591) for one layer on the GPU path:
    gate (fp32 router weights, softmax / sigmoid / sqrt(softplus), + bias for the selection, top-k, renormalised and
    scaled), x fake-quantised to FP8 (model.py:565), the routed FP4 experts, the shared expert (bf16, or FP8 w8.W8 as
    the checkpoint stores it), and
    y = bf16(sum_j w_j y2_j + shared) (model.py:589-591).
      * <= 16 tokens (decode): the router GEMV on fp32 weights as split-K partial sums, then the two fused decode
        launches (routing inside the up launch for one token; a bf16 shared expert rides in both launches when it fits
        them, else runs as its own launches first; an FP8 one runs first as two FP8 GEMM launches and a SwiGLU);
      * > 16 tokens (prefill): router logits and the shared expert's two products as plain library GEMMs (F.linear on
        the GPU, as the reference runs them, model.py:392, 410-412; w8.py:102-103), gate_topk, then the prefill grouped
        GEMMs with the slot-ordered combine.
    Attribute names follow the reference (n_experts, topk, score_func, gate_temp, norm_topk_prob, route_scale,
    swiglu_limit, gate_w, gate_bias, inter, sh_w13, sh_w2). Routing of the last call: last_routing."""

    def __init__(self, experts: ExpertWeights, gate_w: torch.Tensor, gate_bias: torch.Tensor | None = None, topk: int = 8,
                 score_func: str = "softmax", route_scale: float = 1.0, norm_topk_prob: bool = True, gate_temp: float = 1.0,
                 swiglu_limit: float = 0.0, sh_w13: torch.Tensor | None = None, sh_w2: torch.Tensor | None = None,
                 shared_tiled: bool = True):
        experts.check()
        self.ex = experts
        self.n_experts, self.dim, self.inter = experts.E, experts.H, experts.I
        self.topk, self.score_func, self.gate_temp = topk, score_func, float(gate_temp)
        self.norm_topk_prob, self.route_scale, self.swiglu_limit = norm_topk_prob, float(route_scale), float(swiglu_limit)
        self.gate_w = gate_w.to(torch.float32).contiguous()                       # fp32 [E, dim] (model.py:368)
        assert self.gate_w.shape == (self.n_experts, self.dim)
        self.gate_bias = None if gate_bias is None else gate_bias.to(torch.float32).contiguous()
        from .w8 import W8
        self.shared = None
        if isinstance(sh_w13, W8):
            # FP8 shared expert (the checkpoint's format, kept as FP8): inside the decode launches when it fits them, else
            # (and beyond 16 tokens) its own FP8 GEMM launches
            assert isinstance(sh_w2, W8)
            self.sh_w13, self.sh_w2 = sh_w13, sh_w2
            if sh_w13.tiled and sh_w2.tiled:
                self.shared = SharedExpert.prepare_w8(sh_w13, sh_w2)
        else:
            self.sh_w13 = None if sh_w13 is None else sh_w13.to(torch.bfloat16).contiguous()   # [w1; w3] row-major
            self.sh_w2 = None if sh_w2 is None else sh_w2.to(torch.bfloat16).contiguous()
            # the decode kernels stream a bf16 shared expert in the tile_bf16 layout (repacked once)
            if self.sh_w13 is not None:
                self.shared = SharedExpert.prepare(self.sh_w13, self.sh_w2, tiled=shared_tiled)
        self._bufs: dict = {}
        self.last_routing = None

    def _norm(self) -> bool:
        return self.norm_topk_prob and self.topk > 1

    def gate(self, x: torch.Tensor):
        """(weights fp32 [T, topk], indices int32 [T, topk]) as model.MoE.gate (model.py:391-404)."""
        from .fused2 import gate_topk
        T = x.shape[0]
        if T <= 16:
            scores = router_logits_f32w(x.to(torch.bfloat16).contiguous(), self.gate_w)
        else:
            scores = torch.nn.functional.linear(x.float(), self.gate_w)
        eid, wt = gate_topk(scores, self.gate_bias, self.gate_temp, self.topk, self.route_scale, self.score_func, self._norm(),
                            eid=torch.empty(T, self.topk, dtype=torch.int32, device=x.device),
                            wt=torch.empty(T, self.topk, dtype=torch.float32, device=x.device))
        return wt, eid

    def shared_expert(self, x: torch.Tensor) -> torch.Tensor:
        """fp32 [T, dim] = linear_w(swiglu_quant(linear_fp8(x, sh_w13)), sh_w2) (model.py:409-412)."""
        from .quant import fake_quant_fp8
        xq = fake_quant_fp8(x.to(torch.bfloat16))
        if x.shape[0] <= 16 and self.shared is not None and not self.shared.fp8:
            return shared_expert(xq.contiguous(), self.shared.w13, self.shared.w2, self.swiglu_limit, tiled=self.shared.tiled).float()
        return self._shared_rows(xq).float()

    def _shared_rows(self, xq: torch.Tensor) -> torch.Tensor:
        return shared_expert_rows(xq, self.sh_w13, self.sh_w2, self.inter, self.swiglu_limit)

    def _buf(self, dev, T):
        b = self._bufs.get(T)
        if b is None:
            H, E, k = self.dim, self.n_experts, self.topk
            b = self._bufs[T] = {"xq": torch.empty(T, H, dtype=torch.bfloat16, device=dev), "out": torch.empty(T, H, dtype=torch.bfloat16, device=dev),
                                 "part": torch.empty(H // 1024, T, E, dtype=torch.float32, device=dev),
                                 "eid": torch.empty(T, k, dtype=torch.int32, device=dev), "wt": torch.empty(T, k, dtype=torch.float32, device=dev)}
        return b

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.size()
        x2 = x.reshape(-1, self.dim)
        if x2.dtype != torch.bfloat16 or not x2.is_contiguous():
            x2 = x2.to(torch.bfloat16).contiguous()
        dev = _lib.require_cuda(x2)
        T, H = x2.shape
        if T <= 16:
            b = self._buf(dev, T)
            _lib.call("dsv41_quant_fp8", _lib.ptr(x2), 0, T, H, x2.stride(0), 0, None, None, _lib.ptr(b["xq"]), _lib.stream(dev))
            router_logits_f32w(x2, self.gate_w, part=b["part"])
            ys = self._shared_rows(b["xq"]) if self.shared is None and self.sh_w13 is not None else None
            moe_route_experts(b["xq"], b["part"], self.gate_bias, self.gate_temp, self.topk, self.route_scale, self.score_func, self._norm(),
                              self.ex, self.swiglu_limit, ys=ys, out=b["out"], eid_out=b["eid"], wt_out=b["wt"], shared=self.shared)
            self.last_routing = (b["eid"], b["wt"])
            return b["out"].view(shape)
        from .quant import fake_quant_fp8
        wt, eid = self.gate(x2)
        xq = fake_quant_fp8(x2)
        ys = self._shared_rows(xq) if self.sh_w13 is not None else None
        out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        prefill_experts(xq, eid, wt, self.ex, self.swiglu_limit, ys=ys, out=out)
        self.last_routing = (eid, wt)
        return out.view(shape)
