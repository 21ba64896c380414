"""Expert ingest from a checkpoint (the expert part of the reference's load.load_layer, load.py:63-149): per layer,
the routed experts' w1 / w3 / w2 packed E2M1 weights (I8) and E8M0 scales (F8_E8M0) under
layers.{i}.ffn.experts.{e}.w{1,2,3}.{weight,scale} are stacked as w13 = [w1; w3] along N (load.py:128-148) and
repacked into the tile_fp4 layout on the GPU (load.py:145-147); the router (ffn.gate.weight / .bias) and the shared
expert (ffn.shared_experts.w{1,2,3}.weight: bf16, or FP8 E4M3 with per-32x32 E8M0 block scales, kept as FP8 w8.W8 on
the GPU or dequantised to bf16 as quant.dequant_fp8_block does, quant.py:90-95) complete a MoE layer.
"""
from __future__ import annotations

import torch

from .moe import MoE, ExpertWeights, SharedExpert
from .quant import tile_fp4, tile_fp4_scales
from .stio import Checkpoint


def _prefix(layer: int, prefix: str | None) -> str:
    return prefix if prefix is not None else f"layers.{layer}."


def load_experts(ckpt: Checkpoint, layer: int, device, tiled: bool = True, prefix: str | None = None) -> ExpertWeights:
    """The layer's routed experts on `device`: w13 uint8 [E, 2I, H/2], s13 [E, 2I, H/32], w2 [E, H, I/2], s2 [E, H, I/32]
    (experts in id order), in the tile_fp4 layout when `tiled`. Each expert's six tensors are copied from the mapped
    file straight into their rows of the stacked buffers."""
    p = _prefix(layer, prefix) + "ffn.experts."
    ids = sorted({int(n[len(p):].split(".")[0]) for n in ckpt.names(p)})
    if not ids or ids != list(range(len(ids))):
        raise ValueError(f"{p}*: expert ids must be 0 .. E-1, found {ids[:4]}..")
    E = len(ids)
    inter, hh = ckpt.meta(p + "0.w1.weight")[1]
    H = ckpt.meta(p + "0.w2.weight")[1][0]
    u8 = lambda *shape: torch.empty(*shape, dtype=torch.uint8, device=device)
    w13, s13, w2, s2 = u8(E, 2 * inter, hh), u8(E, 2 * inter, H // 32), u8(E, H, inter // 2), u8(E, H, inter // 32)
    for e in ids:
        q = f"{p}{e}."
        get = lambda k: ckpt.get(q + k).view(torch.uint8)
        w13[e, :inter].copy_(get("w1.weight"))
        w13[e, inter:].copy_(get("w3.weight"))
        s13[e, :inter].copy_(get("w1.scale"))
        s13[e, inter:].copy_(get("w3.scale"))
        w2[e].copy_(get("w2.weight"))
        s2[e].copy_(get("w2.scale"))
    if tiled:
        w13, s13, w2, s2 = tile_fp4(w13), tile_fp4_scales(s13), tile_fp4(w2), tile_fp4_scales(s2)
    ex = ExpertWeights(w13, s13, w2, s2, tiled=tiled)
    if w13.is_cuda:
        ex.check()
    return ex


def dequant_fp8_block(w: torch.Tensor, scale: torch.Tensor, block: int = 32) -> torch.Tensor:
    """float8_e4m3fn [N, K] with E8M0 block scales [ceil(N/32), ceil(K/32)] -> bf16 [N, K] (quant.py:90-95): the HIP
    kernel on the GPU; on the host each weight gathers its block's scale value and the fp32 product is cast."""
    from . import quant
    if w.is_cuda:
        return quant.dequant_fp8_block(w, scale, block)
    n, k = w.shape
    blk_r = torch.arange(n, device=w.device) // block
    blk_c = torch.arange(k, device=w.device) // block
    sv = quant.e8m0_to_float(scale)[blk_r[:, None], blk_c[None, :]]
    return (w.view(torch.float8_e4m3fn).float() * sv).to(torch.bfloat16)


def _dense_bf16(ckpt: Checkpoint, name: str, device) -> torch.Tensor:
    dtype, _ = ckpt.meta(name)
    w = ckpt.get(name, device)
    if dtype == "F8_E4M3":
        return dequant_fp8_block(w, ckpt.get(name.replace(".weight", ".scale"), device))
    return w.to(torch.bfloat16)


def load_shared_expert(ckpt: Checkpoint, layer: int, device, tiled: bool = True, prefix: str | None = None,
                       fp8: bool | None = None) -> tuple:
    """(w13 = [w1; w3] [2I, H], w2 [H, I]) of the layer's shared expert (model.py:385-387). FP8 E4M3 checkpoint
    weights stay FP8 on the GPU as w8.W8 (load.py:55-58 of the reference keeps W8 when enabled) unless fp8 is False;
    bf16 weights, or FP8 ones on the host, come back as bf16 row-major tensors."""
    from . import w8
    p = _prefix(layer, prefix) + "ffn.shared_experts."
    names = [p + f"{k}.weight" for k in ("w1", "w3", "w2")]
    keep = (w8.ENABLED if fp8 is None else fp8) and torch.device(device).type == "cuda"
    if keep and all(ckpt.meta(n)[0] == "F8_E4M3" for n in names):
        W = [w8.W8(ckpt.get(n, device).view(torch.uint8), ckpt.get(n.replace(".weight", ".scale"), device).view(torch.uint8))
             for n in names]
        return w8.W8.cat(W[:2]), W[2]
    w1, w3, w2 = (_dense_bf16(ckpt, n, device) for n in names)
    return torch.cat([w1, w3], dim=0).contiguous(), w2.contiguous()


def load_moe(ckpt: Checkpoint, layer: int, device, cfg: dict | None = None, tiled: bool = True, prefix: str | None = None,
             shared_fp8: bool | None = None) -> MoE:
    """One MoE layer (router, routed experts, shared expert) as moe.MoE, with the gate settings from the model config
    (config.json beside the weights, or `cfg`): n_activated_experts, score_func, route_scale, swiglu_limit,
    gate_temp (default 1), norm_topk_prob (default true) (model.py:361-367)."""
    cfg = ckpt.config() if cfg is None else cfg
    p = _prefix(layer, prefix)
    gate_w = ckpt.get(p + "ffn.gate.weight", device).float()
    gate_b = ckpt.get(p + "ffn.gate.bias", device).float() if (p + "ffn.gate.bias") in ckpt else None
    ex = load_experts(ckpt, layer, device, tiled=tiled, prefix=prefix)
    sh_w13 = sh_w2 = None
    if (p + "ffn.shared_experts.w1.weight") in ckpt:
        sh_w13, sh_w2 = load_shared_expert(ckpt, layer, device, prefix=prefix, fp8=shared_fp8)
    return MoE(ex, gate_w, gate_b, topk=int(cfg["n_activated_experts"]), score_func=cfg.get("score_func", "softmax"),
               route_scale=float(cfg.get("route_scale", 1.0)), norm_topk_prob=bool(cfg.get("norm_topk_prob", True)),
               gate_temp=float(cfg.get("gate_temp", 1.0)), swiglu_limit=float(cfg.get("swiglu_limit", 0.0)), sh_w13=sh_w13, sh_w2=sh_w2)
