"""MI355X-native FP4 MoE expert path (DeepSeek-V4.1 expert compute) on hand-written gfx950 HIP kernels.

Modules mirror the reference's call surface for expert compute:
  quant        formats: dequant_fp4 (bit-exact), fake_quant_fp8 / quant_fp8, tile_fp4 layout   (dsv41/quant.py)
  hipkern      fp4_gemv_pairs, fp4_gemm_tc, permute_x, moe_dispatch                         (dsv41/cukern.py)
  fused        fake_quant_fp8, swiglu_quant                                                  (dsv41/fused.py)
  fused2       gate_topk                                                                     (dsv41/fused2.py)
  moe_kernels  GroupedPairs, grouped_fp4_gemm                                                (dsv41/moe_kernels.py)
  moe          MoE layer class, fused decode experts, shared expert, MoEDecodeLayer          (model.MoE / decode.moe2)
  w8           W8, linear_w, linear_fp8, oproj_a (FP8 dense weights)                         (dsv41/w8.py, model.py:55-58)
  stio, load   checkpoint reader, expert / shared-expert / layer loading                     (dsv41/stio.py, load.py)
  offload      OffloadMoE, HotCache, OffloadDecodeRuntime (single-GPU expert offload)         (model.py:455-552, hotcache.py)
  cpumoe       the host expert library's binding                                            (dsv41/cpumoe.py)
"""
from . import _lib  # noqa: F401

__all__ = ["quant", "hipkern", "fused", "fused2", "moe_kernels", "moe", "w8", "stio", "load", "offload", "cpumoe"]
