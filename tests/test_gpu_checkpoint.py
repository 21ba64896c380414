"""Checkpoint ingest at the reference model's own expert shapes (DeepSeek-V4.1: hidden 5120, intermediate 2304, top-6):
a synthetic sharded safetensors checkpoint in the on-disk format (I8 packed E2M1 experts with F8_E8M0 scales, an FP8
E4M3 shared expert with 32 x 32 E8M0 block scales, an fp32 router with bias) is loaded by dsv41_amd.load (the
reference's load_layer, load.py:63-149) and run through decode (one and three tokens) and prefill (40 tokens), against
the oracle on the raw bytes."""
import numpy as np
import pytest
import torch

from _safetensors import write_checkpoint
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _fp8_weight(rng, n, k):
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x10          # no NaN codes
    codes[(codes & 0x78) >= 0x60] &= 0xA7         # keep magnitudes moderate (exponent field < 12)
    scale = rng.integers(118, 122, ((n + 31) // 32, (k + 31) // 32), dtype=np.uint8)
    return codes, scale


def test_v41_checkpoint_moe_layer(tmp_path):
    from dsv41_amd import load, stio
    rng = np.random.default_rng(41)
    E, H, I, k = 12, 5120, 2304, 6
    t = {}
    raw = {"w1": [], "w3": [], "s1": [], "s3": [], "w2": [], "s2": []}
    for e in range(E):
        q = f"layers.3.ffn.experts.{e}."
        for name, (n, kk) in {"w1": (I, H), "w3": (I, H), "w2": (H, I)}.items():
            w = rng.integers(0, 256, (n, kk // 2), dtype=np.uint8)
            s = rng.integers(119, 124, (n, kk // 32), dtype=np.uint8)
            t[q + name + ".weight"] = ("I8", w.shape, w)
            t[q + name + ".scale"] = ("F8_E8M0", s.shape, s)
            raw[name].append(w)
            raw["s" + name[1]].append(s)
    sh = {}
    for name, (n, kk) in {"w1": (I, H), "w3": (I, H), "w2": (H, I)}.items():
        c, s = _fp8_weight(rng, n, kk)
        t[f"layers.3.ffn.shared_experts.{name}.weight"] = ("F8_E4M3", c.shape, c)
        t[f"layers.3.ffn.shared_experts.{name}.scale"] = ("F8_E8M0", s.shape, s)
        sh[name] = (c, s)
    gate_w = (rng.standard_normal((E, H)) / np.sqrt(H)).astype(np.float32)
    gate_b = (rng.standard_normal(E) * 0.05).astype(np.float32)
    t["layers.3.ffn.gate.weight"] = ("F32", gate_w.shape, gate_w)
    t["layers.3.ffn.gate.bias"] = ("F32", gate_b.shape, gate_b)
    cfg = {"n_routed_experts": E, "n_activated_experts": k, "score_func": "sqrtsoftplus", "route_scale": 2.5, "swiglu_limit": 10.0}
    write_checkpoint(str(tmp_path), t, n_files=3, config=cfg)

    ck = stio.Checkpoint(str(tmp_path))
    layer = load.load_moe(ck, 3, DEV)
    assert layer.topk == k and layer.ex.tiled and layer.ex.E == E and layer.inter == I
    W13 = np.stack([np.concatenate([raw["w1"][e], raw["w3"][e]]) for e in range(E)])
    S13 = np.stack([np.concatenate([raw["s1"][e], raw["s3"][e]]) for e in range(E)])
    W2, S2 = np.stack(raw["w2"]), np.stack(raw["s2"])
    deq = lambda c, s, n, kk: O.e4m3_decode(c) * np.repeat(np.repeat(O.e8m0_to_f32(s), 32, 0)[:n], 32, 1)[:, :kk]
    Ws13 = O.f32_to_bf16_bits(np.concatenate([deq(*sh["w1"], I, H), deq(*sh["w3"], I, H)]).astype(np.float32))
    Ws2 = O.f32_to_bf16_bits(deq(*sh["w2"], H, I).astype(np.float32))
    from dsv41_amd import w8
    assert isinstance(layer.sh_w13, w8.W8) and isinstance(layer.sh_w2, w8.W8), "FP8 shared expert is kept as FP8"
    assert np.array_equal(layer.sh_w13.bf16().view(torch.int16).cpu().numpy().view(np.uint16), Ws13)
    assert np.array_equal(layer.sh_w2.bf16().view(torch.int16).cpu().numpy().view(np.uint16), Ws2)
    for T in (1, 3, 40):
        x = torch.from_numpy((rng.standard_normal((T, H)) * 2).astype(np.float32)).to(torch.bfloat16).to(DEV)
        y = layer(x).clone()
        eid, wt = [a.cpu().numpy() for a in layer.last_routing]
        xv = O.bf16_bits_to_f32(x.view(torch.int16).cpu().numpy().view(np.uint16))
        logits = (xv.astype(np.float64) @ gate_w.astype(np.float64).T).astype(np.float32)
        ref_i, ref_w = O.gate_topk(logits, gate_b, 1.0, k, 2.5, "sqrtsoftplus", True)
        assert np.array_equal(eid, ref_i), f"T={T}: routing differs"
        assert np.allclose(wt, ref_w, rtol=1e-4, atol=1e-6)
        ref = O.moe_layer(xv, eid, wt, W13, S13, W2, S2, Ws13, Ws2, I, 10.0)
        got = O.bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16))
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        print(f"V4.1 checkpoint layer T={T}: rel L2 {O.rel_l2(got, ref):.2e}")
        assert O.rel_l2(got, ref) <= 2e-3
        assert np.all(np.abs(got - ref) <= 1e-2 * rms + np.abs(ref) * 2.0 ** -7)
