"""Host-side weight layouts (CPU, torch): the bf16 tile layout of the shared expert is a permutation with the
documented index formula, and untile inverts it."""
import torch

from dsv41_amd import quant


def test_tile_bf16_index_formula_and_round_trip():
    N, K = 48, 96
    w = torch.arange(N * K, dtype=torch.float32).reshape(N, K).to(torch.bfloat16)   # exact up to 256: use the bits below
    bits = torch.arange(N * K, dtype=torch.int32).reshape(N, K).to(torch.int16).view(torch.bfloat16)
    t = quant.tile_bf16(bits)
    flat = t.view(torch.int16).reshape(-1)
    src = bits.view(torch.int16)
    # element (n, k) sits in tile (n / 16, k / 32) at row n % 16, column k % 32
    for n, k in [(0, 0), (5, 31), (16, 32), (47, 95), (20, 70)]:
        off = ((n // 16) * (K // 32) + k // 32) * 512 + (n % 16) * 32 + k % 32
        assert flat[off] == src[n, k]
    assert torch.equal(quant.untile_bf16(t).view(torch.int16), src)
    assert torch.equal(quant.untile_bf16(quant.tile_bf16(w)), w)


def test_attached_codes_follow_the_tensor_version():
    """The FP8 operand recorded on a tensor (quant.attach_codes) is returned for the recorded k order only, and is
    dropped by any in-place change of the tensor, through itself or through a view; views and copies carry none."""
    x = torch.randn(4, 64).to(torch.bfloat16)
    codes = torch.zeros(4, 64, dtype=torch.uint8)
    scales = torch.zeros(4, 2, dtype=torch.uint8)
    assert quant.attached_codes(x, False) is None
    quant.attach_codes(x, codes, scales, permuted=True)
    got = quant.attached_codes(x, True)
    assert got is not None and got[0] is codes and got[1] is scales
    assert quant.attached_codes(x, False) is None
    assert quant.attached_codes(x[1:], True) is None and quant.attached_codes(x.clone(), True) is None
    x[1:].mul_(2)
    assert quant.attached_codes(x, True) is None
    quant.attach_codes(x, codes, scales)
    assert quant.attached_codes(x, False) is not None
    x.add_(1)
    assert quant.attached_codes(x, False) is None
    # a set_ onto other storage, or a resize, drops it too
    quant.attach_codes(x, codes, scales)
    x.set_(torch.randn(4, 64).to(torch.bfloat16))
    assert quant.attached_codes(x, False) is None
    quant.attach_codes(x, codes, scales)
    x.resize_(2, 128)
    assert quant.attached_codes(x, False) is None


def test_inference_tensors_carry_no_record():
    """Tensors made in inference mode keep no version counter: attach_codes leaves them unrecorded (the surfaces then
    quantise them as any input) instead of failing."""
    codes = torch.zeros(2, 64, dtype=torch.uint8)
    scales = torch.zeros(2, 2, dtype=torch.uint8)
    with torch.inference_mode():
        x = torch.randn(2, 64).to(torch.bfloat16)
        assert quant.attach_codes(x, codes, scales) is x
        assert quant.attached_codes(x, False) is None
    assert quant.attached_codes(x, False) is None
