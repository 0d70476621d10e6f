"""GPU: the Hadamard rotation kernel is bit-exact against the CPU restatement,
and attention with ``hadamard=True`` matches the un-rotated dense reference.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_fwd_bwd, oracle_mask, select_heads
from kerneldev_amd import flash_attention, generate_hadamard_signs, hadamard_transform
from kerneldev_amd.hadamard import hadamard_absmax
from kerneldev_amd.synth import CONFIG3_LAYOUT, cocktail_batch, config_inputs, qkvdo
from oracle import hadamard as ref_h

pytestmark = pytest.mark.gpu


def _expected(x_cpu, signs, inverse):
    x = x_cpu.float().numpy()
    y = ref_h.unrotate_fp32(x, signs.numpy()) if inverse else ref_h.rotate_fp32(x, signs.numpy())
    return torch.from_numpy(y).to(x_cpu.dtype)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("inverse", [False, True])
def test_rotation_bit_exact(dev, D, dtype, inverse):
    print(f"hadamard D={D} {dtype} inverse={inverse}", flush=True)
    g = torch.Generator().manual_seed(D)
    x = (torch.randn(2, 3, 77, D, generator=g) * 3).to(dtype)
    x[0, 1, :, 5] *= 20  # outlier channel
    signs = generate_hadamard_signs(D, seed=7)
    y = hadamard_transform(x.to(dev), signs.to(dev), inverse=inverse)
    torch.cuda.synchronize()
    want = _expected(x, signs, inverse)
    assert torch.equal(y.cpu().view(torch.int16), want.view(torch.int16))


def test_rotation_strided_input_and_absmax(dev):
    B, L, H, D = 2, 50, 4, 128
    g = torch.Generator().manual_seed(3)
    base = torch.randn(B, L, H, D, generator=g).to(torch.bfloat16)
    signs = generate_hadamard_signs(D, seed=1)
    y, amax = hadamard_absmax(base.to(dev).transpose(1, 2), signs.to(dev))
    torch.cuda.synchronize()
    want = _expected(base.transpose(1, 2), signs, False)
    assert torch.equal(y.cpu().view(torch.int16), want.view(torch.int16))
    assert torch.equal(amax.cpu(), want.float().abs().amax(dim=(2, 3)))


def test_rotation_roundtrip_and_gradient(dev):
    D = 128
    signs = generate_hadamard_signs(D, seed=2).to(dev)
    x = torch.randn(1, 2, 64, D, device=dev, dtype=torch.bfloat16, requires_grad=True)
    y = hadamard_transform(x, signs)
    gy = torch.randn_like(y)
    y.backward(gy)
    torch.cuda.synchronize()
    # x R R^T = x up to bf16 rounding; the gradient is gy R^T
    back = hadamard_transform(y.detach(), signs, inverse=True)
    assert (back.float() - x.detach().float()).abs().max().item() < 3e-2
    assert torch.equal(x.grad, hadamard_transform(gy, signs, inverse=True))


def test_attention_with_hadamard_matches_unrotated_reference(dev):
    print("attention hadamard cocktail", flush=True)
    tokens, in_span, span_id, is_prefix = cocktail_batch(2, 512, CONFIG3_LAYOUT, seed=12)
    q, k, v, do = qkvdo(2, 2, 512, 128, seed=13)
    qd, kd, vd = (x.to(dev).requires_grad_(True) for x in (q, k, v))
    o = flash_attention(qd, kd, vd, in_span=in_span.to(dev), span_id=span_id.to(dev), is_prefix=is_prefix.to(dev),
                        hadamard=True, hadamard_seed=5)
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    inp = dict(q=q, in_span=in_span, span_id=span_id, is_prefix=is_prefix)
    ref = oracle_fwd_bwd(q, k, v, do, oracle_mask(inp, 512), 128 ** -0.5)
    assert_close("o", o, ref["o"])
    assert_close("dq", qd.grad, ref["dq"])
    assert_close("dk", kd.grad, ref["dk"])
    assert_close("dv", vd.grad, ref["dv"])
