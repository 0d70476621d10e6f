"""GPU: the per-(b, h) e4m3 quantiser is bit-exact against the CPU restatement.

``oracle/fp8.py`` is itself pinned to torch's float8_e4m3fn cast on the CPU
(test_oracle_numerics.py); here the kernel's bytes and scales must equal it
exactly, on plain, strided, outlier, all-zero and saturating inputs, and after
the fused Hadamard + absmax pass that config 4's fp8 run uses.
"""
import numpy as np
import pytest
import torch

from kerneldev_amd import generate_hadamard_signs
from kerneldev_amd.hadamard import _absmax_op, hadamard_absmax, quantize_fp8
from kerneldev_amd.synth import config_inputs
from oracle import fp8 as ref_fp8
from oracle import hadamard as ref_h

pytestmark = pytest.mark.gpu


def _check(x_cpu, got8, got_scale, amax=None):
    x = x_cpu.float().numpy()
    if amax is None:
        want8, want_scale = ref_fp8.quantize_per_head(x)
    else:  # a caller-given amax (smaller than max |x| saturates at +-448)
        safe = np.where(amax > 0, amax, np.float32(448)).astype(np.float32)
        inv = (np.float32(448) / safe).astype(np.float32)
        y = np.clip((x * inv[:, :, None, None]).astype(np.float32), -448, 448).astype(np.float32)
        want8, want_scale = ref_fp8.e4m3_encode(y), (safe / np.float32(448)).astype(np.float32)
    g8 = got8.cpu().numpy()
    bad = int((g8 != want8).sum())
    assert bad == 0, f"{bad} of {g8.size} e4m3 bytes differ"
    assert np.array_equal(got_scale.cpu().numpy(), want_scale)


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_absmax_exact(dev, D, dtype):
    """kd_absmax (quantize_fp8's default amax) equals torch's max |x| per (b, h) exactly,
    on ragged T, an all-zero head, a negative outlier, and a strided [B, T, H, d] view."""
    print(f"absmax D={D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(D + 7)
    x = torch.randn(3, 4, 1037, D, generator=g).to(dtype)
    x[0, 1] = 0
    x[2, 3, 1000, D - 1] = -300.0
    got = _absmax_op(x.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), x.float().abs().amax(dim=(2, 3)))
    base = torch.randn(2, 333, 3, D, generator=g).to(dtype)
    view = base.to(dev).transpose(1, 2)
    got = _absmax_op(view)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), base.transpose(1, 2).float().abs().amax(dim=(2, 3)))


@pytest.mark.parametrize("B,H,T,D", [(32, 64, 64, 128), (8, 100, 300, 256), (1, 3, 70000, 32), (2, 8, 4096, 256)])
def test_absmax_split_over_workgroups(dev, B, H, T, D):
    """kd_absmax splits each (b, h) over up to 256 / (B H) workgroups that stride over
    it and fold their maxima atomically: many heads (one workgroup each, several strides),
    a long head (69 workgroups) and 16 heads of 16 workgroups, two strides each.  Outliers sit in the last chunk,
    on stride boundaries and in every head's last row; one head is all zeros."""
    print(f"absmax split B={B} H={H} T={T} D={D}", flush=True)
    g = torch.Generator(device=dev).manual_seed(B * H + T)
    x = torch.randn(B, H, T, D, generator=g, device=dev).to(torch.bfloat16)
    x[-1, -1, -1, -1] = -4096.0
    flat = x.view(B * H, -1)
    for j, pos in enumerate((256 * 8 - 1, 512 * 8, 1024 * 8 + 3)):
        if pos < flat.shape[1]:
            flat[j % (B * H), pos] = 77.0 + j
    x[:, :, -1, 0] = 50.0
    x[0, 0] = 0
    got = _absmax_op(x)
    torch.cuda.synchronize()
    assert torch.equal(got, x.float().abs().amax(dim=(2, 3)))


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quantize_bit_exact(dev, D, dtype):
    print(f"fp8 quantiser D={D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(D + 1)
    x = (torch.randn(2, 3, 129, D, generator=g) * 2).to(dtype)
    x[0, 2, :, 7] *= 30       # outlier channel
    x[1, 1] = 0               # all-zero head: scale 1, bytes 0
    x[1, 0, 5, :4] = torch.tensor([1e-4, -3e-3, 2.0 ** -10, -(2.0 ** -9)]).to(dtype)  # subnormal range
    x8, scale = quantize_fp8(x.to(dev))
    torch.cuda.synchronize()
    _check(x, x8, scale)


def test_quantize_strided_and_saturating(dev):
    B, L, H, D = 2, 70, 4, 128
    g = torch.Generator().manual_seed(5)
    base = torch.randn(B, L, H, D, generator=g).to(torch.bfloat16)
    view = base.to(dev).transpose(1, 2)  # [B, H, L, D] with model-layout strides
    amax = (view.float().abs().amax(dim=(2, 3)) * 0.5).contiguous()  # half of max |x|: clamps
    x8, scale = quantize_fp8(view, amax)
    torch.cuda.synchronize()
    _check(base.transpose(1, 2), x8, scale, amax.cpu().numpy())
    assert (x8.cpu() & 0x7F).max().item() == 0x7E  # saturated to +-448


def test_hadamard_then_quantize_config4_heads(dev):
    """Config 4's fp8 operands: Q' = bf16(Q R) with its fused absmax, then e4m3."""
    inp = config_inputs(4, seed=0)
    signs = generate_hadamard_signs(128, seed=0)
    q = inp["q"][:, :4].contiguous()  # 2 x 4 heads of the 8192 x 128 config-4 Q
    qr, amax = hadamard_absmax(q.to(dev), signs.to(dev))
    x8, scale = quantize_fp8(qr, amax)
    torch.cuda.synchronize()
    want_r = torch.from_numpy(ref_h.rotate_fp32(q.float().numpy(), signs.numpy())).to(torch.bfloat16)
    assert torch.equal(qr.cpu().view(torch.int16), want_r.view(torch.int16))
    _check(want_r, x8, scale)
