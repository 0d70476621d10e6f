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


@pytest.mark.parametrize("D", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
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
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(y.cpu().view(bits), want.view(bits))


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
    # the form that also returns the absmax: the same gradient, none through amax
    x2 = x.detach().clone().requires_grad_(True)
    y2, amax = hadamard_absmax(x2, signs)
    assert torch.equal(y2, y.detach()) and not amax.requires_grad
    y2.backward(gy)
    torch.cuda.synchronize()
    assert torch.equal(x2.grad, x.grad)


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


def test_backward_epilogue_rotation_matches_separate_pass(dev):
    """kd_attn_bwd with dqk_signs == kd_attn_bwd, then kd_hadamard(inverse) on dQ', dK'.

    The epilogue rotates the fp32 accumulators and rounds once; the separate
    pass rounds dQ' to bf16 first, so the two differ by bf16 roundings only:
    rel-RMS <= 4e-3 and max-abs <= 2^-6 max|ref|.  dV is untouched (bit-equal).
    """
    import ctypes

    from kerneldev_amd import _lib, hadamard_transform
    from kerneldev_amd.attention import _attn_args, _fwd_op, _ptr, _strides3
    from kerneldev_amd.synth import CONFIG3_LAYOUT, cocktail_batch, qkvdo

    print("epilogue rotation vs separate inverse pass, D = 64 and 128", flush=True)
    for D in (64, 128):
        tokens, in_span, span_id, is_prefix = cocktail_batch(2, 1024, CONFIG3_LAYOUT, seed=31)
        q, k, v, do = (x.to(dev) for x in qkvdo(2, 2, 1024, D, seed=32))
        signs = generate_hadamard_signs(D, 5, device=dev)
        qr, kr = hadamard_transform(q, signs), hadamard_transform(k, signs)
        meta = [x.to(dev) for x in (in_span, span_id, is_prefix)]
        sc = D ** -0.5
        o, lse, plan, o_lo, *_ = _fwd_op(qr, kr, v, None, *meta, sc, 0, True)
        lib = _lib.load()
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        outs = []
        for fused in (False, True):
            dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            delta = torch.empty((2,) + tuple(q.shape[:3]), dtype=torch.float32, device=dev)
            a = _attn_args(qr, kr, v, sc)
            a.o, a.o_strides, a.lse, a.o_lo = o.data_ptr(), _strides3(o), lse.data_ptr(), o_lo.data_ptr()
            a.dout, a.do_strides = do.data_ptr(), _strides3(do)
            a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
            a.dq_strides, a.dk_strides, a.dv_strides = _strides3(dq), _strides3(dk), _strides3(dv)
            a.delta = delta.data_ptr()
            a.dqk_signs = signs.data_ptr() if fused else None
            _lib.check(lib.kd_attn_bwd(ctypes.byref(a), *_lib.plan_ref(plan), stream), "bwd")
            if not fused:
                dq, dk = hadamard_transform(dq, signs, inverse=True), hadamard_transform(dk, signs, inverse=True)
            torch.cuda.synchronize()
            outs.append((dq, dk, dv))
        (dq0, dk0, dv0), (dq1, dk1, dv1) = outs
        assert torch.equal(dv0, dv1)
        for name, x, ref in (("dq", dq1, dq0), ("dk", dk1, dk0)):
            x, ref = x.double(), ref.double()
            diff = (x - ref).abs()
            rr = diff.pow(2).mean().sqrt() / ref.pow(2).mean().sqrt()
            print(f"  D={D} {name}: max_abs={diff.max().item():.3e} rel_rms={rr.item():.3e}", flush=True)
            assert diff.max() <= 2.0 ** -6 * ref.abs().max() and rr <= 4e-3, name


@pytest.mark.parametrize("D", [64, 128])
def test_attention_with_hadamard_fp16_ragged_lens(dev, D):
    """The fused path (rotation inside the attention op, dQ / dK rotated back in
    the backward epilogues) on fp16, a ragged T and lens with padded rows."""
    T = 333
    print(f"attention hadamard fp16 causal T={T} D={D}", flush=True)
    q, k, v, do = (x.to(torch.float16) for x in qkvdo(2, 3, T, D, seed=41))
    lens = torch.tensor([T, 200], dtype=torch.int32)
    qd, kd, vd = (x.to(dev).requires_grad_(True) for x in (q, k, v))
    o = flash_attention(qd, kd, vd, lens=lens.to(dev), causal=True, hadamard=True, hadamard_seed=9)
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    mask = oracle_mask(dict(q=q, causal=True), T, lens=lens)
    ref = oracle_fwd_bwd(q, k, v, do, mask, D ** -0.5)
    assert_close("o", o, ref["o"])
    assert_close("dq", qd.grad, ref["dq"])
    assert_close("dk", kd.grad, ref["dk"])
    assert_close("dv", vd.grad, ref["dv"])
