"""Walsh-Hadamard incoherent processing of Q and K.

The reference's README names ``generate_hadamard_signs()`` and
``hadamard_transform()`` (README.md:68-71, :77) but ships no code for them.
Here they are defined as the rotation ``R = diag(s) H_d / sqrt(d)`` (Sylvester
``H_d``, seeded signs ``s``), applied to the last dimension of a
``[B, H, T, d]`` tensor by the gfx950 kernel ``kd_hadamard``.  Because ``R``
is orthogonal, ``(Q R)(K R)^T = Q K^T``: rotating both operands leaves the
attention scores unchanged in exact arithmetic while spreading outlier
channels over all ``d`` lanes (which is what makes per-head fp8 scaling
usable).  The autograd rule of ``y = x R`` is ``dx = dy R^T``, the same kernel
with ``inverse=1``.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import QuantArgs, RotArgs


def generate_hadamard_signs(d: int, seed: int | None = None, device=None) -> torch.Tensor:
    """Seeded random signs ``s in {+1, -1}^d`` as float32 (seed ``None`` -> 0)."""
    if d <= 0 or d & (d - 1):
        raise ValueError(f"d must be a power of two, got {d}")
    g = torch.Generator("cpu").manual_seed(0 if seed is None else int(seed))
    s = torch.randint(0, 2, (d,), generator=g, dtype=torch.int64).to(torch.float32) * 2 - 1
    return s if device is None else s.to(device)


def _strides3(t):
    st = t.stride()
    return (ctypes.c_int64 * 3)(st[0], st[1], st[2])


def _launch(x: torch.Tensor, signs: torch.Tensor, inverse: bool, amax: torch.Tensor | None = None):
    from .attention import _dtype_code, _kernel_ready

    x = _kernel_ready(x)
    B, H, T, D = x.shape
    y = torch.empty((B, H, T, D), dtype=x.dtype, device=x.device)
    a = RotArgs()
    a.x, a.x_strides = x.data_ptr(), _strides3(x)
    a.y, a.y_strides = y.data_ptr(), _strides3(y)
    a.signs = signs.data_ptr()
    a.amax = amax.data_ptr() if amax is not None else None
    a.B, a.H, a.T, a.D = B, H, T, D
    a.dtype = _dtype_code(x.dtype)
    a.inverse = 1 if inverse else 0
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(_lib.load().kd_hadamard(ctypes.byref(a), stream), "kd_hadamard")
    return y


@torch.library.custom_op("kdattn::rot", mutates_args=(), device_types=("cuda",))
def _rot_op(x: torch.Tensor, signs: torch.Tensor, inverse: bool) -> torch.Tensor:
    return _launch(x, signs, inverse)


@_rot_op.register_fake
def _rot_fake(x, signs, inverse):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _rot_setup(ctx, inputs, output):
    _, signs, inverse = inputs
    ctx.save_for_backward(signs)
    ctx.inverse = inverse


def _rot_backward(ctx, gy):
    (signs,) = ctx.saved_tensors
    return _rot_op(gy.contiguous(), signs, not ctx.inverse), None, None


_rot_op.register_autograd(_rot_backward, setup_context=_rot_setup)


@torch.library.custom_op("kdattn::rot_amax", mutates_args=(), device_types=("cuda",))
def _rot_amax_op(x: torch.Tensor, signs: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    amax = torch.zeros(x.shape[:2], dtype=torch.float32, device=x.device)
    return _launch(x, signs, False, amax), amax


@_rot_amax_op.register_fake
def _rot_amax_fake(x, signs):
    return (torch.empty(x.shape, dtype=x.dtype, device=x.device),
            torch.empty(x.shape[:2], dtype=torch.float32, device=x.device))


def _rot_amax_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1])
    ctx.inverse = False
    # amax only feeds the fp8 scales, which are not differentiated
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)


def _rot_amax_backward(ctx, gy, gamax):
    if gy is None:  # x R did not reach the loss
        return None, None
    (signs,) = ctx.saved_tensors
    return _rot_op(gy.contiguous(), signs, True), None


_rot_amax_op.register_autograd(_rot_amax_backward, setup_context=_rot_amax_setup)


def _quant_launch(x: torch.Tensor, amax: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """kd_quant_fp8 of a kernel-ready bf16 / fp16 [B, H, T, d] tensor with its fp32 [B, H] amax."""
    from .attention import _dtype_code

    B, H, T, D = x.shape
    y = torch.empty((B, H, T, D), dtype=torch.uint8, device=x.device)
    scale = torch.empty((B, H), dtype=torch.float32, device=x.device)
    amax = amax.contiguous()
    a = QuantArgs()
    a.x, a.x_strides = x.data_ptr(), _strides3(x)
    a.y, a.amax, a.scale = y.data_ptr(), amax.data_ptr(), scale.data_ptr()
    a.B, a.H, a.T, a.D = B, H, T, D
    a.dtype = _dtype_code(x.dtype)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(_lib.load().kd_quant_fp8(ctypes.byref(a), stream), "kd_quant_fp8")
    return y, scale


@torch.library.custom_op("kdattn::quant", mutates_args=(), device_types=("cuda",))
def _quant_op(x: torch.Tensor, amax: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    from .attention import _kernel_ready

    return _quant_launch(_kernel_ready(x), amax)


@_quant_op.register_fake
def _quant_fake(x, amax):
    return (torch.empty(x.shape, dtype=torch.uint8, device=x.device),
            torch.empty(x.shape[:2], dtype=torch.float32, device=x.device))


def _absmax_launch(x: torch.Tensor, amax: torch.Tensor) -> torch.Tensor:
    """kd_absmax of a kernel-ready bf16 / fp16 [B, H, T, d] tensor into the contiguous fp32 [B, H] amax."""
    from .attention import _dtype_code

    B, H, T, D = x.shape
    a = QuantArgs()
    a.x, a.x_strides = x.data_ptr(), _strides3(x)
    a.B, a.H, a.T, a.D = B, H, T, D
    a.dtype = _dtype_code(x.dtype)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    _lib.check(_lib.load().kd_absmax(ctypes.byref(a), ctypes.c_void_p(amax.data_ptr()), stream), "kd_absmax")
    return amax


@torch.library.custom_op("kdattn::absmax", mutates_args=(), device_types=("cuda",))
def _absmax_op(x: torch.Tensor) -> torch.Tensor:
    """max |x| per (b, h) of a bf16 / fp16 [B, H, T, d] tensor (kd_absmax), exact in fp32."""
    from .attention import _kernel_ready

    x = _kernel_ready(x)
    return _absmax_launch(x, torch.empty(x.shape[:2], dtype=torch.float32, device=x.device))


@_absmax_op.register_fake
def _absmax_fake(x):
    return torch.empty(x.shape[:2], dtype=torch.float32, device=x.device)


def _check(x: torch.Tensor, signs: torch.Tensor):
    if x.dim() != 4:
        raise ValueError("x must be [batch, heads, time, head_dim]")
    if x.shape[-1] not in (16, 32, 64, 128, 256):
        raise ValueError(f"head_dim must be 16, 32, 64, 128 or 256 for the gfx950 transform, got {x.shape[-1]}")
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"x must be bf16, fp16 or fp32, got {x.dtype}")
    if not x.is_cuda:
        raise ValueError("hadamard_transform runs on the GPU only (no CPU fallback)")
    if signs.shape != (x.shape[-1],) or signs.dtype != torch.float32 or signs.device != x.device:
        raise ValueError("signs must be float32 [head_dim] on x's device")


def hadamard_transform(x: torch.Tensor, signs: torch.Tensor, inverse: bool = False) -> torch.Tensor:
    """``x R`` (or ``x R^T`` with ``inverse``), differentiable, on the last dim."""
    _check(x, signs)
    return _rot_op(x, signs, bool(inverse))


def hadamard_absmax(x: torch.Tensor, signs: torch.Tensor):
    """``(x R, amax)`` with ``amax[b, h] = max |x R|`` over (t, d) of the rounded
    output, from the same pass; differentiable in ``x R`` (amax is not)."""
    _check(x, signs)
    return _rot_amax_op(x, signs)


def quantize_fp8(x: torch.Tensor, amax: torch.Tensor | None = None):
    """Per-(b, h) OCP e4m3 quantisation of a bf16 / fp16 ``[B, H, T, d]`` tensor.

    ``x8 = e4m3(clamp(x * fp32(448 / amax), -448, 448))`` with round to nearest
    even, ``scale = amax / 448`` (``amax == 0``: both factors are 1), so that
    ``x ~= scale * x8``.  ``amax`` defaults to ``max |x|`` per (b, h) (kd_absmax).  Returns
    ``(x8 as uint8 bytes [B, H, T, d], scale fp32 [B, H])``; not differentiable.
    """
    if x.dim() != 4 or x.dtype not in (torch.bfloat16, torch.float16) or not x.is_cuda:
        raise ValueError("x must be a bf16 / fp16 [batch, heads, time, head_dim] GPU tensor")
    if x.shape[-1] not in (64, 128, 256):
        raise ValueError(f"head_dim must be 64, 128 or 256, got {x.shape[-1]}")
    if amax is None:
        amax = _absmax_op(x.detach())
    if amax.shape != x.shape[:2] or amax.dtype != torch.float32 or amax.device != x.device:
        raise ValueError("amax must be float32 [batch, heads] on x's device")
    return _quant_op(x.detach(), amax.detach())
