"""``flash_attention()`` -- the drop-in boundary (original_kernel.py:2096-2168).

Keeps the reference's signature, defaults and return forms, and adds three
optional keyword arguments for the incoherent-processing path.  The work goes
through two torch custom ops in the ``kdattn`` namespace (the reference uses
``flash_attention::forward`` / ``::backward``, :1697, :1806), each a thin
shim over the C ABI of ``libkdattn.so``:

* ``kdattn::fwd``  -> plan (codes, tile map, work lists) + forward kernel,
  returns ``(O, LSE2, plan)``; the plan is saved for the backward.
* ``kdattn::bwd``  -> Delta, dQ and dK/dV kernels from the saved plan.
* ``kdattn::fwd_x3`` / ``kdattn::bwd_x3`` -> the 16-bit kernels for fp32
  inputs at precision "tf32" and head dims 16 and 32, as three bf16 products
  per product (see X3_HEAD_DIMS).  Other fp32 inputs go through ``kdattn::fwd``
  / ``::bwd`` to the fp32 MFMA kernels (every head dim).

There is no CPU or PyTorch fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _lib
from ._lib import AttnArgs, MetaArgs

REFERENCE_HEAD_DIMS = (16, 32, 64, 128, 256)  # original_kernel.py:1720
SUPPORTED_HEAD_DIMS = REFERENCE_HEAD_DIMS
# bf16 / fp16 at these head dims run on the MFMA kernels with the fused
# Hadamard epilogues; 16, 32 and 256 run there without them (16 and 32 on
# the d = 64 kernels, which read the missing columns as zeros).  fp8 scores
# are built at 64, 128 and 256.  fp32
# inputs run on the fp32 MFMA kernels at every head dim (kd_f32w.hip; 16 on
# the d = 32 kernels, which read the missing columns as zeros), except at
# precision "tf32" and head dims 16, 32 (X3_ROUTED_HEAD_DIMS: bf16x3, faster
# there)
MFMA_HEAD_DIMS = (64, 128)
FP8_HEAD_DIMS = (64, 128, 256)  # fp8 e4m3 Q K^T (bf16 inputs; fp32 ones are narrowed to bf16 first)

# precision -> arithmetic of P and dS in the kernels.  The reference rounds P
# to V's dtype for P V (original_kernel.py:566-571) and keeps P and dS in fp32
# for its backward dots, taken as tf32 or ieee (:1331-1333, :1517-1523).
# "tf32" (the default): P and dS as a 16-bit hi + lo pair (~16 significant
# bits, above tf32's 11) in all four products.  "ieee": as a hi + mid + lo
# triple (~24 significant bits, the fp32 the reference's ieee dots take), with
# O's rounding residual kept in fp32 so that the backward's Delta sees the fp32
# O.  "bf16" (an extension) rounds P and dS once to the input type: faster, 8
# significant bits.  fp32 inputs get fp32 arithmetic at "ieee" and "tf32" alike.
PRECISIONS = {"ieee": _lib.KD_PREC_SPLIT3, "tf32": _lib.KD_PREC_SPLIT, "bf16": _lib.KD_PREC_SINGLE}


def _lo_dtype(dtype: torch.dtype, prec: int) -> torch.dtype:
    """dtype of the residual buffers (o_lo, dq_lo, ...): fp32 at KD_PREC_SPLIT3."""
    return torch.float32 if prec == _lib.KD_PREC_SPLIT3 else dtype


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _strides3(t):
    s = t.stride()
    return (ctypes.c_int64 * 3)(s[0], s[1], s[2])


def _kernel_ready(x: torch.Tensor) -> torch.Tensor:
    """Unit d-stride, 16-byte aligned base, 8-element-multiple strides, rows that do not overlap."""
    s = x.stride()
    if (s[3] != 1 or x.data_ptr() % 16 != 0 or any(st % 8 for st in s[:3]) or s[2] < x.shape[3]
            or x.shape[2] * s[2] * x.element_size() >= 2 ** 31):
        x = x.contiguous()
    return x


def _dtype_code(dt) -> int:
    if dt == torch.bfloat16:
        return _lib.KD_BF16
    if dt == torch.float16:
        return _lib.KD_F16
    if dt == torch.float32:
        return _lib.KD_F32
    raise ValueError(f"kernel dtype must be bf16, fp16 or fp32, got {dt}")


def _mode(in_span, span_id, is_prefix, has_attention_mask, causal) -> int:
    # original_kernel.py:401 FAST_PATH_NO_RULES; :512-515 fallbacks
    if in_span is None and span_id is None and is_prefix is None and not has_attention_mask:
        return _lib.KD_MODE_CAUSAL if causal else _lib.KD_MODE_ALL
    return _lib.KD_MODE_FORMULA


def build_plan(B, T, D, device, mode, in_span=None, span_id=None, is_prefix=None, lens=None):
    """Run ``kd_plan_build`` and return the plan as a uint8 device tensor."""
    lib = _lib.load()
    # zero-filled: the build leaves the bit masks of non-PARTIAL tiles and the
    # section padding unwritten, and an op's outputs should not carry stale bytes
    plan = torch.zeros(_lib.plan_bytes(B, T, D), dtype=torch.uint8, device=device)
    m = MetaArgs()
    m.B, m.T, m.D, m.mode = B, T, D, mode
    if in_span is not None:
        m.in_span = in_span.data_ptr()
        m.in_span_strides[0], m.in_span_strides[1] = in_span.stride()
    if is_prefix is not None:
        m.is_prefix = is_prefix.data_ptr()
        m.is_prefix_strides[0], m.is_prefix_strides[1] = is_prefix.stride()
    if span_id is not None:
        m.span_id = span_id.data_ptr()
        m.span_id_strides[0], m.span_id_strides[1] = span_id.stride()
        m.span_id_dtype = _lib.KD_I64 if span_id.dtype == torch.int64 else _lib.KD_I32
    if lens is not None:
        m.lens = lens.data_ptr()
        m.lens_stride = lens.stride(0)
    _lib.check(lib.kd_plan_build(ctypes.byref(m), *_lib.plan_ref(plan), _stream(device)), "kd_plan_build")
    return plan


RULES = {"collate": 0, "fallback": 1, "teacher_forcing": 2}  # KD_RULE_*


class AttentionPlan:
    """The tile plan of one mask, built once and passed to any number of
    ``flash_attention(..., plan=...)`` calls on ``[B, *, T, D]`` operands --
    e.g. every layer of one model forward, which share the tokens' mask."""

    def __init__(self, tensor: torch.Tensor, B: int, T: int, D: int):
        self.tensor, self.B, self.T, self.D = tensor, B, T, D


def build_plan_from_tokens(tokens: torch.Tensor, head_dim: int, rule: str = "collate",
                           lens: torch.Tensor | None = None) -> AttentionPlan:
    """Plan straight from token ids ``[B, T]`` on the device (``kd_plan_build_tokens``).

    The metadata rule is one of ``derive_metadata``'s (``"collate"``,
    ``"fallback"``, ``"teacher_forcing"``); the result equals building the plan
    from ``derive_metadata(tokens, rule)``, with no host sync and no metadata
    tensors.
    """
    if tokens.dim() != 2 or tokens.dtype not in (torch.int64, torch.int32) or not tokens.is_cuda:
        raise ValueError("tokens must be an int64 / int32 [B, T] GPU tensor")
    if rule not in RULES:
        raise ValueError(f"unknown metadata rule {rule!r}")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {SUPPORTED_HEAD_DIMS}")
    if lens is not None and (lens.dtype != torch.int32 or lens.dim() != 1 or lens.shape[0] != tokens.shape[0]):
        raise ValueError("lens must be an int32 tensor of shape [batch]")
    B, T = tokens.shape
    plan = torch.zeros(_lib.plan_bytes(B, T, head_dim), dtype=torch.uint8, device=tokens.device)
    t = _lib.TokenArgs()
    t.tokens = tokens.data_ptr()
    t.tokens_strides[0], t.tokens_strides[1] = tokens.stride()
    t.tokens_dtype = _lib.KD_I64 if tokens.dtype == torch.int64 else _lib.KD_I32
    t.rule = RULES[rule]
    if lens is not None:
        t.lens, t.lens_stride = lens.data_ptr(), lens.stride(0)
    t.B, t.T, t.D = B, T, head_dim
    _lib.check(_lib.load().kd_plan_build_tokens(ctypes.byref(t), *_lib.plan_ref(plan), _stream(tokens.device)),
               "kd_plan_build_tokens")
    return AttentionPlan(plan, B, T, head_dim)


def _attn_args(q, k, v, sm_scale, prec=_lib.KD_PREC_SPLIT) -> AttnArgs:
    a = AttnArgs()
    B, H, T, D = q.shape
    a.B, a.H, a.T, a.D = B, H, T, D
    a.dtype = _dtype_code(q.dtype)
    a.sm_scale = float(sm_scale)
    a.precision = int(prec)
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.q_strides, a.k_strides, a.v_strides = _strides3(q), _strides3(k), _strides3(v)
    return a


# ----------------------------------------------------------------- custom ops
def _new_out(B, H, T, D, q, bthd: bool) -> torch.Tensor:
    """O as [B, H, T, D]: contiguous, or a view of [B, T, H, D] memory (bthd)."""
    if bthd:
        return torch.empty((B, T, H, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    return torch.empty((B, H, T, D), dtype=q.dtype, device=q.device)


def _set_fp8(a: AttnArgs, fp8):
    """Point the kernels at the fp8 copies ``(q8, k8, q_scale, k_scale)``, or not."""
    if fp8 is None:
        return
    q8, k8, qs, ks = fp8
    a.q8, a.k8 = q8.data_ptr(), k8.data_ptr()
    a.q_scale, a.k_scale = qs.data_ptr(), ks.data_ptr()


def _fp8_tuple(q8, k8, q_scale, k_scale):
    parts = (q8, k8, q_scale, k_scale)
    if all(x is None for x in parts):
        return None
    if any(x is None for x in parts):
        raise ValueError("q8, k8, q_scale and k_scale go together")
    return parts


@torch.library.custom_op("kdattn::fwd", mutates_args=(), device_types=("cuda",))
def _fwd_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lens: torch.Tensor | None,
            in_span: torch.Tensor | None, span_id: torch.Tensor | None,
            is_prefix: torch.Tensor | None, sm_scale: float, mode: int, need_lo: bool,
            bthd: bool = False, plan_in: torch.Tensor | None = None, signs: torch.Tensor | None = None,
            quant_fp8: bool = False, prec: int = 0,
            ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                       torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    B, H, T, D = q.shape
    # layouts the kernels take (unit d-stride, aligned, 8-element strides);
    # anything else is copied here, inside the op, where the data is real
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    # a caller's plan is used as is (and not returned: outputs may not alias inputs)
    plan = plan_in if plan_in is not None else build_plan(B, T, D, q.device, mode, in_span, span_id, is_prefix, lens)
    # signs: attention of Q R and K R, returned for the backward (which hands
    # back dQ, dK for q, k themselves).  quant_fp8: the scores come from e4m3
    # copies of the (rotated) Q and K, made here and returned, scaled by the
    # rotation pass's absmax or, without one, by kd_absmax's.  Every unused
    # output is its own empty tensor (outputs may not alias).  (The autograd
    # wrapper's per-call cost grows with the square of the argument count, so
    # the op takes no fp8 tensors of a caller's: it makes them itself.)
    q_r, k_r = q.new_empty(0), k.new_empty(0)
    q8_o, k8_o = q.new_empty(0, dtype=torch.uint8), k.new_empty(0, dtype=torch.uint8)
    qs_o, ks_o = q.new_empty(0, dtype=torch.float32), k.new_empty(0, dtype=torch.float32)
    from .hadamard import _absmax_launch, _launch, _quant_launch
    if signs is not None:
        # (the rotation folds its absmax into amax with atomics: zeroed first)
        amax = torch.zeros((2, B, H), dtype=torch.float32, device=q.device) if quant_fp8 else None
        q = q_r = _launch(q, signs, False, None if amax is None else amax[0])
        k = k_r = _launch(k, signs, False, None if amax is None else amax[1])
    elif quant_fp8:
        amax = torch.empty((2, B, H), dtype=torch.float32, device=q.device)
        _absmax_launch(q, amax[0])
        _absmax_launch(k, amax[1])
    if quant_fp8:
        (q8_o, qs_o), (k8_o, ks_o) = _quant_launch(q, amax[0]), _quant_launch(k, amax[1])
    o = _new_out(B, H, T, D, q, bthd)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    # rounding residual of O, kept for the backward's Delta (see kd_bwd.hip)
    o_lo = torch.empty((B, H, T, D) if need_lo else (0,), dtype=_lo_dtype(q.dtype, prec), device=q.device)
    a = _attn_args(q, k, v, sm_scale, prec)
    _set_fp8(a, (q8_o, k8_o, qs_o, ks_o) if quant_fp8 else None)
    a.o, a.o_strides = o.data_ptr(), _strides3(o)
    a.lse = lse.data_ptr()
    a.o_lo = o_lo.data_ptr() if need_lo else None
    _lib.check(_lib.load().kd_attn_fwd(ctypes.byref(a), *_lib.plan_ref(plan), _stream(q.device)), "kd_attn_fwd")
    return o, lse, (plan if plan_in is None else plan.new_empty(0)), o_lo, q_r, k_r, q8_o, k8_o, qs_o, ks_o


@_fwd_op.register_fake
def _fwd_fake(q, k, v, lens, in_span, span_id, is_prefix, sm_scale, mode, need_lo, bthd=False, plan_in=None,
              signs=None, quant_fp8=False, prec=0):
    B, H, T, D = q.shape
    rot_shape = (B, H, T, D) if signs is not None else (0,)
    q8_shape = (B, H, T, D) if quant_fp8 else (0,)
    sc_shape = (B, H) if quant_fp8 else (0,)
    return (_new_out(B, H, T, D, q, bthd),
            torch.empty((B, H, T), dtype=torch.float32, device=q.device),
            torch.empty(_lib.plan_nbytes(B, T, D) if plan_in is None else 0, dtype=torch.uint8, device=q.device),
            torch.empty((B, H, T, D) if need_lo else (0,), dtype=_lo_dtype(q.dtype, prec), device=q.device),
            torch.empty(rot_shape, dtype=q.dtype, device=q.device),
            torch.empty(rot_shape, dtype=k.dtype, device=k.device),
            torch.empty(q8_shape, dtype=torch.uint8, device=q.device),
            torch.empty(q8_shape, dtype=torch.uint8, device=q.device),
            torch.empty(sc_shape, dtype=torch.float32, device=q.device),
            torch.empty(sc_shape, dtype=torch.float32, device=q.device))


@torch.library.custom_op("kdattn::bwd", mutates_args=(), device_types=("cuda",))
def _bwd_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, lse: torch.Tensor,
            do: torch.Tensor, plan: torch.Tensor, sm_scale: float, o_lo: torch.Tensor,
            q8: torch.Tensor | None = None, k8: torch.Tensor | None = None,
            q_scale: torch.Tensor | None = None, k_scale: torch.Tensor | None = None,
            dqk_signs: torch.Tensor | None = None, prec: int = 0,
            ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, H, T, D = q.shape
    q, k, v, o, do = (_kernel_ready(x) for x in (q, k, v, o, do))
    dq = torch.empty((B, H, T, D), dtype=q.dtype, device=q.device)
    dk = torch.empty((B, H, T, D), dtype=q.dtype, device=q.device)
    dv = torch.empty((B, H, T, D), dtype=q.dtype, device=q.device)
    delta = torch.empty((2, B, H, T), dtype=torch.float32, device=q.device)  # Delta, LSE for bwd
    a = _attn_args(q, k, v, sm_scale, prec)
    a.o, a.o_strides = o.data_ptr(), _strides3(o)
    a.lse = lse.data_ptr()
    a.dout, a.do_strides = do.data_ptr(), _strides3(do)
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.dq_strides, a.dk_strides, a.dv_strides = _strides3(dq), _strides3(dk), _strides3(dv)
    a.delta = delta.data_ptr()
    a.o_lo = o_lo.data_ptr() if o_lo.numel() > 0 else None
    _set_fp8(a, _fp8_tuple(q8, k8, q_scale, k_scale))
    a.dqk_signs = dqk_signs.data_ptr() if dqk_signs is not None else None
    _lib.check(_lib.load().kd_attn_bwd(ctypes.byref(a), *_lib.plan_ref(plan), _stream(q.device)), "kd_attn_bwd")
    return dq, dk, dv


@_bwd_op.register_fake
def _bwd_fake(q, k, v, o, lse, do, plan, sm_scale, o_lo, q8=None, k8=None, q_scale=None, k_scale=None,
              dqk_signs=None, prec=0):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _setup_context(ctx, inputs, output):
    (q, k, v, lens, in_span, span_id, is_prefix, sm_scale, mode, need_lo, bthd, plan_in, signs, quant_fp8,
     prec) = inputs
    o, lse, plan, o_lo, q_r, k_r, q8_o, k8_o, qs_o, ks_o = output
    if plan_in is not None:
        plan = plan_in
    # O's residual and the fp8 / rotated copies are internal; LSE stays
    # differentiable but its gradient is ignored, so the gradients of unused
    # outputs are left as None rather than filled with zeros (o_lo's fill alone
    # would write B H T d 16-bit zeros every backward)
    ctx.mark_non_differentiable(q_r, k_r, q8_o, k8_o, qs_o, ks_o, o_lo)
    ctx.set_materialize_grads(False)
    ctx.fp8 = quant_fp8
    ctx.rot = signs is not None
    if ctx.rot:  # the backward recomputes from the rotated operands and rotates dQ, dK back
        q, k = q_r, k_r
    extra = (q8_o, k8_o, qs_o, ks_o) if ctx.fp8 else ()
    ctx.save_for_backward(q, k, v, o, lse, plan, o_lo, *((signs,) if ctx.rot else ()), *extra)
    ctx.sm_scale = sm_scale
    ctx.prec = prec


def _backward(ctx, do, dlse, dplan, do_lo, *_unused):
    # dlse is ignored, as in original_kernel.py:1965-1992.  With fp8 scores the
    # backward recomputes P from the same fp8 Q8 K8^T and forms dQ = dS K,
    # dK = dS^T Q from the 16-bit operands: the straight-through estimator.
    if do is None:  # O did not reach the loss (only LSE did, whose gradient is ignored)
        return (None,) * 15
    q, k, v, o, lse, plan, o_lo, *rest = ctx.saved_tensors
    signs = rest.pop(0) if ctx.rot else None
    fp8 = tuple(rest) if ctx.fp8 else (None, None, None, None)
    dq, dk, dv = _bwd_op(q, k, v, o, lse, do, plan, ctx.sm_scale, o_lo, *fp8, dqk_signs=signs, prec=ctx.prec)
    return (dq, dk, dv) + (None,) * 12


_fwd_op.register_autograd(_backward, setup_context=_setup_context)


# ---------------------------------------------- fp32 inputs on the MFMA kernels
# For fp32 inputs at precision "tf32" (the reference's default) and head dims
# up to 64, every product runs as three bf16 products on the MFMA kernels, on
# operands of three times the head dim (zero-padded to a built one):
#   Q' = [Qh, Qh, Ql], K' = [Kh, Kl, Kh]    Q' K'^T = Qh Kh^T + Qh Kl^T + Ql Kh^T
#   V' = [Vh, Vl, Vh], dO' = [dOh, dOh, dOl] dP = dO' V'^T likewise; O = P V' in
#                                            columns [0, d) plus [d, 2d)
# with xh = bf16(x), xl = bf16(x - xh): each operand to ~16 significant bits,
# and only the xl yl terms (~2^-16 relative) dropped -- more than the
# reference's tf32 dots (10-bit mantissas, original_kernel.py:452, :1239,
# :1331-1333, :1425, :1517-1523).  P and dS are split by the kernels as for
# 16-bit inputs.  O and the gradients come back with their rounding residuals
# (o_lo, dq_lo, dk_lo, dv_lo), so they too carry ~16 bits.  The gradients of
# the copies that hold xh are the gradient of x (straight through the split):
# dQ = dQ'[0, d) + dQ'[d, 2d), dK = dK'[0, d) + dK'[2d, 3d), dV likewise.
X3_HEAD_DIMS = {16: 64, 32: 128, 64: 256}
# where flash_attention takes this path: at head dim 64 and above the fp32
# MFMA kernels are faster (causal B2 H8 T4096, fwd+bwd: d = 32 1.02 ms here
# against 1.28 ms there, d = 64 2.14 against 1.93 ms) and exact in fp32
X3_ROUTED_HEAD_DIMS = (16, 32)


def _x3(x: torch.Tensor, pattern: str, Dp: int) -> torch.Tensor:
    """[B, H, T, d] fp32 -> contiguous bf16 [B, H, T, Dp]: the parts named by pattern ('h', 'l'), then zeros."""
    xh = x.to(torch.bfloat16)
    xl = (x - xh.to(torch.float32)).to(torch.bfloat16)
    parts = [xh if c == "h" else xl for c in pattern]
    pad = Dp - len(pattern) * x.shape[-1]
    if pad:
        parts.append(xh.new_zeros(x.shape[:-1] + (pad,)))
    return torch.cat(parts, dim=-1)


def _hi_lo(hi: torch.Tensor, lo: torch.Tensor, d: int, second: int) -> torch.Tensor:
    """fp32 (hi + lo)[..., 0:d] + (hi + lo)[..., second * d:(second + 1) * d]."""
    x = hi.to(torch.float32).add_(lo.to(torch.float32))
    return x[..., :d] + x[..., second * d:(second + 1) * d]


@torch.library.custom_op("kdattn::fwd_x3", mutates_args=(), device_types=("cuda",))
def _fwd_x3_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lens: torch.Tensor | None,
               in_span: torch.Tensor | None, span_id: torch.Tensor | None,
               is_prefix: torch.Tensor | None, sm_scale: float, mode: int,
               bthd: bool = False, plan_in: torch.Tensor | None = None,
               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, H, T, d = q.shape
    Dp = X3_HEAD_DIMS[d]
    qx, kx, vx = _x3(q, "hhl", Dp), _x3(k, "hlh", Dp), _x3(v, "hlh", Dp)
    plan = plan_in if plan_in is not None else build_plan(B, T, Dp, q.device, mode, in_span, span_id, is_prefix, lens)
    ox = torch.empty((B, H, T, Dp), dtype=torch.bfloat16, device=q.device)
    ox_lo = torch.empty_like(ox)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    a = _attn_args(qx, kx, vx, sm_scale, _lib.KD_PREC_SPLIT)
    a.o, a.o_strides = ox.data_ptr(), _strides3(ox)
    a.lse = lse.data_ptr()
    a.o_lo = ox_lo.data_ptr()
    _lib.check(_lib.load().kd_attn_fwd(ctypes.byref(a), *_lib.plan_ref(plan), _stream(q.device)), "kd_attn_fwd")
    o = _new_out(B, H, T, d, q, bthd)
    o.copy_(_hi_lo(ox, ox_lo, d, 1))
    return o, lse, (plan if plan_in is None else plan.new_empty(0))


@_fwd_x3_op.register_fake
def _fwd_x3_fake(q, k, v, lens, in_span, span_id, is_prefix, sm_scale, mode, bthd=False, plan_in=None):
    B, H, T, d = q.shape
    return (_new_out(B, H, T, d, q, bthd),
            torch.empty((B, H, T), dtype=torch.float32, device=q.device),
            torch.empty(_lib.plan_nbytes(B, T, X3_HEAD_DIMS[int(d)]) if plan_in is None else 0, dtype=torch.uint8,
                        device=q.device))


@torch.library.custom_op("kdattn::bwd_x3", mutates_args=(), device_types=("cuda",))
def _bwd_x3_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, lse: torch.Tensor,
               do: torch.Tensor, plan: torch.Tensor, sm_scale: float,
               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, H, T, d = q.shape
    Dp = X3_HEAD_DIMS[d]
    qx, kx, vx, dox = _x3(q, "hhl", Dp), _x3(k, "hlh", Dp), _x3(v, "hlh", Dp), _x3(do, "hhl", Dp)
    # the workspace of kd_attn_bwd_dq / kd_attn_bwd_dkdv (kd_attn_args.delta):
    # -Delta with Delta = rowsum(dO O) in fp32, then -LSE / c (-inf where LSE is)
    ws = torch.empty((2, B, H, T), dtype=torch.float32, device=q.device)
    torch.sum(do.to(torch.float32) * o.to(torch.float32), dim=-1, out=ws[0]).neg_()
    # -1/c as the kernels form it, in fp32 on the host: a Python float (exactly that
    # fp32 value) enters the product as a scalar, with no host-to-device copy, so the
    # op stays capturable in a HIP graph
    neg_inv_c = -float(np.float32(1.0) / (np.float32(sm_scale) * np.float32(LOG2E)))
    ninf = torch.full_like(lse, -math.inf)
    torch.where(lse == -math.inf, ninf, lse * neg_inv_c, out=ws[1])
    outs = [torch.empty((B, H, T, Dp), dtype=torch.bfloat16, device=q.device) for _ in range(6)]
    dqx, dkx, dvx, dq_lo, dk_lo, dv_lo = outs
    a = _attn_args(qx, kx, vx, sm_scale, _lib.KD_PREC_SPLIT)
    a.lse = lse.data_ptr()
    a.dout, a.do_strides = dox.data_ptr(), _strides3(dox)
    a.dq, a.dk, a.dv = dqx.data_ptr(), dkx.data_ptr(), dvx.data_ptr()
    a.dq_strides, a.dk_strides, a.dv_strides = _strides3(dqx), _strides3(dkx), _strides3(dvx)
    a.dq_lo, a.dk_lo, a.dv_lo = dq_lo.data_ptr(), dk_lo.data_ptr(), dv_lo.data_ptr()
    a.delta = ws.data_ptr()
    lib, st = _lib.load(), _stream(q.device)
    _lib.check(lib.kd_attn_bwd_dq(ctypes.byref(a), *_lib.plan_ref(plan), st), "kd_attn_bwd_dq")
    _lib.check(lib.kd_attn_bwd_dkdv(ctypes.byref(a), *_lib.plan_ref(plan), st), "kd_attn_bwd_dkdv")
    return _hi_lo(dqx, dq_lo, d, 1), _hi_lo(dkx, dk_lo, d, 2), _hi_lo(dvx, dv_lo, d, 2)


@_bwd_x3_op.register_fake
def _bwd_x3_fake(q, k, v, o, lse, do, plan, sm_scale):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _setup_context_x3(ctx, inputs, output):
    q, k, v, lens, in_span, span_id, is_prefix, sm_scale, mode, bthd, plan_in = inputs
    o, lse, plan = output
    ctx.save_for_backward(q, k, v, o, lse, plan_in if plan_in is not None else plan)
    ctx.set_materialize_grads(False)  # (LSE's gradient is ignored: no zeros made for it)
    ctx.sm_scale = sm_scale


def _backward_x3(ctx, do, dlse, dplan):
    if do is None:  # only LSE reached the loss
        return (None,) * 11
    q, k, v, o, lse, plan = ctx.saved_tensors
    dq, dk, dv = _bwd_x3_op(q, k, v, o, lse, do, plan, ctx.sm_scale)
    return (dq, dk, dv) + (None,) * 8


_fwd_x3_op.register_autograd(_backward_x3, setup_context=_setup_context_x3)


def head_dim_route(dtype: torch.dtype, D: int, precision: str) -> bool:
    """Whether flash_attention runs inputs of this dtype, head dim and precision
    on the bf16x3 ops (fp32 at "tf32" and d = 16, 32); everything else goes to
    the C ABI's kernels as it is, with no padding: 16-bit inputs on the MFMA
    kernels at every head dim (d = 16, 32 on the d = 64 kernels, which read the
    missing columns as zeros), fp32 on the fp32 MFMA kernels (d = 16 on the
    d = 32 ones, the same way)."""
    return dtype == torch.float32 and precision == "tf32" and D in X3_ROUTED_HEAD_DIMS


# -------------------------------------------------------------- public entry
def _check_meta(name, t, B, T, device, dtypes):
    if t is None:
        return None
    if t.shape != (B, T):
        raise ValueError(f"{name} must have shape [B, T] = [{B}, {T}], got {tuple(t.shape)}")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} dtype must be one of {dtypes}, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name} must be on {device}")
    return t


def flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    lens: torch.Tensor | None = None,
    sm_scale: float | None = None,
    causal: bool = True,
    autotune=False,
    return_lse=False,
    prescale_qk=False,
    precision="tf32",
    attention_mask: torch.Tensor | None = None,
    in_span: torch.Tensor | None = None,
    span_id: torch.Tensor | None = None,
    is_prefix: torch.Tensor | None = None,
    return_attention_mask: bool = False,
    *,
    hadamard: bool = False,
    hadamard_seed: int | None = None,
    qk_dtype: str = "bf16",
    out_layout: str = "bhtd",
    plan: AttentionPlan | None = None,
):
    """Hierarchical-mask flash attention on MI355X (same contract as the reference).

    Args mirror ``original_kernel.py:2096-2112``.  ``autotune`` and
    ``prescale_qk`` are accepted and ignored (tile shapes are compile-time
    constants here and the scale is always applied in fp32).  ``precision``
    is ``"ieee"`` or ``"tf32"`` as in the reference.  ``"tf32"`` runs the
    kernels that carry P and dS as 16-bit hi + lo pairs (about 16 significant
    bits in P V, dV, dQ and dK, at or above the reference's bf16 P V and tf32
    backward dots); ``"ieee"`` carries them as hi + mid + lo triples (about 24
    bits, the fp32 of the reference's ieee dots), with O's residual kept in
    fp32 for the backward's Delta.  The extension ``"bf16"`` rounds P and dS
    once to the input type instead (faster; 8 significant bits with bf16
    inputs).  fp32
    inputs get fp32 arithmetic at both "ieee" and "tf32": the fp32 MFMA
    kernels at every head dim, except
    "tf32" at 16 and 32, which runs as bf16x3
    on the 16-bit kernels (see head_dim_route).  O and the gradients stay fp32.
    ``attention_mask``'s contents are not
    read, exactly as in the reference: when it is given without metadata the
    mask formula runs with default metadata, i.e. ``i >= j``.

    Extra keyword-only arguments: ``hadamard`` rotates Q and K by
    ``diag(s) H_d / sqrt(d)`` with signs ``generate_hadamard_signs(d,
    hadamard_seed)`` before the product (exact in real arithmetic);
    ``qk_dtype="fp8_e4m3"`` additionally runs Q K^T on fp8 with per-(b, h)
    absmax scales.  ``out_layout="bthd"`` returns O as a ``[B, H, T, d]`` view of
    ``[B, T, H, d]`` memory, so that ``o.transpose(1, 2).reshape(B, T, H * d)``
    -- what ``MultiHeadAttention`` feeds ``o_proj`` (model.py:95) -- is a view;
    the default is the reference's contiguous O.  ``plan`` (from
    ``build_plan_from_tokens``) replaces the metadata arguments with a plan
    built once and shared, e.g. by all layers of a model.

    Returns ``O``, ``(O, LSE)``, ``(O, mask)`` or ``((O, LSE), mask)`` as at
    ``:2083-2089``; LSE is fp32 ``[B, H, T]`` in log2 units, mask is bool
    ``[B, H, T, T]``.
    """
    if q.dim() != 4:
        raise ValueError("q must be [batch, heads, time, head_dim]")
    B, H, T, D = q.shape
    if D not in REFERENCE_HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {REFERENCE_HEAD_DIMS}, got {D}")
    if k.shape[-1] != D or v.shape[-1] != D:
        raise ValueError("q, k and v must share head_dim")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k and v must have the same [B, H, T, d] shape")
    if precision not in PRECISIONS:
        raise ValueError(f"precision must be 'ieee' or 'tf32' (or the extension 'bf16'), got {precision!r}")
    if lens is not None and (lens.dtype != torch.int32 or lens.dim() != 1 or lens.shape[0] != B):
        raise ValueError("lens must be an int32 tensor of shape [batch]")
    if plan is not None:
        if any(x is not None for x in (in_span, span_id, is_prefix, lens, attention_mask)):
            raise ValueError("plan replaces in_span / span_id / is_prefix / lens / attention_mask")
        if (plan.B, plan.T, plan.D) != (B, T, D) or plan.tensor.device != q.device:
            raise ValueError(f"plan is for [B, T, D] = {[plan.B, plan.T, plan.D]} on {plan.tensor.device}, "
                             f"not {[B, T, D]} on {q.device}")
    if out_layout not in ("bhtd", "bthd"):
        raise ValueError(f"out_layout must be 'bhtd' or 'bthd', got {out_layout!r}")
    if qk_dtype not in ("bf16", "fp8_e4m3"):
        raise ValueError(f"qk_dtype must be 'bf16' or 'fp8_e4m3', got {qk_dtype!r}")
    if qk_dtype == "fp8_e4m3" and precision == "ieee":
        raise ValueError("the fp8 QK^T path runs at precision 'tf32' or 'bf16' (its scores carry 4 significant bits)")
    if not q.is_cuda:
        raise ValueError("flash_attention runs on the GPU only (no CPU fallback)")
    if k.device != q.device or v.device != q.device:
        raise ValueError("q, k and v must be on the same device")
    if qk_dtype == "fp8_e4m3" and (D not in FP8_HEAD_DIMS or q.dtype not in (torch.bfloat16, torch.float32)):
        raise ValueError(f"the fp8 QK^T path is built for head_dim in {FP8_HEAD_DIMS} with bf16 (or fp32) inputs")

    if sm_scale is None:
        sm_scale = D ** -0.5  # original_kernel.py:2145-2147
    device = q.device
    in_span = _check_meta("in_span", in_span, B, T, device, (torch.bool, torch.uint8))
    is_prefix = _check_meta("is_prefix", is_prefix, B, T, device, (torch.bool, torch.uint8))
    span_id = _check_meta("span_id", span_id, B, T, device, (torch.int64, torch.int32))
    if lens is not None and lens.device != device:
        raise ValueError("lens must be on the same device as q")
    mode = _mode(in_span, span_id, is_prefix, attention_mask is not None, causal)

    in_dtype = q.dtype
    if in_dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"unsupported dtype {in_dtype}")
    if qk_dtype == "fp8_e4m3" and in_dtype == torch.float32:
        # fp8 scores come from bf16 operands: fp32 inputs are rounded to bf16
        # for this path and O cast back
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    from .hadamard import _rot_op, generate_hadamard_signs

    fused_signs = None
    if hadamard:
        # (Q R)(K R)^T = Q K^T with R = diag(s) H_d / sqrt(d).  On the MFMA
        # kernels the attention op rotates Q and K itself (fp8: the rotation
        # pass also yields the per-(b, h) absmax that scales the e4m3 copies),
        # and its backward kernels return dQ' R^T, dK' R^T directly.  Elsewhere
        # (fp32, other head dims) Q and K go through the differentiable
        # rotation op first.  With fp8 scores the attention op quantises the
        # Q and K it attends with (after the rotation) itself.
        signs = generate_hadamard_signs(D, hadamard_seed, device=device)
        if q.dtype != torch.float32 and D in MFMA_HEAD_DIMS:
            fused_signs = signs
        else:
            q, k = _rot_op(q, signs, False), _rot_op(k, signs, False)
    x3 = head_dim_route(q.dtype, D, precision)

    if x3:
        # fp32 at the reference's default precision: bf16x3 on the MFMA kernels
        o, lse, plan_t = _fwd_x3_op(q, k, v, lens, in_span, span_id, is_prefix, float(sm_scale), int(mode),
                                    bthd=out_layout == "bthd", plan_in=None if plan is None else plan.tensor)
    else:
        # O's rounding residual, kept for the backward's Delta (16-bit O only)
        need_lo = (q.dtype != torch.float32 and torch.is_grad_enabled()
                   and any(x.requires_grad for x in (q, k, v)))
        o, lse, plan_t, *_ = _fwd_op(q, k, v, lens, in_span, span_id, is_prefix, float(sm_scale), int(mode),
                                     need_lo, bthd=out_layout == "bthd",
                                     plan_in=None if plan is None else plan.tensor, signs=fused_signs,
                                     quant_fp8=qk_dtype == "fp8_e4m3", prec=PRECISIONS[precision])
    if plan is not None:
        plan_t = plan.tensor
    if in_dtype == torch.float32:
        o = o.to(torch.float32)

    mask = None
    if return_attention_mask:
        mask = torch.empty((B, H, T, T), dtype=torch.bool, device=device)
        st = (ctypes.c_int64 * 4)(*mask.stride())
        _lib.check(_lib.load().kd_mask_dense(*_lib.plan_ref(plan_t), B, H, T, D, _ptr(mask), st, _stream(device)),
                   "kd_mask_dense")
    if return_attention_mask:
        if return_lse:
            return (o, lse), mask
        return o, mask
    if return_lse:
        return o, lse
    return o


def plan_views(plan: torch.Tensor, B: int, T: int, D: int) -> dict:
    """Typed views of a plan tensor's sections (codes, class map, lists, work orders)."""
    L = _lib.plan_layout(B, T, D)
    nT = L["nT"]

    def view(off, n, dtype):
        nbytes = n * torch.tensor([], dtype=dtype).element_size()
        return plan[off: off + nbytes].view(dtype)

    nf, nq, nk = L["n_fwd_blocks"], L["n_dq_blocks"], L["n_dkdv_blocks"]
    return {
        "codes": view(L["codes"], B * T, torch.int32).view(B, T),
        "cls": view(L["cls"], B * nT * nT, torch.uint8).view(B, nT, nT),
        "nnz": view(L["nnz"], B * nT * nT, torch.int32).view(B, nT, nT),
        "fwd_list": view(L["fwd_list"], B * nf * nT, torch.int32).view(B, nf, nT),
        "fwd_count": view(L["fwd_count"], B * nf, torch.int32).view(B, nf),
        "dq_list": view(L["dq_list"], B * nq * nT, torch.int32).view(B, nq, nT),
        "dq_count": view(L["dq_count"], B * nq, torch.int32).view(B, nq),
        "dkdv_list": view(L["dkdv_list"], B * nk * nT, torch.int32).view(B, nk, nT),
        "dkdv_count": view(L["dkdv_count"], B * nk, torch.int32).view(B, nk),
        # work orders: items b n + block by descending list length
        "fwd_order": view(L["fwd_order"], B * nf, torch.int32),
        "dq_order": view(L["dq_order"], B * nq, torch.int32),
        "dkdv_order": view(L["dkdv_order"], B * nk, torch.int32),
        "layout": L,
    }


def tile_masks(plan: torch.Tensor, B: int, T: int, D: int):
    """Every 64x64 tile's row and column bit masks ``(rows, cols)``, int64
    ``[B, nT, nT, 64]`` each, from the functions the kernels apply to PARTIAL
    tiles (``kd_tile_masks``): bit j of ``rows[b, qt, kt, r]`` = query 64 qt + r
    may see key 64 kt + j; bit r of ``cols[b, qt, kt, j]`` = the same pair."""
    nT = (T + 63) // 64
    rows = torch.empty((B, nT, nT, 64), dtype=torch.int64, device=plan.device)
    cols = torch.empty_like(rows)
    _lib.check(_lib.load().kd_tile_masks(*_lib.plan_ref(plan), B, T, D, _ptr(rows), _ptr(cols), _stream(plan.device)),
               "kd_tile_masks")
    return rows, cols


def mask_mode(in_span=None, span_id=None, is_prefix=None, attention_mask=None, causal=True) -> int:
    return _mode(in_span, span_id, is_prefix, attention_mask is not None, causal)


LOG2E = math.log2(math.e)
