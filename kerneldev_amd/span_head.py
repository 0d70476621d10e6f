"""Cocktail-party head: span-interior mean pooling and scores on gfx950.

Replaces the head of KernelDev's ``GPTModel.forward`` (``model.py:263-298``):
the hidden state at each row's first ``[MASK]`` is dotted with the mean hidden
state of every span interior.  The reference fills ``h_spans`` with a Python
double loop over rows and over the zipped ``[SPAN]`` / ``[ES]`` positions
(``:287-293``); here ``kd_span_scores`` does the pooling and the scores in two
kernel launches and ``kd_span_scores_bwd`` returns ``d h``.

Pairing: the j-th ``[SPAN]`` of a row goes with the row's j-th ``[ES]``, as the
reference's ``zip(st_indices, ed_indices)`` does when a row holds as many of
each (``:287-291``).  When the counts differ the reference indexes
``span_ends`` with the start list's row mask, which raises (different totals)
or pairs across rows; the kernel keeps each row's own lists.  The interior is
``[st + 1, ed)``; a pair with ``st + 1 >= ed`` or without a partner scores 0
(the zero row of ``h_spans``, ``:285``, ``:292``).

Scores are fp32: the reference forms them in the model dtype (``einsum`` of
bf16), but at random init they are large and nearly equal, where the
rounding of a bf16 result would decide the loss.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import SpanArgs
from .metadata import ES, MASK, SPAN


def _dtype_code(dt):
    from .attention import _dtype_code as f

    return f(dt)


def _args(tokens, h, n):
    a = SpanArgs()
    a.tokens = tokens.data_ptr()
    a.tokens_strides = (ctypes.c_int64 * 2)(*tokens.stride())
    a.tokens_dtype = 0 if tokens.dtype == torch.int64 else 1
    a.dtype = _dtype_code(h.dtype)
    a.h = h.data_ptr()
    a.h_strides = (ctypes.c_int64 * 2)(h.stride(0), h.stride(1))
    a.B, a.T, a.D = h.shape
    a.n_spans = n
    return a


def _check_inputs(tokens, h):
    if tokens.dim() != 2 or h.dim() != 3 or tuple(tokens.shape) != tuple(h.shape[:2]):
        raise ValueError(f"tokens [B, T] and h [B, T, D] expected, got {tuple(tokens.shape)} and {tuple(h.shape)}")
    if tokens.dtype not in (torch.int64, torch.int32):
        raise ValueError(f"tokens must be int64 or int32, got {tokens.dtype}")
    if h.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"h must be bf16 or fp16, got {h.dtype}")
    if h.device.type != "cuda" or tokens.device != h.device:
        raise ValueError("tokens and h must be on the same GPU")


@torch.library.custom_op("kdattn::span_fwd", mutates_args=(), device_types=("cuda",))
def _span_fwd_op(tokens: torch.Tensor, h: torch.Tensor, n_spans: int) -> tuple[
        torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    if h.stride(2) != 1:
        h = h.contiguous()
    B, T, D = h.shape
    f32, i32 = dict(dtype=torch.float32, device=h.device), dict(dtype=torch.int32, device=h.device)
    scores = torch.empty(B, n_spans, **f32)
    h_ctx = torch.empty(B, D, **f32)
    h_spans = torch.empty(B, n_spans, D, **f32)
    lo = torch.empty(B, n_spans, **i32)
    hi = torch.empty(B, n_spans, **i32)
    mpos = torch.empty(B, **i32)
    a = _args(tokens, h, n_spans)
    a.scores, a.h_ctx, a.h_spans = scores.data_ptr(), h_ctx.data_ptr(), h_spans.data_ptr()
    a.span_lo, a.span_hi, a.mask_pos = lo.data_ptr(), hi.data_ptr(), mpos.data_ptr()
    stream = ctypes.c_void_p(torch.cuda.current_stream(h.device).cuda_stream)
    _lib.check(_lib.load().kd_span_scores(ctypes.byref(a), stream), "kd_span_scores")
    return scores, h_ctx, h_spans, lo, hi, mpos


@_span_fwd_op.register_fake
def _span_fwd_fake(tokens, h, n_spans):
    B, T, D = h.shape
    f32, i32 = dict(dtype=torch.float32, device=h.device), dict(dtype=torch.int32, device=h.device)
    return (torch.empty(B, n_spans, **f32), torch.empty(B, D, **f32), torch.empty(B, n_spans, D, **f32),
            torch.empty(B, n_spans, **i32), torch.empty(B, n_spans, **i32), torch.empty(B, **i32))


@torch.library.custom_op("kdattn::span_bwd", mutates_args=(), device_types=("cuda",))
def _span_bwd_op(tokens: torch.Tensor, h: torch.Tensor, dscores: torch.Tensor, h_ctx: torch.Tensor,
                 h_spans: torch.Tensor, lo: torch.Tensor, hi: torch.Tensor, mpos: torch.Tensor) -> torch.Tensor:
    B, T, D = h.shape
    n = dscores.shape[1]
    dscores = dscores.float().contiguous()
    dh = torch.empty(B, T, D, dtype=h.dtype, device=h.device)
    a = _args(tokens, h, n)
    a.h_ctx, a.h_spans = h_ctx.data_ptr(), h_spans.data_ptr()
    a.span_lo, a.span_hi, a.mask_pos = lo.data_ptr(), hi.data_ptr(), mpos.data_ptr()
    a.dscores = dscores.data_ptr()
    a.dh = dh.data_ptr()
    a.dh_strides = (ctypes.c_int64 * 2)(dh.stride(0), dh.stride(1))
    stream = ctypes.c_void_p(torch.cuda.current_stream(h.device).cuda_stream)
    _lib.check(_lib.load().kd_span_scores_bwd(ctypes.byref(a), stream), "kd_span_scores_bwd")
    return dh


@_span_bwd_op.register_fake
def _span_bwd_fake(tokens, h, dscores, h_ctx, h_spans, lo, hi, mpos):
    return torch.empty(h.shape, dtype=h.dtype, device=h.device)


def _span_setup(ctx, inputs, output):
    tokens, h, _ = inputs
    _, h_ctx, h_spans, lo, hi, mpos = output
    ctx.save_for_backward(tokens, h, h_ctx, h_spans, lo, hi, mpos)
    ctx.mark_non_differentiable(h_ctx, h_spans, lo, hi, mpos)
    ctx.set_materialize_grads(False)  # (no zero tensors for the gradients of those outputs)


def _span_backward(ctx, dscores, *_):
    if dscores is None:  # the scores did not reach the loss
        return None, None, None
    tokens, h, h_ctx, h_spans, lo, hi, mpos = ctx.saved_tensors
    return None, _span_bwd_op(tokens, h, dscores, h_ctx, h_spans, lo, hi, mpos), None


_span_fwd_op.register_autograd(_span_backward, setup_context=_span_setup)


def max_spans(tokens: torch.Tensor) -> int:
    """The reference's ``max_spans``: the largest per-row ``[SPAN]`` count (one host sync)."""
    return int((tokens == SPAN).sum(dim=1).max().item())


def span_scores(tokens: torch.Tensor, h: torch.Tensor, n_spans: int | None = None) -> torch.Tensor:
    """Scores ``[B, n_spans]`` (fp32) of each span interior's mean against h at the first ``[MASK]``.

    ``n_spans`` defaults to :func:`max_spans` (the reference's column count).
    Differentiable in ``h``.
    """
    _check_inputs(tokens, h)
    n = max_spans(tokens) if n_spans is None else int(n_spans)
    if n < 1:
        raise ValueError("no [SPAN] token in the batch (the reference returns an empty result there)")
    return _span_fwd_op(tokens, h, n)[0]


def has_cocktail_layout(tokens: torch.Tensor) -> bool:
    """The reference's output-mode test (``model.py:255-256``), in one host sync."""
    flags = torch.stack([(tokens == MASK).any(), (tokens == SPAN).any(), (tokens == ES).any()]).tolist()
    return all(flags)
