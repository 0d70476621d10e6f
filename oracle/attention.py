"""Dense masked attention on the CPU (test oracle and CPU baseline).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Forward follows the algebra of ``original_kernel.py:550-579`` and ``:603-604``
(softmax in base 2, LSE stored in log2 units), backward the algebra of
``:1239-1335`` (dQ) and ``:1425-1524`` (dK/dV), with Delta from ``:695``.
Evaluated densely in fp64 (or fp32), with ONE fp32-exact scale
``sm_scale * log2(e)`` -- the reference's bf16-rounded scale constants
(``:415``, ``:1214``) are deliberately not reproduced.

Fully masked rows give O = 0, LSE = -inf and zero gradient (the guarded
``q_attended`` path of ``:547-576``, not the NaN path).
"""
from __future__ import annotations

import math

import torch

LOG2E = math.log2(math.e)


def _mask_t(mask, B, H, T):
    m = torch.as_tensor(mask)
    if m.dim() == 3:  # [B, T, T] shared across heads
        m = m[:, None]
    return m.expand(B, H, T, T)


def forward(q, k, v, mask, sm_scale, dtype=torch.float64):
    """Return ``(O, LSE2)``; O in ``dtype``, LSE2 = log2-sum-exp2 of S*c."""
    B, H, T, D = q.shape
    m = _mask_t(mask, B, H, T)
    q, k, v = (x.to(dtype) for x in (q, k, v))
    s = torch.matmul(q, k.transpose(-1, -2)) * (sm_scale * LOG2E)
    s = s.masked_fill(~m, float("-inf"))
    mx = s.amax(dim=-1, keepdim=True)
    row_any = m.any(dim=-1, keepdim=True)
    mx_safe = torch.where(row_any, mx, torch.zeros_like(mx))
    p = torch.exp2(s - mx_safe)
    l = p.sum(dim=-1, keepdim=True)
    l_safe = torch.where(row_any, l, torch.ones_like(l))
    o = torch.matmul(p / l_safe, v)
    lse = torch.where(row_any, mx_safe + torch.log2(l_safe), torch.full_like(l, float("-inf")))
    return o, lse[..., 0]


def probabilities(q, k, mask, sm_scale, dtype=torch.float64):
    B, H, T, D = q.shape
    m = _mask_t(mask, B, H, T)
    s = torch.matmul(q.to(dtype), k.to(dtype).transpose(-1, -2)) * (sm_scale * LOG2E)
    s = s.masked_fill(~m, float("-inf"))
    mx = s.amax(dim=-1, keepdim=True)
    mx = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
    p = torch.exp2(s - mx)
    l = p.sum(dim=-1, keepdim=True)
    return p / torch.where(l > 0, l, torch.ones_like(l))


def backward(q, k, v, o, do, mask, sm_scale, dtype=torch.float64, score_q=None, score_k=None):
    """Closed-form gradients ``(dQ, dK, dV, Delta)`` of :func:`forward`.

    ``Delta = rowsum(O * dO)`` (``original_kernel.py:695``),
    ``dS = P * (dP - Delta)`` (``:1332``), ``dQ = scale * dS K`` (``:1333-1335``),
    ``dK = scale * dS^T Q`` (``:1523-1524``), ``dV = P^T dO`` (``:1517``).

    ``score_q`` / ``score_k`` (the fp8 QK^T variant, which the reference does
    not have): P is formed from them -- the dequantised fp8 copies
    ``scale * e4m3`` whose product gave the forward's O and LSE -- while dQ and
    dK use ``k`` and ``q``: the straight-through estimator applied to the
    score product (its value is the fp8 product, its gradient that of
    ``q k^T``).
    """
    q, k, v, o, do = (x.to(dtype) for x in (q, k, v, o, do))
    if score_q is None:
        p = probabilities(q, k, mask, sm_scale, dtype)
    else:
        p = probabilities(score_q.to(dtype), score_k.to(dtype), mask, sm_scale, dtype)
    delta = (o * do).sum(-1)
    dp = torch.matmul(do, v.transpose(-1, -2))
    ds = p * (dp - delta[..., None])
    dq = torch.matmul(ds, k) * sm_scale
    dk = torch.matmul(ds.transpose(-1, -2), q) * sm_scale
    dv = torch.matmul(p.transpose(-1, -2), do)
    return dq, dk, dv, delta


def autograd_reference(q, k, v, do, mask, sm_scale, dtype=torch.float64, score_q=None, score_k=None):
    """Independent route: torch autograd through a naive masked softmax.

    With ``score_q`` / ``score_k`` the scores are ``q k^T + (score_q score_k^T -
    q k^T).detach()``: the value of the score operands' product, the gradient
    of ``q k^T`` (straight through the quantised product).
    """
    B, H, T, D = q.shape
    m = _mask_t(mask, B, H, T)
    q, k, v = (x.detach().to(dtype).requires_grad_(True) for x in (q, k, v))
    s = torch.matmul(q, k.transpose(-1, -2))
    if score_q is not None:
        s8 = torch.matmul(score_q.to(dtype), score_k.to(dtype).transpose(-1, -2))
        s = s + (s8 - s).detach()
    s = s * sm_scale
    s = s.masked_fill(~m, float("-inf"))
    row_any = m.any(-1, keepdim=True)
    s = torch.where(row_any, s, torch.zeros_like(s))
    p = torch.softmax(s, dim=-1) * row_any
    o = torch.matmul(p, v)
    o.backward(do.to(dtype))
    return o.detach(), q.grad, k.grad, v.grad


def sdpa_baseline(q, k, v, do, mask, sm_scale):
    """The reference's eager dense-masked attention pattern on the CPU.

    ``original_kernel.py:2002-2032`` (``flash_attention_reference``) calls
    ``F.scaled_dot_product_attention`` with a dense boolean mask; here the
    mask is the hierarchical one and everything runs in fp32 on the host,
    forward then backward through autograd.  Returns ``(O, dQ, dK, dV)``.
    """
    B, H, T, D = q.shape
    m = _mask_t(mask, B, H, T)
    q, k, v = (x.detach().float().requires_grad_(True) for x in (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=m, scale=sm_scale)
    o.backward(do.float())
    return o.detach(), q.grad, k.grad, v.grad

