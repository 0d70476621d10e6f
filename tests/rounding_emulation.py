"""CPU emulation of the attention kernels' roundings of P and dS.

Test infrastructure.  The kernels compute S, dP and every product in fp32 on
the MFMA; the only roundings that matter on outlier data are those of the
16-bit B operands P (into P V and dV = P^T dO) and dS (into dQ = dS K and
dK = dS^T Q), and of the outputs.  This module restates those steps in numpy
for one (b, h) head and measures, per product, the worst error beyond one
output ulp (the per-element part of the parity bar, ``helpers.assert_close``)
against an fp64 evaluation of the same inputs, for three forms of P and dS:

* ``"bf16"``: one rounding to bf16 (8 significant bits; the reference rounds P
  to V's dtype, original_kernel.py:566-571, and this is ``precision="bf16"``);
* ``"fp16"``: one rounding to fp16 (11 significant bits), with the product's
  other operand (V, dO, K or Q, bf16 inputs) converted to fp16 as the fp16
  MFMA would need it -- exact for |x| in [2^-14, 65504];
* ``"bf16x2"``: the pair hi = bf16(x), lo = bf16(x - hi) (about 16 significant
  bits; the kernels' default split precision, ``pack8_residual``).

The kernel steps restated (kd_fwd.hip, kd_bwd.hip):

* forward: p = exp2(fma(S, c, -m c)) in fp32 with m the row max (the lazy
  rescale only changes m by a power of two, which no form's relative rounding
  sees), O = sum_j form(p_j) V_j / sum_j form(p_j), stored as bf16;
* backward: P = exp2(fma(S, c, -LSE)) in fp32, dP = dO V^T accumulated in fp32,
  Delta = rowsum(dO O) (O carried to ~16 bits by O + O_lo), dS = P (dP - Delta)
  in fp32; dV = form(P)^T dO, dQ = sm_scale form(dS) K, dK = sm_scale
  form(dS)^T Q, each stored as bf16; with Hadamard, dQ and dK are taken back
  through R^T before the rounding, as the kernels' epilogues do.

The products' own fp32 accumulation is evaluated in fp64 here: its error
(~2^-24 relative per term) is three orders below every form's rounding.
"""
from __future__ import annotations

import math

import numpy as np

LOG2E = math.log2(math.e)
FORMS = ("bf16", "fp16", "bf16x2")
PRODUCTS = ("O", "dV", "dQ", "dK")  # P V, P^T dO, dS K, dS^T Q
FP16_MAX = 65504.0


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32, as v_cvt_pk_bf16_f32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def fp16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 (round to nearest even, subnormals kept) -> fp32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def as_form(x: np.ndarray, form: str) -> np.ndarray:
    """What the MFMA sees of the fp32 values x in the given form (fp64 result)."""
    if form == "bf16":
        return bf16_round(x).astype(np.float64)
    if form == "fp16":
        return fp16_round(x).astype(np.float64)
    if form == "bf16x2":
        hi = bf16_round(x)
        lo = bf16_round(x - hi)
        return hi.astype(np.float64) + lo.astype(np.float64)
    raise ValueError(form)


def operand(x: np.ndarray, form: str) -> np.ndarray:
    """The other operand (bf16 input values) as the product of this form takes it."""
    if form == "fp16":
        return fp16_round(x).astype(np.float64)
    return x.astype(np.float64)


def ulp_bf16(ref: np.ndarray) -> np.ndarray:
    a = np.maximum(np.abs(ref), 1e-30)
    return np.where(ref == 0, 0.0, np.exp2(np.floor(np.log2(a)) - 7))


def excess(got_f64: np.ndarray, ref: np.ndarray) -> float:
    """max |bf16(got) - ref| beyond one bf16 ulp of ref."""
    out = bf16_round(got_f64.astype(np.float32)).astype(np.float64)
    return float(np.max(np.maximum(np.abs(out - ref) - ulp_bf16(ref), 0.0), initial=0.0))


def emulate_head(q, k, v, do, mask, sm_scale, rot=None, block=1024):
    """Worst error beyond one bf16 ulp per (product, form) for one head.

    q, k, v, do: float32 arrays [T, d] holding the bf16 inputs (q and k already
    rotated and rounded when ``rot`` is given); mask: bool [T, T]; rot: the
    fp64 rotation R (dQ, dK are reported for the unrotated inputs, times R^T).
    Returns ``{"excess": {(product, form): float}, "max_abs_ds": float,
    "ref_max": {product: float}}``.
    """
    T, d = q.shape
    c32 = np.float32(sm_scale * LOG2E)
    c64 = float(c32)
    k64, v64, q64, do64 = (x.astype(np.float64) for x in (k, v, q, do))
    row_any = mask.any(axis=1)

    # forward, query blocks: O per form, and the exact O and LSE for the backward
    ex = {(p, f): 0.0 for p in PRODUCTS for f in FORMS}
    o_ref = np.zeros((T, d))
    lse = np.full(T, -np.inf)
    for r0 in range(0, T, block):
        rows = slice(r0, min(T, r0 + block))
        mb = mask[rows]
        s64 = q64[rows] @ k64.T
        s32 = s64.astype(np.float32)
        m = np.where(mb, s32, -np.inf).max(axis=1)
        m = np.where(np.isfinite(m), m, 0.0).astype(np.float32)
        p32 = np.exp2(np.where(mb, s32 * c32 - (m * c32)[:, None], -np.inf)).astype(np.float32)
        p64 = np.where(mb, np.exp2(s64 * c64 - (m.astype(np.float64) * c64)[:, None]), 0.0)
        l64 = p64.sum(axis=1)
        ok = row_any[rows]
        ref = np.where(ok[:, None], (p64 @ v64) / np.where(ok, l64, 1.0)[:, None], 0.0)
        o_ref[rows] = ref
        lse[rows] = np.where(ok, m.astype(np.float64) * c64 + np.log2(np.where(ok, l64, 1.0)), -np.inf)
        for f in FORMS:
            pf = as_form(p32, f)
            lf = pf.sum(axis=1)
            got = np.where(ok[:, None], (pf @ operand(v, f)) / np.where(lf > 0, lf, 1.0)[:, None], 0.0)
            ex[("O", f)] = max(ex[("O", f)], excess(got, ref))

    # backward: dQ per query block, dV and dK accumulated over the blocks
    lse32 = lse.astype(np.float32)
    delta64 = (do64 * o_ref).sum(axis=1)  # Delta from O to ~16 bits (O + O_lo)
    delta32 = delta64.astype(np.float32)
    dv_ref = np.zeros((T, d))
    dk_ref = np.zeros((T, d))
    dv = {f: np.zeros((T, d)) for f in FORMS}
    dk = {f: np.zeros((T, d)) for f in FORMS}
    max_ds = 0.0
    dq_parts = {f: [] for f in FORMS}
    dq_ref_parts = []
    for r0 in range(0, T, block):
        rows = slice(r0, min(T, r0 + block))
        mb = mask[rows]
        s64 = q64[rows] @ k64.T
        s32 = s64.astype(np.float32)
        l32 = np.where(np.isfinite(lse32[rows]), lse32[rows], np.float32(np.inf))
        P32 = np.where(mb, np.exp2(s32 * c32 - l32[:, None]), 0.0).astype(np.float32)
        l64 = np.where(np.isfinite(lse[rows]), lse[rows], np.inf)
        P64 = np.where(mb, np.exp2(s64 * c64 - l64[:, None]), 0.0)
        dp64 = do64[rows] @ v64.T
        dS32 = (P32 * (dp64.astype(np.float32) - delta32[rows][:, None])).astype(np.float32)
        dS64 = P64 * (dp64 - delta64[rows][:, None])
        max_ds = max(max_ds, float(np.abs(dS32).max(initial=0.0)))
        dv_ref += P64.T @ do64[rows]
        dk_ref += dS64.T @ q64[rows]
        dq_ref_parts.append(dS64 @ k64)
        for f in FORMS:
            Pf, dSf = as_form(P32, f), as_form(dS32, f)
            dv[f] += Pf.T @ operand(do[rows], f)
            dk[f] += dSf.T @ operand(q[rows], f)
            dq_parts[f].append(dSf @ operand(k, f))

    def finish(x):  # scale, and back through R^T for the rotated inputs
        x = x * sm_scale
        return x @ rot.T if rot is not None else x

    dq_ref = finish(np.concatenate(dq_ref_parts))
    dk_ref = finish(dk_ref)
    refs = {"O": o_ref, "dV": dv_ref, "dQ": dq_ref, "dK": dk_ref}
    for f in FORMS:
        ex[("dV", f)] = excess(dv[f], dv_ref)
        ex[("dQ", f)] = excess(finish(np.concatenate(dq_parts[f])), dq_ref)
        ex[("dK", f)] = excess(finish(dk[f]), dk_ref)
    return {"excess": ex, "max_abs_ds": max_ds, "ref_max": {p: float(np.abs(r).max()) for p, r in refs.items()}}


def config4_head(b: int, h: int, hadamard: bool, seed: int = 0):
    """Inputs of one config-4 head as emulate_head takes them, plus its mask."""
    import torch

    from kerneldev_amd.hadamard import generate_hadamard_signs
    from kerneldev_amd.synth import config_inputs
    from oracle.hadamard import rotate_fp32, rotation_matrix
    from oracle.mask import dense_mask

    inp = config_inputs(4, seed=seed)
    T, D = inp["q"].shape[2], inp["q"].shape[3]
    mask = dense_mask(T, B=inp["q"].shape[0], in_span=inp["in_span"].numpy(), span_id=inp["span_id"].numpy(),
                      is_prefix=inp["is_prefix"].numpy())[b]
    q, k, v, do = (inp[n][b, h].to(torch.float32).numpy() for n in ("q", "k", "v", "do"))
    rot = None
    if hadamard:
        signs = generate_hadamard_signs(D, 0).numpy()
        q, k = (bf16_round(rotate_fp32(x, signs)) for x in (q, k))
        rot = rotation_matrix(signs)
    return q, k, v, do, mask, D ** -0.5, rot
