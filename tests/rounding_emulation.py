"""CPU emulation of the attention kernels' roundings of P and dS.

Test infrastructure.  The kernels compute S, dP and every product in fp32 on
the MFMA; the roundings that matter on outlier data are those of the 16-bit B
operands P (into P V and dV = P^T dO) and dS (into dQ = dS K and dK = dS^T Q),
and of the outputs.  This module restates those steps in numpy for one (b, h)
head and measures, per product, the worst error beyond one output ulp (the
per-element part of the parity bar, ``helpers.assert_close``) against an fp64
evaluation of the same inputs, for three forms of P and dS:

* ``"bf16"``: one rounding to bf16 (8 significant bits; the reference rounds P
  to V's dtype, original_kernel.py:566-571, and this is ``precision="bf16"``);
* ``"fp16"``: one rounding to fp16 (11 significant bits), with the product's
  other operand (V, dO, K or Q, bf16 inputs) converted to fp16 as the fp16
  MFMA would need it -- exact for |x| in [2^-14, 65504];
* ``"bf16x2"``: the pair hi = bf16(x), lo = bf16(x - hi) (about 16 significant
  bits; the kernels' default split precision, ``pack8_residual``).

The kernel steps restated (kd_fwd.hip, kd_bwd.hip):

* forward: p = exp2(S c - m c) in fp32 with m the row max (the lazy rescale
  only changes m by a power of two, which no form's relative rounding sees),
  O = sum_j form(p_j) V_j / sum_j form(p_j), stored as bf16, and
  LSE = m c + log2(sum_j form(p_j));
* backward: P = exp2(S c - LSE) in fp32, dP = dO V^T accumulated in fp32,
  Delta = rowsum(dO O) with the forward's O (carried to ~16 bits by O + O_lo),
  dS = P (dP - Delta) in fp32; dV = form(P)^T dO, dQ = sm_scale form(dS) K,
  dK = sm_scale form(dS)^T Q, each stored as bf16; with Hadamard, dQ and dK go
  back through R^T before the rounding, as the kernels' epilogues do.

The backward is evaluated twice: with the forward's O and LSE from the split
forward (what the kernels run), which isolates each backward product's own
rounding, and with the O and LSE of a forward whose P V took P rounded once to
fp16 ("coupled"), which shows what that cheaper forward would do to the
gradients through Delta = rowsum(dO O) and the dP - Delta cancellation.

The products' own fp32 accumulation is evaluated in fp64 here: its error
(~2^-24 relative per term) is three orders below every form's rounding.

``python tests/rounding_emulation.py [b,h ...]`` prints the table for the
listed config-4 heads (default: every head).
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

LOG2E = math.log2(math.e)
FORMS = ("bf16", "fp16", "bf16x2")
PRODUCTS = ("O", "dV", "dQ", "dK")  # P V, P^T dO, dS K, dS^T Q


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


def emulate_head(q, k, v, do, mask, sm_scale, rot=None, block=256):
    """Worst error beyond one bf16 ulp per (product, form) for one head.

    block: query rows per pass (256: [256, T] temporaries of 16 MB in fp64;
    the fp64 sums over passes change with it in the last bits only).
    q, k, v, do: float32 arrays [T, d] holding the bf16 inputs (q and k already
    rotated and rounded when ``rot`` is given); mask: bool [T, T]; rot: the
    fp64 rotation R (dQ, dK are reported for the unrotated inputs, times R^T).
    Returns ``{"excess": {(product, form): float}, "coupled": {product: float},
    "max_abs_ds": float, "ref_max": {product: float}, "refs": {product: array}}``:
    "coupled" holds dV, dQ, dK in the split form with Delta and LSE from a
    forward whose P V took P rounded once to fp16; "refs" the fp64 results the
    excesses are measured against.
    """
    T, d = q.shape
    c32 = np.float32(sm_scale * LOG2E)
    c64 = float(c32)
    k64, v64, q64, do64 = (x.astype(np.float64) for x in (k, v, q, do))
    row_any = mask.any(axis=1)

    # forward, query blocks: O per form; O and LSE of the exact, split and fp16 forwards
    ex = {(p, f): 0.0 for p in PRODUCTS for f in FORMS}
    o_ref = np.zeros((T, d))
    o_fwd = {"bf16x2": np.zeros((T, d)), "fp16": np.zeros((T, d))}
    lse = np.full(T, -np.inf)
    lse_fwd = {f: np.full(T, -np.inf) for f in o_fwd}
    for r0 in range(0, T, block):
        rows = slice(r0, min(T, r0 + block))
        mb = mask[rows]
        ok = row_any[rows]
        s64 = q64[rows] @ k64.T
        s32 = s64.astype(np.float32)
        m = np.where(mb, s32, -np.inf).max(axis=1)
        m = np.where(np.isfinite(m), m, 0.0).astype(np.float32)
        p32 = np.exp2(np.where(mb, s32 * c32 - (m * c32)[:, None], -np.inf)).astype(np.float32)
        p64 = np.where(mb, np.exp2(s64 * c64 - (m.astype(np.float64) * c64)[:, None]), 0.0)
        l64 = p64.sum(axis=1)
        ref = np.where(ok[:, None], (p64 @ v64) / np.where(ok, l64, 1.0)[:, None], 0.0)
        o_ref[rows] = ref
        lse[rows] = np.where(ok, m.astype(np.float64) * c64 + np.log2(np.where(ok, l64, 1.0)), -np.inf)
        for f in FORMS:
            pf = as_form(p32, f)
            lf = pf.sum(axis=1)
            got = np.where(ok[:, None], (pf @ operand(v, f)) / np.where(lf > 0, lf, 1.0)[:, None], 0.0)
            ex[("O", f)] = max(ex[("O", f)], excess(got, ref))
            if f in o_fwd:
                o_fwd[f][rows] = got
                lse_fwd[f][rows] = np.where(ok, m.astype(np.float64) * c64 + np.log2(np.where(lf > 0, lf, 1.0)),
                                            -np.inf)

    # backward: dQ per query block, dV and dK accumulated over the blocks; the
    # exact gradients use the exact O and LSE, the emulated ones the forward's
    delta64 = (do64 * o_ref).sum(axis=1)
    fwd_delta = {f: (do64 * o_fwd[f]).sum(axis=1).astype(np.float32) for f in o_fwd}
    fwd_lse = {f: lse_fwd[f].astype(np.float32) for f in o_fwd}
    runs = [("bf16x2", f) for f in FORMS] + [("fp16", "bf16x2")]  # (forward form, backward form)
    acc = {r: {"dv": np.zeros((T, d)), "dk": np.zeros((T, d)), "dq": []} for r in runs}
    dv_ref, dk_ref, dq_ref = np.zeros((T, d)), np.zeros((T, d)), []
    max_ds = 0.0
    for r0 in range(0, T, block):
        rows = slice(r0, min(T, r0 + block))
        mb = mask[rows]
        s64 = q64[rows] @ k64.T
        s32 = s64.astype(np.float32)
        l64 = np.where(np.isfinite(lse[rows]), lse[rows], np.inf)
        P64 = np.where(mb, np.exp2(s64 * c64 - l64[:, None]), 0.0)
        dp64 = do64[rows] @ v64.T
        dp32 = dp64.astype(np.float32)
        dS64 = P64 * (dp64 - delta64[rows][:, None])
        dv_ref += P64.T @ do64[rows]
        dk_ref += dS64.T @ q64[rows]
        dq_ref.append(dS64 @ k64)
        for ff in o_fwd:
            l32 = np.where(np.isfinite(fwd_lse[ff][rows]), fwd_lse[ff][rows], np.float32(np.inf))
            P32 = np.where(mb, np.exp2(s32 * c32 - l32[:, None]), 0.0).astype(np.float32)
            dS32 = (P32 * (dp32 - fwd_delta[ff][rows][:, None])).astype(np.float32)
            if ff == "bf16x2":
                max_ds = max(max_ds, float(np.abs(dS32).max(initial=0.0)))
            for fwd, f in runs:
                if fwd != ff:
                    continue
                Pf, dSf = as_form(P32, f), as_form(dS32, f)
                a = acc[(fwd, f)]
                a["dv"] += Pf.T @ operand(do[rows], f)
                a["dk"] += dSf.T @ operand(q[rows], f)
                a["dq"].append(dSf @ operand(k, f))

    def finish(x):  # scale, and back through R^T for the rotated inputs
        x = x * sm_scale
        return x @ rot.T if rot is not None else x

    dq_ref = finish(np.concatenate(dq_ref))
    dk_ref = finish(dk_ref)
    refs = {"O": o_ref, "dV": dv_ref, "dQ": dq_ref, "dK": dk_ref}

    def grads(a):
        return {"dV": excess(a["dv"], dv_ref), "dQ": excess(finish(np.concatenate(a["dq"])), dq_ref),
                "dK": excess(finish(a["dk"]), dk_ref)}

    for f in FORMS:
        for p, e in grads(acc[("bf16x2", f)]).items():
            ex[(p, f)] = e
    return {"excess": ex, "coupled": grads(acc[("fp16", "bf16x2")]), "max_abs_ds": max_ds,
            "ref_max": {p: float(np.abs(r).max()) for p, r in refs.items()}, "refs": refs}


def head_qkvdo(b, h, B, H, L, d, seed, outlier_frac=0.0, outlier_mult=20.0):
    """Head (b, h) of ``kerneldev_amd.synth.qkvdo(B, H, L, d, seed, ...)``'s
    Q, K, V, dO (bf16), drawn without the other heads: the same generator
    calls in the same order, one [L, d] slice at a time.  torch's CPU normal
    fill draws its uniforms in order and transforms them in independent blocks
    of 16, so slices of L d values (a multiple of 16) reproduce the whole
    tensor's draw (tests/test_rounding_budget.py pins this against qkvdo).
    Config 4's full inputs are ~1 GB each in fp32; one head is 4 MB."""
    import math

    import torch

    g = torch.Generator("cpu").manual_seed(seed)
    out = []
    for idx in range(4):
        x = None
        for bh in range(B * H):
            c = torch.randn(L, d, generator=g, dtype=torch.float32)
            if bh == b * H + h:
                x = c
        if outlier_frac > 0 and idx < 3:
            n_out = math.ceil(outlier_frac * d)
            for hh in range(H):
                ch = torch.randperm(d, generator=g)[:n_out]
                if hh == h:
                    x[:, ch] *= outlier_mult
        out.append(x.to(torch.bfloat16))
    return tuple(out)


def config4_head(b: int, h: int, hadamard: bool, seed: int = 0):
    """Inputs of one config-4 head (``kerneldev_amd.synth.config_inputs(4,
    seed)[.][b, h]``) as emulate_head takes them, plus its mask."""
    import torch

    from kerneldev_amd.hadamard import generate_hadamard_signs
    from kerneldev_amd.synth import CONFIG4_LAYOUT, cocktail_batch
    from oracle.hadamard import rotate_fp32, rotation_matrix
    from oracle.mask import dense_mask

    B, H, T, D = 2, 32, 8192, 128
    _, in_span, span_id, is_prefix = cocktail_batch(B, T, CONFIG4_LAYOUT, seed)
    mask = dense_mask(T, B=1, in_span=in_span[b:b + 1].numpy(), span_id=span_id[b:b + 1].numpy(),
                      is_prefix=is_prefix[b:b + 1].numpy())[0]
    q, k, v, do = (x.to(torch.float32).numpy() for x in head_qkvdo(b, h, B, H, T, D, seed + 1, outlier_frac=0.01))
    rot = None
    if hadamard:
        signs = generate_hadamard_signs(D, 0).numpy()
        q, k = (bf16_round(rotate_fp32(x, signs)) for x in (q, k))
        rot = rotation_matrix(signs)
    return q, k, v, do, mask, D ** -0.5, rot


def main(argv):
    heads = [tuple(int(x) for x in a.split(",")) for a in argv] or [(b, h) for b in range(2) for h in range(32)]
    print("head       product  " + "  ".join(f"{f:>8}" for f in FORMS) + "  coupled")
    for b, h in heads:
        r = emulate_head(*config4_head(b, h, hadamard=True))
        for p in PRODUCTS:
            row = "  ".join(f"{r['excess'][(p, f)]:8.2e}" for f in FORMS)
            print(f"({b:d},{h:2d})  {p:>6}  {row}  {r['coupled'].get(p, float('nan')):8.2e}", flush=True)


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    main(sys.argv[1:])
