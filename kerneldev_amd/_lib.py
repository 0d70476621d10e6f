"""ctypes binding of ``libkdattn.so`` (the gfx950 C ABI in ``include/kdattn.h``).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already mapped (same SONAME),
i.e. torch's streams and device pointers are valid inside it.  There is no
fallback: if the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

import torch  # noqa: F401  (must precede the dlopen, see module docstring)

LIB_NAME = "libkdattn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

KD_OK, KD_ERR_INVALID, KD_ERR_UNSUPPORTED, KD_ERR_LAUNCH = 0, -1, -2, -3
KD_BF16, KD_F16, KD_F32 = 0, 1, 2
KD_I64, KD_I32 = 0, 1
KD_MODE_FORMULA, KD_MODE_CAUSAL, KD_MODE_ALL = 0, 1, 2
KD_PREC_SPLIT, KD_PREC_SINGLE, KD_PREC_SPLIT3 = 0, 1, 2
KD_NOALLOC_WORKSPACE_FLOATS = 1 << 22

I64x2 = c_int64 * 2
I64x3 = c_int64 * 3


class MetaArgs(ctypes.Structure):
    """Mirror of ``kd_meta_args``."""

    _fields_ = [
        ("in_span", c_void_p), ("in_span_strides", I64x2),
        ("span_id", c_void_p), ("span_id_strides", I64x2),
        ("span_id_dtype", c_int32), ("mode", c_int32),
        ("is_prefix", c_void_p), ("is_prefix_strides", I64x2),
        ("lens", c_void_p), ("lens_stride", c_int64),
        ("B", c_int32), ("T", c_int32), ("D", c_int32), ("pad_", c_int32),
    ]


class AttnArgs(ctypes.Structure):
    """Mirror of ``kd_attn_args``."""

    _fields_ = [
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p),
        ("q_strides", I64x3), ("k_strides", I64x3), ("v_strides", I64x3),
        ("o", c_void_p), ("o_strides", I64x3),
        ("lse", c_void_p),
        ("dout", c_void_p), ("do_strides", I64x3),
        ("dq", c_void_p), ("dk", c_void_p), ("dv", c_void_p),
        ("dq_strides", I64x3), ("dk_strides", I64x3), ("dv_strides", I64x3),
        ("delta", c_void_p), ("o_lo", c_void_p),
        ("q8", c_void_p), ("k8", c_void_p), ("q_scale", c_void_p), ("k_scale", c_void_p),
        ("dqk_signs", c_void_p),
        ("dq_lo", c_void_p), ("dk_lo", c_void_p), ("dv_lo", c_void_p),
        ("B", c_int32), ("H", c_int32), ("T", c_int32), ("D", c_int32),
        ("dtype", c_int32), ("sm_scale", c_float),
        ("precision", c_int32), ("pad_", c_int32),
    ]


class RotArgs(ctypes.Structure):
    """Mirror of ``kd_rot_args``."""

    _fields_ = [
        ("x", c_void_p), ("x_strides", I64x3),
        ("y", c_void_p), ("y_strides", I64x3),
        ("signs", c_void_p), ("amax", c_void_p),
        ("B", c_int32), ("H", c_int32), ("T", c_int32), ("D", c_int32),
        ("dtype", c_int32), ("inverse", c_int32),
    ]


class TokenArgs(ctypes.Structure):
    """Mirror of ``kd_token_args``."""

    _fields_ = [
        ("tokens", c_void_p), ("tokens_strides", c_int64 * 2),
        ("tokens_dtype", c_int32), ("rule", c_int32),
        ("lens", c_void_p), ("lens_stride", c_int64),
        ("B", c_int32), ("T", c_int32), ("D", c_int32), ("pad_", c_int32),
    ]


class QuantArgs(ctypes.Structure):
    """Mirror of ``kd_quant_args``."""

    _fields_ = [
        ("x", c_void_p), ("x_strides", I64x3),
        ("y", c_void_p), ("amax", c_void_p), ("scale", c_void_p),
        ("B", c_int32), ("H", c_int32), ("T", c_int32), ("D", c_int32),
        ("dtype", c_int32), ("pad_", c_int32),
    ]


class SpanArgs(ctypes.Structure):
    """Mirror of ``kd_span_args``."""

    _fields_ = [
        ("tokens", c_void_p), ("tokens_strides", c_int64 * 2), ("tokens_dtype", c_int32), ("dtype", c_int32),
        ("h", c_void_p), ("h_strides", c_int64 * 2),
        ("B", c_int32), ("T", c_int32), ("D", c_int32), ("n_spans", c_int32),
        ("scores", c_void_p), ("h_ctx", c_void_p), ("h_spans", c_void_p),
        ("span_lo", c_void_p), ("span_hi", c_void_p), ("mask_pos", c_void_p),
        ("dscores", c_void_p), ("dh", c_void_p), ("dh_strides", c_int64 * 2),
    ]


# name -> (restype, argtypes); every symbol include/kdattn.h declares
SIGNATURES = {
    "kd_version": (c_int, []),
    "kd_last_error_string": (c_char_p, []),
    "kd_struct_sizes": (None, [POINTER(c_size_t), POINTER(c_size_t)]),
    "kd_struct_sizes2": (None, [POINTER(c_size_t), POINTER(c_size_t)]),
    "kd_struct_sizes3": (None, [POINTER(c_size_t)]),
    "kd_struct_sizes4": (None, [POINTER(c_size_t)]),
    "kd_span_scores": (c_int, [POINTER(SpanArgs), c_void_p]),
    "kd_span_scores_bwd": (c_int, [POINTER(SpanArgs), c_void_p]),
    "kd_plan_build_tokens": (c_int, [POINTER(TokenArgs), c_void_p, c_int64, c_void_p]),
    "kd_hadamard": (c_int, [POINTER(RotArgs), c_void_p]),
    "kd_quant_fp8": (c_int, [POINTER(QuantArgs), c_void_p]),
    "kd_absmax": (c_int, [POINTER(QuantArgs), c_void_p, c_void_p]),
    "kd_plan_bytes": (c_int64, [c_int32, c_int32, c_int32]),
    "kd_plan_layout": (c_int, [c_int32, c_int32, c_int32, POINTER(c_int64)]),
    "kd_plan_build": (c_int, [POINTER(MetaArgs), c_void_p, c_int64, c_void_p]),
    "kd_attn_fwd": (c_int, [POINTER(AttnArgs), c_void_p, c_int64, c_void_p]),
    "kd_attn_bwd_delta": (c_int, [POINTER(AttnArgs), c_void_p]),
    "kd_attn_bwd_dq": (c_int, [POINTER(AttnArgs), c_void_p, c_int64, c_void_p]),
    "kd_attn_bwd_dq_delta": (c_int, [POINTER(AttnArgs), c_void_p, c_int64, c_void_p]),
    "kd_attn_bwd_dkdv": (c_int, [POINTER(AttnArgs), c_void_p, c_int64, c_void_p]),
    "kd_attn_bwd": (c_int, [POINTER(AttnArgs), c_void_p, c_int64, c_void_p]),
    "kd_attn_bwd_noalloc": (c_int, [POINTER(AttnArgs), c_void_p, c_int64, c_void_p]),
    "kd_mask_dense": (c_int, [c_void_p, c_int64, c_int32, c_int32, c_int32, c_int32, c_void_p,
                              POINTER(c_int64), c_void_p]),
    "kd_tile_masks": (c_int, [c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
}

_lib = None


class KernelError(RuntimeError):
    pass


def load():
    """Load (once) and return the ctypes library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build the gfx950 extension first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ms, as_ = c_size_t(), c_size_t()
    lib.kd_struct_sizes(ctypes.byref(ms), ctypes.byref(as_))
    rs, qs = c_size_t(), c_size_t()
    lib.kd_struct_sizes2(ctypes.byref(rs), ctypes.byref(qs))
    ts, ss = c_size_t(), c_size_t()
    lib.kd_struct_sizes3(ctypes.byref(ts))
    lib.kd_struct_sizes4(ctypes.byref(ss))
    if (ms.value != ctypes.sizeof(MetaArgs) or as_.value != ctypes.sizeof(AttnArgs)
            or rs.value != ctypes.sizeof(RotArgs) or qs.value != ctypes.sizeof(QuantArgs)
            or ts.value != ctypes.sizeof(TokenArgs) or ss.value != ctypes.sizeof(SpanArgs)):
        raise ImportError(
            f"struct layout mismatch: C meta={ms.value} attn={as_.value} rot={rs.value} quant={qs.value} "
            f"tokens={ts.value} span={ss.value}, ctypes meta={ctypes.sizeof(MetaArgs)} "
            f"attn={ctypes.sizeof(AttnArgs)} rot={ctypes.sizeof(RotArgs)} quant={ctypes.sizeof(QuantArgs)} "
            f"tokens={ctypes.sizeof(TokenArgs)} span={ctypes.sizeof(SpanArgs)}")
    _lib = lib
    return lib


def check(status: int, what: str):
    if status != KD_OK:
        msg = load().kd_last_error_string().decode(errors="replace")
        if status in (KD_ERR_INVALID, KD_ERR_UNSUPPORTED):
            raise ValueError(f"{what}: {msg}")
        raise KernelError(f"{what}: {msg} (status {status})")


def plan_ref(plan) -> tuple:
    """``(pointer, size in bytes)`` of a plan tensor, the pair every plan-taking
    entry point receives (the library refuses a plan smaller than its shape needs)."""
    return c_void_p(plan.data_ptr()), c_int64(plan.numel() * plan.element_size())


def plan_bytes(B: int, T: int, D: int) -> int:
    n = load().kd_plan_bytes(B, T, D)
    if n < 0:
        raise ValueError("invalid plan shape")
    return int(n)


def plan_nbytes(B, T, D):
    """kd_plan_bytes restated in integer arithmetic that also accepts torch
    SymInts (the custom ops' fake kernels size the plan with it under
    torch.compile with dynamic shapes).  Sections in kd_plan_layout's order,
    each rounded up to 256 bytes; the work lists group two 64-row tiles."""
    def r(x):
        return ((x + 255) // 256) * 256

    nT = (T + 63) // 64
    nb = (nT + 1) // 2  # blocks of the forward, dQ and dK/dV lists
    BT, BTT = B * T, B * nT * nT
    return (r(BT * 4) + r(BT * 4) + r(BT * 4) + r(BT * 8) + r(B * 4) + r(BT) + r(BT * 8) + r(BT)
            + r(BTT) + r(BTT * 4)
            + 3 * (r(B * nb * nT * 4) + r(B * nb * 4))
            + 3 * r(B * nb * 4))


PLAN_FIELDS = ("codes", "rep", "cls", "nnz", "fwd_list", "fwd_count", "dq_list", "dq_count",
               "dkdv_list", "dkdv_count", "nT", "fwd_group", "dq_group", "dkdv_group",
               "n_fwd_blocks", "n_dq_blocks", "n_dkdv_blocks", "fwd_order", "dq_order", "dkdv_order")


def plan_layout(B: int, T: int, D: int) -> dict:
    off = (c_int64 * len(PLAN_FIELDS))()
    check(load().kd_plan_layout(B, T, D, off), "kd_plan_layout")
    return dict(zip(PLAN_FIELDS, [int(x) for x in off]))
