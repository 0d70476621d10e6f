"""CPU: the C-ABI library loads, exports every symbol include/kdattn.h declares,
and rejects bad arguments with a status before touching the GPU; the Python
boundary validates like the reference's adapter (original_kernel.py:1720-1726)
but raises ValueError.
"""
import ctypes
import os
import re

import pytest
import torch

from kerneldev_amd import _lib, flash_attention
from kerneldev_amd.attention import REFERENCE_HEAD_DIMS

# a plan size no shape in these tests exceeds (the calls fail on other arguments first)
BIG = 1 << 40

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "kdattn.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?(?:int|int64_t|void|char)\s*\*?\s*(kd_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 13, names
    for n in names:
        assert hasattr(lib, n), f"{n} missing from {_lib.LIB_PATH}"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_struct_layouts_and_version():
    lib = _lib.load()  # load() itself checks the three struct sizes
    # 3.0: plan sizes at the boundary; 3.1: the dK/dV work order; 3.2: kd_absmax; 3.3: fp8 scores at d = 256
    assert lib.kd_version() >= 30300
    assert ctypes.sizeof(_lib.AttnArgs) % 8 == 0


def test_plan_sizes_and_layout_offsets():
    lib = _lib.load()
    assert lib.kd_plan_bytes(0, 10, 64) < 0
    L = _lib.plan_layout(2, 8192, 128)
    assert L["nT"] == 128 and L["n_fwd_blocks"] == 64 and L["fwd_group"] == 2
    offs = [L[k] for k in _lib.PLAN_FIELDS[:10]]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)
    assert _lib.plan_bytes(2, 8192, 128) > L["dkdv_count"]
    tail = [L[k] for k in ("dkdv_count", "fwd_order", "dq_order", "dkdv_order")]
    assert tail == sorted(tail) and all(o % 256 == 0 for o in tail)
    assert _lib.plan_bytes(2, 8192, 128) >= L["dkdv_order"] + 4 * 2 * L["n_dkdv_blocks"]


def test_bad_arguments_return_status_without_gpu():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    assert lib.kd_attn_fwd(None, null, 0, null) == _lib.KD_ERR_INVALID
    assert "NULL" in lib.kd_last_error_string().decode()
    a = _lib.AttnArgs()
    a.B, a.H, a.T, a.D, a.dtype, a.sm_scale = 1, 1, 16, 96, _lib.KD_BF16, 0.1
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_UNSUPPORTED
    a.D, a.dtype = 64, 5
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_UNSUPPORTED
    a.D, a.dtype, a.dqk_signs = 256, _lib.KD_BF16, 64  # the fused un-rotation is built for D 64 / 128
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_UNSUPPORTED
    assert "dqk_signs" in lib.kd_last_error_string().decode()
    a.dqk_signs = None
    a.D = 64
    a.sm_scale = float("nan")
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_INVALID
    a.sm_scale = 0.125
    a.precision = 3  # KD_PREC_SPLIT (0), KD_PREC_SINGLE (1), KD_PREC_SPLIT3 (2) only
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_INVALID
    assert "precision" in lib.kd_last_error_string().decode()
    a.precision = _lib.KD_PREC_SPLIT3
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_INVALID  # q is NULL
    a.precision = _lib.KD_PREC_SPLIT
    a.q = a.k = a.v = a.o = 32
    a.q_strides[:] = [1024, 1024, 8]  # t stride < head dim: rows overlap
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_INVALID
    assert "overlap" in lib.kd_last_error_string().decode()
    a.q_strides[:] = [1024, 1024, 64]
    a.q8 = 64  # fp8 operands: q8 without k8, then fp16 inputs (fp8 scores are built for bf16 at 64 / 128 / 256)
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_INVALID
    assert "q8 and k8" in lib.kd_last_error_string().decode()
    a.k8 = 64
    a.dtype = _lib.KD_F16
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_UNSUPPORTED
    assert "bf16" in lib.kd_last_error_string().decode()
    a.dtype = _lib.KD_BF16
    a.D = 128
    a.q_strides[:] = [1024, 1024, 128]
    a.precision = _lib.KD_PREC_SPLIT3  # the three-part split is not built with fp8 scores
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_UNSUPPORTED
    assert "SPLIT3" in lib.kd_last_error_string().decode()
    a.precision = _lib.KD_PREC_SPLIT
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_INVALID  # no scales
    assert "scale" in lib.kd_last_error_string().decode()
    a.D = 256  # head dim 256 passes the fp8 checks as far as the scales too
    a.q_strides[:] = [4096, 4096, 256]
    assert lib.kd_attn_fwd(ctypes.byref(a), ctypes.c_void_p(16), BIG, null) == _lib.KD_ERR_INVALID
    assert "scale" in lib.kd_last_error_string().decode()
    b = _lib.AttnArgs()  # the backward's rounding-residual outputs: 16-bit MFMA paths only, aligned
    b.B, b.H, b.T, b.D, b.dtype, b.sm_scale = 1, 1, 16, 64, _lib.KD_F32, 0.125
    b.lse, b.delta, b.dq_lo = 64, 64, 64
    assert lib.kd_attn_bwd(ctypes.byref(b), ctypes.c_void_p(256), BIG, null) == _lib.KD_ERR_UNSUPPORTED
    assert "dq_lo" in lib.kd_last_error_string().decode()
    b.dtype, b.dq_lo, b.dv_lo = _lib.KD_BF16, None, 72
    assert lib.kd_attn_bwd(ctypes.byref(b), ctypes.c_void_p(256), BIG, null) == _lib.KD_ERR_INVALID
    assert "aligned" in lib.kd_last_error_string().decode()
    c = _lib.AttnArgs()  # O's rounding residual is for 16-bit O: fp32 inputs with o_lo are refused
    c.B, c.H, c.T, c.D, c.dtype, c.sm_scale = 1, 1, 16, 64, _lib.KD_F32, 0.125
    c.q = c.k = c.v = c.o = c.o_lo = 64
    for st in (c.q_strides, c.k_strides, c.v_strides, c.o_strides):
        st[:] = [1024, 1024, 64]
    assert lib.kd_attn_fwd(ctypes.byref(c), ctypes.c_void_p(256), BIG, null) == _lib.KD_ERR_INVALID
    assert "o_lo" in lib.kd_last_error_string().decode()
    r = _lib.RotArgs()
    r.B, r.H, r.T, r.D, r.dtype = 1, 1, 4, 48, _lib.KD_BF16
    assert lib.kd_hadamard(ctypes.byref(r), null) == _lib.KD_ERR_UNSUPPORTED  # not a power of two
    r.D, r.dtype = 32, 3
    assert lib.kd_hadamard(ctypes.byref(r), null) == _lib.KD_ERR_UNSUPPORTED  # unknown dtype
    r.dtype = _lib.KD_F32
    assert lib.kd_hadamard(ctypes.byref(r), null) == _lib.KD_ERR_INVALID  # signs missing
    qa = _lib.QuantArgs()
    qa.B, qa.H, qa.T, qa.D, qa.dtype = 1, 1, 4, 128, _lib.KD_BF16
    assert lib.kd_quant_fp8(ctypes.byref(qa), null) == _lib.KD_ERR_INVALID  # amax / scale / y missing
    qa.D = 256
    assert lib.kd_quant_fp8(ctypes.byref(qa), null) == _lib.KD_ERR_INVALID  # 256 is built; buffers still missing
    qa.D = 96
    assert lib.kd_quant_fp8(ctypes.byref(qa), null) == _lib.KD_ERR_UNSUPPORTED
    buf = ctypes.c_void_p(256)  # never dereferenced on the host
    assert lib.kd_absmax(ctypes.byref(qa), buf, null) == _lib.KD_ERR_UNSUPPORTED  # head dim 96
    qa.D, qa.dtype = 64, _lib.KD_F32
    assert lib.kd_absmax(ctypes.byref(qa), buf, null) == _lib.KD_ERR_UNSUPPORTED  # 16-bit inputs only
    qa.dtype = _lib.KD_BF16
    assert lib.kd_absmax(ctypes.byref(qa), null, null) == _lib.KD_ERR_INVALID  # amax missing
    assert lib.kd_absmax(ctypes.byref(qa), buf, null) == _lib.KD_ERR_INVALID  # x missing
    m = _lib.MetaArgs()
    m.B, m.T, m.mode = 1, 8, 7
    assert lib.kd_plan_build(ctypes.byref(m), ctypes.c_void_p(256), BIG, null) == _lib.KD_ERR_INVALID
    t = _lib.TokenArgs()
    t.B, t.T, t.D, t.rule = 1, 8, 64, 0
    assert lib.kd_plan_build_tokens(ctypes.byref(t), ctypes.c_void_p(256), BIG, null) == _lib.KD_ERR_INVALID  # no tokens
    t.tokens, t.rule = 64, 9
    assert lib.kd_plan_build_tokens(ctypes.byref(t), ctypes.c_void_p(256), BIG, null) == _lib.KD_ERR_INVALID
    assert "rule" in lib.kd_last_error_string().decode()
    sp = _lib.SpanArgs()
    assert lib.kd_span_scores(None, null) == _lib.KD_ERR_INVALID
    sp.B, sp.T, sp.D, sp.n_spans, sp.dtype = 2, 16, 65537, 3, _lib.KD_BF16
    assert lib.kd_span_scores(ctypes.byref(sp), null) == _lib.KD_ERR_UNSUPPORTED  # D > 65536
    assert lib.kd_span_scores_bwd(ctypes.byref(sp), null) == _lib.KD_ERR_UNSUPPORTED
    sp.B, sp.T, sp.D, sp.n_spans, sp.dtype = 2, 16, 64, 0, _lib.KD_BF16
    assert lib.kd_span_scores(ctypes.byref(sp), null) == _lib.KD_ERR_UNSUPPORTED  # n_spans 0
    sp.n_spans = 3
    assert lib.kd_span_scores(ctypes.byref(sp), null) == _lib.KD_ERR_INVALID  # tokens / h missing
    sp.tokens, sp.h = 64, 128
    sp.tokens_strides[:] = [16, 1]
    sp.h_strides[:] = [1024, 32]  # t stride < D
    assert lib.kd_span_scores(ctypes.byref(sp), null) == _lib.KD_ERR_INVALID
    sp.h_strides[:] = [1024, 64]
    assert lib.kd_span_scores(ctypes.byref(sp), null) == _lib.KD_ERR_INVALID  # outputs missing
    assert lib.kd_span_scores_bwd(ctypes.byref(sp), null) == _lib.KD_ERR_INVALID  # dscores / dh missing
    assert "dh" in lib.kd_last_error_string().decode()


def test_python_boundary_validation():
    q = torch.zeros(1, 2, 16, 64)
    with pytest.raises(ValueError, match="GPU only"):
        flash_attention(q, q, q)
    with pytest.raises(ValueError, match="head_dim"):
        z = torch.zeros(1, 2, 16, 48)
        flash_attention(z, z, z)
    with pytest.raises(ValueError, match="precision"):
        flash_attention(q, q, q, precision="fp16")
    with pytest.raises(ValueError, match="lens"):
        flash_attention(q, q, q, lens=torch.zeros(1, dtype=torch.int64))
    with pytest.raises(ValueError, match="qk_dtype"):
        flash_attention(q, q, q, qk_dtype="int8")
    with pytest.raises(ValueError, match="fp8"):
        z = torch.zeros(1, 2, 16, 128)
        flash_attention(z, z, z, qk_dtype="fp8_e4m3", precision="ieee")
    assert 32 in REFERENCE_HEAD_DIMS and 256 in REFERENCE_HEAD_DIMS


def test_plan_is_linear_in_tiles_not_elements():
    """No per-element masks: config 4's plan is under 1 MiB, a B=8, L=32768 plan under 64 MiB."""
    assert _lib.plan_bytes(2, 8192, 128) < 1 << 20
    assert _lib.plan_bytes(8, 32768, 128) < 64 << 20


def test_python_plan_size_matches_the_library():
    """plan_nbytes (the fake kernels' SymInt-friendly plan size) == kd_plan_bytes."""
    for B in (1, 2, 3, 8):
        for T in (1, 17, 63, 64, 65, 127, 128, 129, 300, 1024, 8192, 8193):
            for D in REFERENCE_HEAD_DIMS:
                assert _lib.plan_nbytes(B, T, D) == _lib.plan_bytes(B, T, D), (B, T, D)


def test_undersized_plan_is_refused_before_any_launch():
    """Every entry point that reads or writes a plan refuses one smaller than
    kd_plan_bytes of its shape, with KD_ERR_INVALID and a message naming both
    sizes, before anything else is looked at that needs the GPU (there is none
    here: a launch would return KD_ERR_LAUNCH)."""
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    B, H, T, D = 2, 3, 1000, 64
    need = _lib.plan_bytes(B, T, D)
    plan = ctypes.c_void_p(1 << 20)  # aligned stand-in; never dereferenced on the host
    a = _lib.AttnArgs()
    a.B, a.H, a.T, a.D, a.dtype, a.sm_scale = B, H, T, D, _lib.KD_BF16, 0.125
    a.lse, a.delta = 256, 256
    m = _lib.MetaArgs()
    m.B, m.T, m.D, m.mode = B, T, D, _lib.KD_MODE_CAUSAL
    t = _lib.TokenArgs()
    t.B, t.T, t.D, t.tokens = B, T, D, 256
    rows = ctypes.c_void_p(256)
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    calls = {
        "kd_plan_build": lambda n: lib.kd_plan_build(ctypes.byref(m), plan, n, null),
        "kd_plan_build_tokens": lambda n: lib.kd_plan_build_tokens(ctypes.byref(t), plan, n, null),
        "kd_attn_fwd": lambda n: lib.kd_attn_fwd(ctypes.byref(a), plan, n, null),
        "kd_attn_bwd_dq": lambda n: lib.kd_attn_bwd_dq(ctypes.byref(a), plan, n, null),
        "kd_attn_bwd_dq_delta": lambda n: lib.kd_attn_bwd_dq_delta(ctypes.byref(a), plan, n, null),
        "kd_attn_bwd_dkdv": lambda n: lib.kd_attn_bwd_dkdv(ctypes.byref(a), plan, n, null),
        "kd_attn_bwd": lambda n: lib.kd_attn_bwd(ctypes.byref(a), plan, n, null),
        "kd_attn_bwd_noalloc": lambda n: lib.kd_attn_bwd_noalloc(ctypes.byref(a), plan, n, null),
        "kd_tile_masks": lambda n: lib.kd_tile_masks(plan, n, B, T, D, rows, rows, null),
        "kd_mask_dense": lambda n: lib.kd_mask_dense(plan, n, B, H, T, D, rows, st, null),
    }
    for name, call in calls.items():
        for n in (0, need - 1):
            assert call(n) == _lib.KD_ERR_INVALID, name
            msg = lib.kd_last_error_string().decode()
            assert f"plan is {n} bytes" in msg and f"needs {need}" in msg, (name, msg)
        if name.startswith("kd_attn"):
            # with the full size the plan passes, and the call stops at the next
            # argument check, still on the host: q is NULL
            assert call(need) == _lib.KD_ERR_INVALID, name
            msg = lib.kd_last_error_string().decode()
            assert "plan is" not in msg and "q is NULL" in msg, (name, msg)
    # kd_attn_bwd checks both halves before it launches either
    assert calls["kd_attn_bwd"](need - 1) == _lib.KD_ERR_INVALID


def test_c_caller_is_built_against_the_library():
    """The C test caller exists after the build and resolves libkdattn.so through its rpath."""
    import shutil
    import subprocess

    from kerneldev_amd.build import C_ABI_BIN

    assert os.path.exists(C_ABI_BIN)
    if shutil.which("ldd"):
        out = subprocess.run(["ldd", C_ABI_BIN], capture_output=True, text=True).stdout
        assert "libkdattn.so =>" in out and "not found" not in out.split("libkdattn.so")[1].split("\n")[0]


def test_grid_limits_are_refused_before_any_launch():
    """Shapes whose plan launches would exceed a grid dimension (65535 workgroups
    on y and z) get KD_ERR_UNSUPPORTED from the host checks: B > 65535 for the
    plan builds, and kd_tile_masks (one workgroup row per q-tile) past
    T = 65535 * 64."""
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    plan = ctypes.c_void_p(1 << 20)
    m = _lib.MetaArgs()
    m.B, m.T, m.D, m.mode = 65536, 64, 64, _lib.KD_MODE_CAUSAL
    assert lib.kd_plan_build(ctypes.byref(m), plan, BIG, null) == _lib.KD_ERR_UNSUPPORTED
    assert "B must be" in lib.kd_last_error_string().decode()
    t = _lib.TokenArgs()
    t.B, t.T, t.D, t.tokens = 65536, 64, 64, 256
    assert lib.kd_plan_build_tokens(ctypes.byref(t), plan, BIG, null) == _lib.KD_ERR_UNSUPPORTED
    rows = ctypes.c_void_p(256)
    assert lib.kd_tile_masks(plan, BIG, 1, 65535 * 64 + 1, 64, rows, rows, null) == _lib.KD_ERR_UNSUPPORTED
    assert "kd_tile_masks" in lib.kd_last_error_string().decode()
