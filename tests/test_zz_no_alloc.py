"""GPU: kd_attn_bwd_noalloc (workspace in the library's device array) against
kd_attn_bwd (caller's workspace), through the C ABI, on two calls in a row --
the second smaller -- so the array's contents from the first call must not
leak into the second (bf16 and fp32 inputs, and fp8 scores at d = 64 and
256).  Both run the same kernels on the same inputs, so dQ, dK and dV must
agree bit for bit.  And captured in a HIP graph on its first
call in a process (the call that resolves the array's device address, in a
child process so that no earlier test has made it), replayed three times,
each replay bit-equal to the eager kd_attn_bwd.
"""
import ctypes
import os
import subprocess
import sys
import textwrap

import pytest
import torch

from kerneldev_amd import _lib
from kerneldev_amd.attention import _attn_args, _fwd_op, _ptr, _set_fp8, _strides3
from kerneldev_amd.synth import CONFIG3_LAYOUT, cocktail_batch, qkvdo

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _backward_both(dev, B, H, T, D, seed, dtype=torch.bfloat16, fp8=False):
    tokens, in_span, span_id, is_prefix = cocktail_batch(B, 1024, CONFIG3_LAYOUT, seed=seed)
    meta = [x[:, :T].to(dev) for x in (in_span, span_id, is_prefix)]
    q, k, v, do = (x.to(dev) for x in qkvdo(B, H, T, D, seed=seed + 1, dtype=dtype))
    sc = D ** -0.5
    fp32 = dtype == torch.float32  # (fp32 O carries no residual)
    # fp8: the forward op's e4m3 copies of Q and K and their scales feed both backward calls
    o, lse, plan, o_lo, _, _, *q8k8 = _fwd_op(q, k, v, None, *meta, sc, 0, not fp32, quant_fp8=fp8)
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for noalloc in (False, True):
        dq, dk, dv = torch.full_like(q, float("nan")), torch.full_like(k, float("nan")), torch.full_like(v, float("nan"))
        a = _attn_args(q, k, v, sc)
        a.o, a.o_strides, a.lse = o.data_ptr(), _strides3(o), lse.data_ptr()
        a.o_lo = None if fp32 else o_lo.data_ptr()
        a.dout, a.do_strides = do.data_ptr(), _strides3(do)
        a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
        a.dq_strides, a.dk_strides, a.dv_strides = _strides3(dq), _strides3(dk), _strides3(dv)
        _set_fp8(a, tuple(q8k8) if fp8 else None)
        if noalloc:
            a.delta = None  # ignored: the library's own workspace is used
            _lib.check(lib.kd_attn_bwd_noalloc(ctypes.byref(a), *_lib.plan_ref(plan), stream), "kd_attn_bwd_noalloc")
        else:
            delta = torch.empty((2, B, H, T), dtype=torch.float32, device=dev)
            a.delta = delta.data_ptr()
            _lib.check(lib.kd_attn_bwd(ctypes.byref(a), *_lib.plan_ref(plan), stream), "kd_attn_bwd")
        torch.cuda.synchronize()
        outs.append((dq, dk, dv))
    return outs


def test_noalloc_backward_matches_allocating_entry_point(dev):
    cases = ((2, 4, 1024, 128, 80, torch.bfloat16, False), (1, 2, 300, 64, 82, torch.bfloat16, False),
             (1, 3, 700, 256, 84, torch.float32, False), (1, 2, 200, 16, 86, torch.float32, False),
             (1, 2, 600, 256, 88, torch.bfloat16, True), (2, 1, 300, 64, 90, torch.bfloat16, True))
    for B, H, T, D, seed, dtype, fp8 in cases:
        print(f"noalloc backward B={B} H={H} T={T} D={D} {dtype} fp8={fp8}", flush=True)
        ref, got = _backward_both(dev, B, H, T, D, seed, dtype, fp8)
        for name, x, y in zip(("dq", "dk", "dv"), ref, got):
            assert torch.isfinite(y).all(), name
            assert torch.equal(x, y), f"{name} differs (B={B} T={T} D={D})"


def test_noalloc_rejects_oversized_workspace():
    lib = _lib.load()
    a = _lib.AttnArgs()
    a.B, a.H, a.T, a.D = 64, 64, 8192, 128  # 2 B H T floats > KD_NOALLOC_WORKSPACE_FLOATS
    assert 2 * a.B * a.H * a.T > _lib.KD_NOALLOC_WORKSPACE_FLOATS
    assert lib.kd_attn_bwd_noalloc(ctypes.byref(a), None, 0, None) == _lib.KD_ERR_UNSUPPORTED
    assert "exceeds the workspace" in lib.kd_last_error_string().decode()


CHILD = textwrap.dedent("""
    import ctypes, sys
    import torch
    sys.path.insert(0, ROOT)
    from kerneldev_amd import _lib
    from kerneldev_amd.attention import _attn_args, _fwd_op, _strides3
    from kerneldev_amd.synth import CONFIG3_LAYOUT, cocktail_batch, qkvdo

    dev = torch.device("cuda:0")
    B, H, T, D = 2, 3, 700, 64
    _, in_span, span_id, is_prefix = cocktail_batch(B, 1024, CONFIG3_LAYOUT, seed=91)
    meta = [x[:, :T].contiguous().to(dev) for x in (in_span, span_id, is_prefix)]
    q, k, v, do = (x.to(dev) for x in qkvdo(B, H, T, D, seed=92))
    sc = D ** -0.5
    o, lse, plan, o_lo, *_ = _fwd_op(q, k, v, None, *meta, sc, 0, True)
    lib = _lib.load()

    def args(dq, dk, dv, delta):
        a = _attn_args(q, k, v, sc)
        a.o, a.o_strides, a.lse, a.o_lo = o.data_ptr(), _strides3(o), lse.data_ptr(), o_lo.data_ptr()
        a.dout, a.do_strides = do.data_ptr(), _strides3(do)
        a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
        a.dq_strides, a.dk_strides, a.dv_strides = _strides3(dq), _strides3(dk), _strides3(dv)
        a.delta = None if delta is None else delta.data_ptr()
        return a

    want = [torch.empty_like(q) for _ in range(3)]
    delta = torch.empty((2, B, H, T), dtype=torch.float32, device=dev)
    a_ref = args(*want, delta)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.kd_attn_bwd(ctypes.byref(a_ref), *_lib.plan_ref(plan), st), "kd_attn_bwd")
    torch.cuda.synchronize()

    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    a = args(*got, None)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):  # the first kd_attn_bwd_noalloc call of this process
        cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.kd_attn_bwd_noalloc(ctypes.byref(a), *_lib.plan_ref(plan), cs), "kd_attn_bwd_noalloc")
    for rep in range(3):
        for t in got:
            t.fill_(float("nan"))
        other = torch.randn(1 << 20, device=dev).sum()  # eager work between the replays
        g.replay()
        torch.cuda.synchronize()
        for name, x, y in zip(("dq", "dk", "dv"), want, got):
            assert torch.equal(x, y), f"replay {rep}: {name} differs"
        print(f"replay {rep} bit-equal", flush=True)
    print("ok", flush=True)
""").replace("ROOT", repr(ROOT))


def test_noalloc_first_call_inside_graph_capture(dev):
    print("child: kd_attn_bwd_noalloc first called inside a graph capture", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD], capture_output=True, text=True, timeout=150)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), f"child exited {r.returncode}"
