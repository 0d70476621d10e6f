"""GPU: kd_attn_bwd_noalloc captured in a HIP graph on its first call in the
process (the call that resolves the workspace array's device address), then
replayed, each replay bit-equal to kd_attn_bwd run eagerly with a caller-owned
workspace.  Runs in a child process so that no earlier test has made that
first call."""
import os
import subprocess
import sys
import textwrap

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

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
