"""GPU: the kdattn custom ops trace like the reference's (original_kernel.py:2035-2036
runs its op inside torch.compile(fullgraph=True, dynamic=True), with fake
implementations at :1781-1803 and :1901-1923).

* torch.library.opcheck on every kdattn op: kdattn::fwd (also quantising Q and K
  for fp8 scores), kdattn::bwd, kdattn::fwd_x3, kdattn::bwd_x3, kdattn::rot,
  kdattn::rot_amax, kdattn::quant, kdattn::absmax, kdattn::span_fwd and kdattn::span_bwd:
  schema, autograd registration, fake kernels against the real outputs, and
  AOT dispatch with dynamic shapes.
* flash_attention under torch.compile(fullgraph=True), static and dynamic
  shapes, forward and backward: bit for bit the eager result.
"""
import pytest
import torch

from kerneldev_amd import flash_attention, generate_hadamard_signs
from kerneldev_amd.attention import _bwd_op, _bwd_x3_op, _fwd_op, _fwd_x3_op, _lib
from kerneldev_amd.hadamard import _absmax_op, _quant_op, _rot_amax_op, _rot_op
from kerneldev_amd.span_head import _span_bwd_op, _span_fwd_op, max_spans
from kerneldev_amd.synth import CONFIG3_LAYOUT, cocktail_batch, qkvdo

pytestmark = pytest.mark.gpu


def _inputs(dev, B=2, H=2, T=320, D=64, seed=90):
    _, in_span, span_id, is_prefix = cocktail_batch(B, 1024, CONFIG3_LAYOUT, seed=seed)
    meta = [x[:, :T].contiguous().to(dev) for x in (in_span, span_id, is_prefix)]
    q, k, v, do = (x.to(dev) for x in qkvdo(B, H, T, D, seed=seed + 1))
    return q, k, v, do, meta


def test_opcheck_forward_and_backward_ops(dev):
    q, k, v, do, meta = _inputs(dev)
    sc = q.shape[-1] ** -0.5
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    print("opcheck kdattn::fwd", flush=True)
    torch.library.opcheck(_fwd_op, (qg, kg, vg, None, *meta, sc, _lib.KD_MODE_FORMULA, True))
    o, lse, plan, o_lo, *_ = _fwd_op(q, k, v, None, *meta, sc, _lib.KD_MODE_FORMULA, True)
    print("opcheck kdattn::bwd", flush=True)
    torch.library.opcheck(_bwd_op, (q, k, v, o, lse, do, plan, sc, o_lo))


@pytest.mark.parametrize("D,rotate", [(128, True), (128, False), (256, False)])
def test_opcheck_forward_op_with_fp8_scores(dev, D, rotate):
    """kdattn::fwd quantising Q and K itself (quant_fp8): the e4m3 copies and scales it returns
    come after its fused rotation's absmax, or from kd_absmax without one."""
    q, k, v, do, meta = _inputs(dev, D=D)
    sc = D ** -0.5
    signs = generate_hadamard_signs(D, 1, device=dev) if rotate else None
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    print(f"opcheck kdattn::fwd with fp8 scores, D={D} rotate={rotate}", flush=True)
    torch.library.opcheck(_fwd_op, (qg, kg, vg, None, *meta, sc, _lib.KD_MODE_FORMULA, True),
                          {"signs": signs, "quant_fp8": True})


def test_opcheck_fp32_bf16x3_ops(dev):
    q, k, v, do, meta = _inputs(dev)
    q, k, v, do = (x.float() for x in (q, k, v, do))
    sc = q.shape[-1] ** -0.5
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    print("opcheck kdattn::fwd_x3", flush=True)
    torch.library.opcheck(_fwd_x3_op, (qg, kg, vg, None, *meta, sc, _lib.KD_MODE_FORMULA))
    o, lse, plan = _fwd_x3_op(q, k, v, None, *meta, sc, _lib.KD_MODE_FORMULA)
    print("opcheck kdattn::bwd_x3", flush=True)
    torch.library.opcheck(_bwd_x3_op, (q, k, v, o, lse, do, plan, sc))


def test_opcheck_rotation_and_quantiser_ops(dev):
    q, *_ = _inputs(dev, D=128)
    signs = generate_hadamard_signs(128, 3, device=dev)
    print("opcheck kdattn::rot", flush=True)
    torch.library.opcheck(_rot_op, (q.clone().requires_grad_(True), signs, False))
    amax = q.float().abs().amax(dim=(2, 3)).contiguous()
    print("opcheck kdattn::quant", flush=True)
    torch.library.opcheck(_quant_op, (q, amax))
    print("opcheck kdattn::absmax", flush=True)
    torch.library.opcheck(_absmax_op, (q,))
    print("opcheck kdattn::rot_amax", flush=True)
    torch.library.opcheck(_rot_amax_op, (q.clone().requires_grad_(True), signs))


def test_opcheck_span_head_ops(dev):
    tokens, *_ = cocktail_batch(2, 1024, CONFIG3_LAYOUT, seed=91)
    tokens = tokens.to(dev)
    h = torch.randn(2, 1024, 64, generator=torch.Generator().manual_seed(92)).to(torch.bfloat16).to(dev)
    n = max_spans(tokens)
    print("opcheck kdattn::span_fwd", flush=True)
    torch.library.opcheck(_span_fwd_op, (tokens, h.clone().requires_grad_(True), n))
    scores, h_ctx, h_spans, lo, hi, mpos = _span_fwd_op(tokens, h, n)
    print("opcheck kdattn::span_bwd", flush=True)
    torch.library.opcheck(_span_bwd_op, (tokens, h, torch.randn_like(scores), h_ctx, h_spans, lo, hi, mpos))


def _fwd_bwd(fn, q, k, v, do, meta):
    qg, kg, vg = (x.clone().requires_grad_(True) for x in (q, k, v))
    o, lse = fn(qg, kg, vg, *meta)
    o.backward(do)
    torch.cuda.synchronize()
    return o.detach(), lse.detach(), qg.grad, kg.grad, vg.grad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dynamic", [False, True])
def test_compiled_flash_attention_matches_eager(dev, dynamic, dtype):
    def attn(q, k, v, in_span, span_id, is_prefix):
        return flash_attention(q, k, v, in_span=in_span, span_id=span_id, is_prefix=is_prefix, return_lse=True)

    torch._dynamo.reset()
    compiled = torch.compile(attn, fullgraph=True, dynamic=dynamic)
    for T in (320, 200):  # a second length re-uses (dynamic) or re-traces (static) the graph
        q, k, v, do, meta = _inputs(dev, T=T)
        q, k, v, do = (x.to(dtype) for x in (q, k, v, do))
        print(f"torch.compile dynamic={dynamic} {dtype} T={T}", flush=True)
        want = _fwd_bwd(attn, q, k, v, do, meta)
        got = _fwd_bwd(compiled, q, k, v, do, meta)
        for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), got, want):
            assert torch.equal(x, y), f"{name} differs between compiled and eager (T={T})"


def test_timing_module_runs(dev):
    """kerneldev_amd.timing (the fwd+bwd timer for shapes outside the benchmark) runs end to end."""
    from kerneldev_amd.timing import time_step

    for dtype in (torch.bfloat16, torch.float32):
        s, nnz = time_step(1, 2, 200, 64, dtype, steps=1, warmup=1)
        assert s > 0 and nnz == 2 * 200 * 201 // 2


@pytest.mark.parametrize("case", ["bf16_d64", "fp32_d32_tf32"])
def test_hip_graph_capture_and_replay(dev, case):
    """flash_attention forward + backward captured in one HIP graph (torch.cuda.CUDAGraph) and
    replayed three times, with eager work on other inputs between the replays: every replay
    gives the eager result bit for bit (no host synchronisation or allocation outside the
    graph's pool inside the ops).  fp32 inputs at precision "tf32" and head dim 32 take the
    bf16x3 ops, whose backward forms its workspace with torch operations."""
    q, k, v, do, meta = _inputs(dev)
    if case == "fp32_d32_tf32":
        q, k, v, do = (x[..., :32].float().contiguous() for x in (q, k, v, do))
    qs, ks, vs = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    dos = do.clone()

    def step():
        for t in (qs, ks, vs):
            t.grad = None
        o = flash_attention(qs, ks, vs, in_span=meta[0], span_id=meta[1], is_prefix=meta[2], precision="tf32")
        o.backward(dos)
        return o

    o_eager = step().detach().clone()
    want = [o_eager] + [t.grad.clone() for t in (qs, ks, vs)]
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up off the default stream, as graph capture requires
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        o_g = step()
    for rep in range(3):
        other = flash_attention(*(x.flip(2).contiguous() for x in (q, k, v)))  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        got = [o_g] + [t.grad for t in (qs, ks, vs)]
        for name, a, b in zip(("o", "dq", "dk", "dv"), got, want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs"
        assert torch.isfinite(other).all()
