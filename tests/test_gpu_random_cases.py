"""GPU: seeded random cases through flash_attention against the fp64 oracle.

Each small case draws B, H, T (ragged, 1 .. 640), the head dim, the input dtype,
the precision, the mask mode (causal or not, cocktail-party metadata with
int64 or int32 span ids, lens with empty rows) and Hadamard on or off, runs
forward and backward and checks O, LSE, dQ, dK, dV against the oracle with
the north_star bar (helpers.assert_close; fp32 results against the same bar).
The long cases draw one head with T from 1000 to 4096 the same way.
"""
import random

import pytest
import torch

from helpers import assert_close, oracle_fwd_bwd, oracle_mask, single_key_rows
from kerneldev_amd import flash_attention, generate_hadamard_signs
from kerneldev_amd.synth import CONFIG3_LAYOUT, cocktail_batch, qkvdo
from oracle import hadamard as ref_h

pytestmark = pytest.mark.gpu

N_CASES = 96


def _draw(rng):
    T = rng.choice([1, 7, 64, 65, 127, 200, 333, 512, 640])
    d = rng.choice([16, 32, 64, 64, 128, 128, 256])
    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    precision = rng.choice(["tf32", "ieee", "bf16"]) if dtype != torch.float32 else rng.choice(["tf32", "ieee"])
    return dict(B=rng.choice([1, 2, 3]), H=rng.choice([1, 2]), T=T, d=d, dtype=dtype, precision=precision,
                causal=rng.random() < 0.7, meta=rng.random() < 0.5, sid32=rng.random() < 0.5,
                lens=rng.random() < 0.3, hadamard=rng.random() < 0.3, seed=rng.randrange(1 << 20))


N_LONG = 16


def _draw_long(rng):
    """Longer rows (T 1000-4096, ragged), head dims 64-256, one head."""
    d = rng.choice([64, 128, 128, 256])
    dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    precision = rng.choice(["tf32", "ieee", "bf16"]) if dtype != torch.float32 else rng.choice(["tf32", "ieee"])
    return dict(B=rng.choice([1, 2]), H=1, T=rng.choice([1000, 1170, 2048, 3001, 4096]), d=d, dtype=dtype,
                precision=precision, causal=rng.random() < 0.7, meta=rng.random() < 0.6, sid32=rng.random() < 0.5,
                lens=rng.random() < 0.3, hadamard=rng.random() < 0.3, seed=rng.randrange(1 << 20))


@pytest.mark.parametrize("case", range(N_CASES))
def test_random_case(dev, case):
    _run_case(dev, case, _draw(random.Random(1000 + case)))


@pytest.mark.parametrize("case", range(N_LONG))
def test_random_long_case(dev, case):
    _run_case(dev, case, _draw_long(random.Random(5000 + case)))


def _run_case(dev, case, c):
    B, H, T, d = c["B"], c["H"], c["T"], c["d"]
    print(f"random case {case}: {c}", flush=True)
    q, k, v, do = qkvdo(B, H, T, d, seed=c["seed"], dtype=torch.float32)
    meta = {}
    if c["meta"]:
        _, in_span, span_id, is_prefix = cocktail_batch(B, max(T, 1170), CONFIG3_LAYOUT, seed=c["seed"])
        meta = dict(in_span=in_span[:, :T].contiguous(), span_id=span_id[:, :T].contiguous(),
                    is_prefix=is_prefix[:, :T].contiguous())
        if c["sid32"]:
            meta["span_id"] = meta["span_id"].to(torch.int32)
    lens = None
    if c["lens"]:
        lens = torch.tensor([random.Random(c["seed"] + b).randint(0, T) for b in range(B)], dtype=torch.int32)
    # the operands the kernels see: the inputs rounded to the dtype (the oracle gets the same values)
    q, k, v, do = (x.to(c["dtype"]) for x in (q, k, v, do))
    qd, kd, vd = (x.to(dev).requires_grad_(True) for x in (q, k, v))
    o, lse = flash_attention(qd, kd, vd, causal=c["causal"], return_lse=True, precision=c["precision"],
                             lens=None if lens is None else lens.to(dev),
                             hadamard=c["hadamard"], hadamard_seed=c["seed"] % 7,
                             **{n: t.to(dev) for n, t in meta.items()})
    o.backward(do.to(dev))
    torch.cuda.synchronize()

    inp = dict(q=q, causal=c["causal"], **meta)
    mask = oracle_mask(inp, T, lens=lens)
    qs, ks, rot = q, k, None
    if c["hadamard"]:  # the attention sees Q R, K R rounded to the dtype; gradients map back through R^T
        signs = generate_hadamard_signs(d, c["seed"] % 7).numpy()
        rot = torch.from_numpy(ref_h.rotation_matrix(signs))
        qs = torch.from_numpy(ref_h.rotate_fp32(q.float().numpy(), signs)).to(q.dtype)
        ks = torch.from_numpy(ref_h.rotate_fp32(k.float().numpy(), signs)).to(k.dtype)
    ref = oracle_fwd_bwd(qs, ks, v, do, mask, d ** -0.5)
    if rot is not None:
        ref["dq"] = ref["dq"] @ rot.T
        ref["dk"] = ref["dk"] @ rot.T
    out_dtype = c["dtype"]
    for name, got in (("o", o), ("dq", qd.grad), ("dk", kd.grad), ("dv", vd.grad)):
        assert got.dtype == c["dtype"]
        assert_close(name, got, ref[name], out_dtype=out_dtype, zero_ref_ok=name in ("dq", "dk") and single_key_rows(mask))
    g, r = lse.double().cpu(), ref["lse"].double()
    assert torch.equal(torch.isinf(g), torch.isinf(r)), "LSE -inf pattern differs"
    fin = torch.isfinite(r)
    if fin.any():
        assert_close("lse", g[fin], r[fin], out_dtype=torch.float32)
