"""GPU: sequences past config 4's length (T = 16384 cocktail-party, T = 65536 and 196608 causal).

Where the sizes grow -- 256 and 1024 key tiles per row, lists of that length
in the plan, per-head byte offsets of 8-16 MiB in the buffer loads -- the
kernels are checked against a plain PyTorch fp32 reference computed on the GPU
one chunk of query rows at a time (one chunk's scores in memory), with the
oracle's dense mask (``oracle/mask.py``) for the cocktail-party case and the
closed-form causal / ``lens`` mask for the causal one (the oracle's own
special case, pinned in ``test_oracle_mask.py``).

Bar: ``helpers.assert_close`` (per element beyond one output ulp <= 2e-2,
rel-RMS <= 1e-2); LSE on the finite rows with the -inf pattern exact.
"""
import math

import numpy as np
import pytest
import torch

from helpers import assert_close, oracle_mask
from kerneldev_amd import flash_attention
from kerneldev_amd.synth import CocktailLayout, cocktail_batch, qkvdo

pytestmark = pytest.mark.gpu

CHUNK = 4096  # query rows per reference chunk


def _reference(q, k, v, do, scale, mask_rows):
    """fp32 forward + backward of one head; mask_rows(r0, r1) -> ([r1 - r0, kmax] bool, kmax)."""
    T, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(T, device=q.device)
    dq = torch.empty_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    for r0 in range(0, T, CHUNK):
        r1 = min(T, r0 + CHUNK)
        m_, kmax = mask_rows(r0, r1)
        kk, vv = k[:kmax], v[:kmax]
        s = torch.mm(q[r0:r1], kk.t().contiguous()).mul_(scale).masked_fill_(~m_, -math.inf)
        m = s.amax(dim=1, keepdim=True)
        m0 = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = s.sub_(m0).exp_()
        l = p.sum(dim=1, keepdim=True)
        p.div_(l.clamp_min(1e-30))
        oc = torch.mm(p, vv)
        o[r0:r1] = oc
        lse[r0:r1] = torch.where(l[:, 0] > 0, (m0[:, 0] + torch.log(l[:, 0])) / math.log(2.0),
                                 torch.full_like(l[:, 0], -math.inf))
        delta = (do[r0:r1] * oc).sum(dim=1, keepdim=True)
        ds = torch.mm(do[r0:r1], vv.t().contiguous()).sub_(delta).mul_(p)
        dq[r0:r1] = torch.mm(ds, kk).mul_(scale)
        dk[:kmax] += torch.mm(ds.t().contiguous(), q[r0:r1]).mul_(scale)
        dv[:kmax] += torch.mm(p.t().contiguous(), do[r0:r1])
    return o, lse, dq, dk, dv


def _check(got, refs):
    o, lse, dq, dk, dv = refs
    fin = torch.isfinite(lse)
    assert torch.equal(torch.isinf(got["lse"]), torch.isinf(lse)), "LSE -inf pattern differs"
    assert_close("lse", got["lse"][fin], lse[fin], out_dtype=torch.float32)
    for name, r in (("o", o), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert_close(name, got[name].float(), r, out_dtype=torch.bfloat16)


def _run(q, k, v, do, **kw):
    ql, kl, vl = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    o, lse = flash_attention(ql, kl, vl, return_lse=True, **kw)
    o.backward(do)
    torch.cuda.synchronize()
    return {"o": o.detach(), "lse": lse.detach(), "dq": ql.grad, "dk": kl.grad, "dv": vl.grad}


def test_cocktail_16k(dev):
    """A cocktail-party row twice config 4's: 512-byte prefix, 4096 context, 32-80 spans."""
    T, H, D = 16384, 2, 128
    layout = CocktailLayout((512, 512), (4096, 4096), (32, 80), (64, 192))
    tokens, in_span, span_id, is_prefix = cocktail_batch(1, T, layout, seed=5)
    q, k, v, do = qkvdo(1, H, T, D, seed=6)
    print(f"cocktail B=1 H={H} T={T} D={D}: {int(in_span.sum())} span tokens; kernels", flush=True)
    meta = dict(in_span=in_span.to(dev), span_id=span_id.to(dev), is_prefix=is_prefix.to(dev))
    qd, kd, vd, dod = (x.to(dev) for x in (q, k, v, do))
    got = _run(qd, kd, vd, dod, causal=True, **meta)
    print("  oracle mask", flush=True)
    inp = dict(q=q, in_span=in_span, span_id=span_id, is_prefix=is_prefix, causal=True)
    mask = torch.from_numpy(np.ascontiguousarray(oracle_mask(inp, T)[0])).to(dev)
    for h in range(H):
        print(f"  reference head {h}", flush=True)
        refs = _reference(qd[0, h].float(), kd[0, h].float(), vd[0, h].float(), dod[0, h].float(), D ** -0.5,
                          lambda r0, r1: (mask[r0:r1], T))
        _check({n: t[0, h] for n, t in got.items()}, refs)


def test_causal_lens_64k(dev):
    """Causal at T = 65536 with lens = 61000: rows and keys past lens are masked, their rows give O = 0."""
    T, H, D, n = 65536, 1, 64, 61000
    q, k, v, do = (x.to(dev) for x in qkvdo(1, H, T, D, seed=7, scale=D ** -0.25))
    lens = torch.tensor([n], dtype=torch.int32, device=dev)
    print(f"causal B=1 H={H} T={T} D={D} lens={n}: kernels", flush=True)
    got = _run(q, k, v, do, causal=True, lens=lens)
    cols = torch.arange(T, device=dev)

    def mask_rows(r0, r1):  # causal & i < n & j < n; keys past r1 are masked for every row here
        rows = torch.arange(r0, r1, device=dev)[:, None]
        kmax = min(r1, T)
        c = cols[None, :kmax]
        return (rows >= c) & (rows < n) & (c < n), kmax

    print("  reference", flush=True)
    refs = _reference(q[0, 0].float(), k[0, 0].float(), v[0, 0].float(), do[0, 0].float(), D ** -0.5, mask_rows)
    _check({nm: t[0, 0] for nm, t in got.items()}, refs)
    assert got["o"][0, 0, n:].abs().max().item() == 0.0


def test_causal_196k(dev):
    """Causal at T = 196608 (3072 key tiles per row, a 3072 x 3072 class map and lists of up to 3072
    entries per block), past where a per-tile mask store would need more than 32 bits of bytes."""
    T, H, D = 196608, 1, 64
    q, k, v, do = (x.to(dev) for x in qkvdo(1, H, T, D, seed=8, scale=D ** -0.25))
    print(f"causal B=1 H={H} T={T} D={D}: kernels", flush=True)
    got = _run(q, k, v, do, causal=True)
    cols = torch.arange(T, device=dev)

    def mask_rows(r0, r1):
        rows = torch.arange(r0, r1, device=dev)[:, None]
        return rows >= cols[None, :r1], r1

    print("  reference", flush=True)
    refs = _reference(q[0, 0].float(), k[0, 0].float(), v[0, 0].float(), do[0, 0].float(), D ** -0.5, mask_rows)
    _check({nm: t[0, 0] for nm, t in got.items()}, refs)
