"""GPU: config 4 at its full size, every (b, h) head.

The selected-head tests in ``test_gpu_attention.py`` compare against the fp64
oracle on the CPU.  Here all 64 heads of B2 H32 L8192 d128 are checked
against a plain PyTorch fp32 reference computed on the GPU one head at a time,
with the dense mask from the oracle (``oracle/mask.py``) and, for the Hadamard
run, Q' and K' from the oracle's bit-exact rotation (``oracle/hadamard.py``).

Bar: the north_star bar in units of each tensor's magnitude, as in
``helpers.assert_close_scaled`` (config 4 carries 20-sigma outlier channels):
max-abs <= 2e-2 * max(1, max|ref|) and rel-RMS <= 1e-2 over all heads; LSE
(log2 units) on the finite rows, and the -inf pattern exact.
"""
import math

import numpy as np
import pytest
import torch

from helpers import MAX_ABS, REL_RMS, oracle_mask
from kerneldev_amd import flash_attention, generate_hadamard_signs
from kerneldev_amd.synth import config_inputs
from oracle import hadamard as ref_h

pytestmark = pytest.mark.gpu


class _Err:
    """Running max-abs / RMS error of one tensor over the heads."""

    def __init__(self):
        self.max_diff = self.max_ref = self.sq_diff = self.sq_ref = 0.0
        self.n = 0

    def add(self, got, ref):
        d = (got.double() - ref.double()).abs()
        self.max_diff = max(self.max_diff, d.max().item())
        self.max_ref = max(self.max_ref, ref.abs().max().item())
        self.sq_diff += d.pow(2).sum().item()
        self.sq_ref += ref.double().pow(2).sum().item()
        self.n += d.numel()

    def check(self, name):
        scale = max(1.0, self.max_ref)
        rr = math.sqrt(self.sq_diff / max(self.sq_ref, 1e-300))
        print(f"  {name}: max_abs={self.max_diff:.3e} (scaled bar {MAX_ABS * scale:.3e}) rel_rms={rr:.3e}", flush=True)
        assert np.isfinite(self.max_diff), f"{name}: non-finite values"
        assert self.max_diff <= MAX_ABS * scale and rr <= REL_RMS, (
            f"{name}: max_abs={self.max_diff:.3e} (bar {MAX_ABS * scale:.3e}) rel_rms={rr:.3e}")


def _ref_head(q, k, v, do, mask, scale):
    """fp32 forward + backward of one head (T x d operands, T x T bool mask)."""
    s = torch.mm(q, k.t().contiguous()).mul_(scale)
    s.masked_fill_(~mask, -math.inf)
    m = s.amax(dim=1, keepdim=True)
    m0 = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    p = s.sub_(m0).exp_()
    l = p.sum(dim=1, keepdim=True)
    p.div_(l.clamp_min(1e-30))
    o = torch.mm(p, v)
    lse = torch.where(l[:, 0] > 0, (m0[:, 0] + torch.log(l[:, 0])) * (1.0 / math.log(2.0)),
                      torch.full_like(l[:, 0], -math.inf))
    delta = (do * o).sum(dim=1, keepdim=True)
    ds = torch.mm(do, v.t().contiguous()).sub_(delta).mul_(p)
    dq = torch.mm(ds, k).mul_(scale)
    dk = torch.mm(ds.t().contiguous(), q).mul_(scale)
    dv = torch.mm(p.t().contiguous(), do)
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("hadamard", [False, True])
def test_config4_every_head_against_torch_fp32(dev, hadamard):
    inp = config_inputs(4, seed=0)
    B, H, T, D = inp["q"].shape
    print(f"config 4 full size B={B} H={H} T={T} D={D} hadamard={hadamard}: kernels", flush=True)
    q, k, v, do = (inp[x].to(dev) for x in ("q", "k", "v", "do"))
    ql, kl, vl = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    meta = {n: inp[n].to(dev) for n in ("in_span", "span_id", "is_prefix")}
    o, lse = flash_attention(ql, kl, vl, causal=True, return_lse=True, hadamard=hadamard, hadamard_seed=0, **meta)
    o.backward(do)
    torch.cuda.synchronize()
    got = {"o": o.detach(), "lse": lse.detach(), "dq": ql.grad, "dk": kl.grad, "dv": vl.grad}

    print("  reference operands", flush=True)
    mask = torch.from_numpy(np.ascontiguousarray(oracle_mask(inp, T))).to(dev)
    rot = None
    qs, ks = q, k
    if hadamard:  # the attention sees Q' = bf16(Q R), K' = bf16(K R); dQ, dK map back through R^T
        signs = generate_hadamard_signs(D, 0).numpy()
        qs = torch.from_numpy(ref_h.rotate_fp32(inp["q"].float().numpy(), signs)).to(torch.bfloat16).to(dev)
        ks = torch.from_numpy(ref_h.rotate_fp32(inp["k"].float().numpy(), signs)).to(torch.bfloat16).to(dev)
        rot = torch.from_numpy(ref_h.rotation_matrix(signs)).float().to(dev)
    scale = D ** -0.5
    err = {n: _Err() for n in ("o", "dq", "dk", "dv", "lse")}
    print("  reference heads", flush=True)
    for b in range(B):
        for h in range(H):
            r_o, r_lse, r_dq, r_dk, r_dv = _ref_head(qs[b, h].float(), ks[b, h].float(), v[b, h].float(),
                                                     do[b, h].float(), mask[b], scale)
            if rot is not None:
                r_dq = torch.mm(r_dq, rot.t().contiguous())
                r_dk = torch.mm(r_dk, rot.t().contiguous())
            g_lse = got["lse"][b, h]
            assert torch.equal(torch.isinf(g_lse), torch.isinf(r_lse)), f"LSE -inf pattern differs at head {(b, h)}"
            fin = torch.isfinite(r_lse)
            err["lse"].add(g_lse[fin], r_lse[fin])
            for name, r in (("o", r_o), ("dq", r_dq), ("dk", r_dk), ("dv", r_dv)):
                err[name].add(got[name][b, h].float(), r)
    torch.cuda.synchronize()
    failures = []
    for name, e in err.items():
        try:
            e.check(name)
        except AssertionError as exc:
            failures.append(str(exc))
    assert not failures, "; ".join(failures)
