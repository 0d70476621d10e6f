"""GPU: config 4 at its full size, every (b, h) head.

The selected-head tests in ``test_gpu_attention.py`` compare against the fp64
oracle on the CPU.  Here all 64 heads of B2 H32 L8192 d128 are checked
against a plain PyTorch fp32 reference computed on the GPU one head at a time,
with the dense mask from the oracle (``oracle/mask.py``) and, for the Hadamard
run, Q' and K' from the oracle's bit-exact rotation (``oracle/hadamard.py``).

Bar: the north_star bar per element, as in ``helpers.assert_close``: the
error beyond one output ulp (bf16 for O and the gradients, fp32 for LSE) at
each element <= 2e-2, and rel-RMS <= 1e-2 over all heads; LSE (log2 units) on
the finite rows, and the -inf pattern exact.
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
    """Running max-abs, beyond-one-ulp and RMS error of one tensor over the heads."""

    def __init__(self, mantissa_bits):
        self.bits = mantissa_bits
        self.max_diff = self.max_excess = self.sq_diff = self.sq_ref = 0.0
        self.worst = ""

    def add(self, got, ref, where):
        ref = ref.double()
        d = (got.double() - ref).abs()
        a = ref.abs()
        ulp = torch.where(a > 0, torch.exp2(torch.floor(torch.log2(a.clamp_min(1e-30))) - self.bits),
                          torch.zeros_like(a))
        ex = (d - ulp).clamp_min(0).flatten()
        i = int(ex.argmax())
        if ex[i].item() > self.max_excess or not self.worst:
            self.max_excess = max(self.max_excess, ex[i].item())
            self.worst = (f"head {where} element {i}: got {got.flatten()[i].item():.6g} "
                          f"ref {ref.flatten()[i].item():.6g}")
        self.max_diff = max(self.max_diff, d.max().item())
        self.sq_diff += d.pow(2).sum().item()
        self.sq_ref += ref.pow(2).sum().item()

    def check(self, name):
        rr = math.sqrt(self.sq_diff / max(self.sq_ref, 1e-300))
        print(f"  {name}: max_abs={self.max_diff:.3e} beyond_ulp={self.max_excess:.3e} rel_rms={rr:.3e} "
              f"(worst: {self.worst})", flush=True)
        assert np.isfinite(self.max_diff), f"{name}: non-finite values"
        assert self.max_excess <= MAX_ABS and rr <= REL_RMS, (
            f"{name}: max_abs={self.max_diff:.3e} beyond_ulp={self.max_excess:.3e} rel_rms={rr:.3e} "
            f"worst {self.worst}")


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
    err = {n: _Err(7) for n in ("o", "dq", "dk", "dv")}  # bf16 outputs
    err["lse"] = _Err(23)  # fp32
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
            err["lse"].add(g_lse[fin], r_lse[fin], (b, h))
            for name, r in (("o", r_o), ("dq", r_dq), ("dk", r_dk), ("dv", r_dv)):
                err[name].add(got[name][b, h].float(), r, (b, h))
    torch.cuda.synchronize()
    failures = []
    for name, e in err.items():
        try:
            e.check(name)
        except AssertionError as exc:
            failures.append(str(exc))
    assert not failures, "; ".join(failures)
