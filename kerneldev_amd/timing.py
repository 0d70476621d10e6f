"""Time ``flash_attention`` forward + backward at a given shape and dtype.

``python -m kerneldev_amd.timing --dtype fp32 --B 2 --H 8 --T 4096 --D 128``

Causal attention (``--no-causal``: all keys) on seeded N(0, 1) inputs, through
the public API exactly as a model calls it (plan, forward, backward).  It runs
``--warmup`` untimed steps, then ``--steps`` timed ones between two
synchronisations.  It prints one line per run with the time per step and the
useful TFLOP/s (14 d per allowed score entry, as ``bench.py`` counts).  This
is for head dims, dtypes and precisions outside the benchmark's configuration.
"""
from __future__ import annotations

import argparse
import time

import torch

from . import flash_attention
from .synth import qkvdo

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def time_step(B, H, T, D, dtype, precision="tf32", causal=True, steps=10, warmup=3, seed=1):
    """Seconds per fwd+bwd step and the step's allowed score entries."""
    dev = torch.device("cuda:0")
    q, k, v, do = (x.to(dev) for x in qkvdo(B, H, T, D, seed=seed, dtype=dtype))
    q, k, v = (x.requires_grad_(True) for x in (q, k, v))

    def step():
        o = flash_attention(q, k, v, causal=causal, precision=precision)
        o.backward(do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    nnz = B * H * (T * (T + 1) // 2 if causal else T * T)
    return (time.perf_counter() - t0) / steps, nnz


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--dtype", default="bf16", choices=tuple(DTYPES))
    ap.add_argument("--precision", default="tf32", choices=("tf32", "ieee", "bf16"))
    ap.add_argument("--B", type=int, default=2)
    ap.add_argument("--H", type=int, default=8)
    ap.add_argument("--T", type=int, default=4096)
    ap.add_argument("--D", type=int, nargs="+", default=[128])
    ap.add_argument("--no-causal", action="store_true")
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    args = ap.parse_args()
    for D in args.D:
        s, nnz = time_step(args.B, args.H, args.T, D, DTYPES[args.dtype], args.precision, not args.no_causal,
                           args.steps, args.warmup)
        print(f"{args.dtype} {args.precision} B={args.B} H={args.H} T={args.T} D={D} "
              f"{'all keys' if args.no_causal else 'causal'}: {s * 1e3:.3f} ms fwd+bwd, "
              f"{14 * D * nnz / s / 1e12:.1f} TFLOP/s useful", flush=True)


if __name__ == "__main__":
    main()
