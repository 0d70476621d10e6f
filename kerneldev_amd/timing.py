"""Time ``flash_attention`` forward + backward at a given shape and dtype.

``python -m kerneldev_amd.timing --dtype fp32 --B 2 --H 8 --T 4096 --D 128``
(``--qk-dtype fp8_e4m3`` and ``--hadamard`` as ``flash_attention`` takes them)

Causal attention (``--no-causal``: all keys) on seeded N(0, 1) inputs, through
the public API exactly as a model calls it (plan, forward, backward).  It runs
``--warmup`` untimed steps, then ``--steps`` timed ones between two
synchronisations.  It prints one line per run with the time per step and the
useful TFLOP/s (14 d per allowed score entry, as ``bench.py`` counts).  This
is for head dims, dtypes and precisions outside the benchmark's configuration.

``python -m kerneldev_amd.timing --gpt kdattn sdpa_fp32 sdpa_bf16`` times config 5's
training step instead (``time_gpt_step``), once per attention named.
"""
from __future__ import annotations

import argparse
import time

import torch

from . import flash_attention
from .synth import qkvdo

DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def time_step(B, H, T, D, dtype, precision="tf32", causal=True, steps=10, warmup=3, seed=1, qk_dtype="bf16",
              hadamard=False):
    """Seconds per fwd+bwd step and the step's allowed score entries."""
    dev = torch.device("cuda:0")
    q, k, v, do = (x.to(dev) for x in qkvdo(B, H, T, D, seed=seed, dtype=dtype))
    q, k, v = (x.requires_grad_(True) for x in (q, k, v))

    def step():
        o = flash_attention(q, k, v, causal=causal, precision=precision, qk_dtype=qk_dtype, hadamard=hadamard)
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


def _dense_sdpa(mask, backend, dtype):
    """A GPTModel attention that ignores the metadata and applies torch SDPA with
    a precomputed dense [B, 1, T, T] bool mask (the pattern of the reference's
    eager ``flash_attention_reference``, original_kernel.py:2002-2032), computing
    in ``dtype`` on the given SDPA backend and casting back."""
    def attention(q, k, v, lens=None, causal=True, attention_mask=None, in_span=None, span_id=None,
                  is_prefix=None):
        with torch.nn.attention.sdpa_kernel(backend):
            o = torch.nn.functional.scaled_dot_product_attention(q.to(dtype), k.to(dtype), v.to(dtype),
                                                                 attn_mask=mask, scale=q.shape[-1] ** -0.5)
        return o.to(q.dtype)
    return attention


def time_gpt_step(attention="kdattn", B=8, L=2048, steps=5, warmup=2, seed=4):
    """Milliseconds per config-5 training step: GPTModel (d_model 768, 12 layers,
    12 heads of 64, SwiGLU 2048, bf16 weights) forward on a cocktail-party
    batch, span-score cross entropy, backward and an AdamW update (the step of
    train_loop.py's inner loop, without its DDP and logging).

    ``attention``: ``"kdattn"`` (flash_attention, one plan shared by the layers),
    ``"sdpa_bf16"`` (torch SDPA in bf16 on its memory-efficient backend with the
    dense mask) or ``"sdpa_fp32"`` (torch SDPA in fp32, math backend).  The
    dense mask comes from flash_attention's own mask output and is built once,
    outside the timed steps.  Returns (ms per step, last loss)."""
    from torch.nn.attention import SDPBackend

    from .gpt import GPTModel, config5_batch

    dev = torch.device("cuda:0")
    tokens, in_span, span_id, is_prefix, correct = (x.to(dev) for x in config5_batch(B=B, L=L, seed=seed))
    torch.manual_seed(seed)
    if attention == "kdattn":
        model = GPTModel(max_seq_len=L)
    else:
        probe = torch.zeros(B, 1, L, 64, device=dev, dtype=torch.bfloat16)
        _, mask = flash_attention(probe, probe, probe, return_attention_mask=True,
                                  in_span=in_span, span_id=span_id, is_prefix=is_prefix)
        backend, dt = {"sdpa_bf16": (SDPBackend.EFFICIENT_ATTENTION, torch.bfloat16),
                       "sdpa_fp32": (SDPBackend.MATH, torch.float32)}[attention]
        model = GPTModel(max_seq_len=L, attention=_dense_sdpa(mask, backend, dt))
    model = model.to(dev).to(torch.bfloat16)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4)

    def step():
        opt.zero_grad(set_to_none=True)
        _, loss = model(tokens, correct_idx=correct, in_span=in_span, span_id=span_id, is_prefix=is_prefix)
        loss.backward()
        opt.step()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3, loss.item()


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpt", nargs="*", choices=("kdattn", "sdpa_bf16", "sdpa_fp32"),
                    help="time config-5 training steps with these attentions instead")
    ap.add_argument("--dtype", default="bf16", choices=tuple(DTYPES))
    ap.add_argument("--precision", default="tf32", choices=("tf32", "ieee", "bf16"))
    ap.add_argument("--B", type=int, default=2)
    ap.add_argument("--H", type=int, default=8)
    ap.add_argument("--T", type=int, default=4096)
    ap.add_argument("--D", type=int, nargs="+", default=[128])
    ap.add_argument("--no-causal", action="store_true")
    ap.add_argument("--qk-dtype", default="bf16", choices=("bf16", "fp8_e4m3"))
    ap.add_argument("--hadamard", action="store_true")
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    args = ap.parse_args()
    if args.gpt is not None:
        for att in args.gpt or ["kdattn"]:
            print(f"config 5 (B=8, L=2048) training step, attention {att}", flush=True)
            ms, loss = time_gpt_step(att, steps=args.steps, warmup=args.warmup)
            print(f"config 5 step with {att}: {ms:.2f} ms (fwd, span-score loss, bwd, AdamW), "
                  f"loss {loss:.4f}", flush=True)
        return
    for D in args.D:
        s, nnz = time_step(args.B, args.H, args.T, D, DTYPES[args.dtype], args.precision, not args.no_causal,
                           args.steps, args.warmup, qk_dtype=args.qk_dtype, hadamard=args.hadamard)
        print(f"{args.dtype} {args.precision} qk {args.qk_dtype}{' hadamard' if args.hadamard else ''} B={args.B} H={args.H} T={args.T} D={D} "
              f"{'all keys' if args.no_causal else 'causal'}: {s * 1e3:.3f} ms fwd+bwd, "
              f"{14 * D * nnz / s / 1e12:.1f} TFLOP/s useful", flush=True)


if __name__ == "__main__":
    main()
