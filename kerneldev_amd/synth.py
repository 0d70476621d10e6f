"""Seeded synthetic inputs for the benchmark configurations.

Cocktail-party sequences follow the layout the reference's collate builds
(``data_builder.py:597-601``)::

    prefix bytes + [CLS] | context (one [MASK] inside) | ([SPAN] bytes [ES]) x n | [MASKQ] | [PAD]...

with the metadata the collate writes while it assembles the row
(``data_builder.py:603-643``): ``is_prefix`` over the prefix bytes and [CLS],
``in_span`` / ``span_id`` over each ``[SPAN]..[ES]`` inclusive with ids 1..n in
the order the spans are placed, and ``span_id = -1`` at [MASKQ].  The
metadata comes from the construction itself (where each piece was put), not
from re-reading the tokens.  Byte tokens are ``6 + byte`` (ids 6..261,
``data_builder.py:141``).  A layout that does not fit in ``L`` is redrawn
(the survey notes the maximal layouts of configs 3 and 4 overflow L).

Everything is drawn from ``torch.Generator('cpu')`` so the device run and
the CPU oracle see identical bits.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

PAD, CLS, MASK, SPAN, ES, MASKQ = 0, 1, 2, 3, 4, 5
NUM_SPECIAL = 6
VOCAB = 256 + NUM_SPECIAL


@dataclass
class CocktailLayout:
    prefix_bytes: tuple  # (min, max) byte tokens before [CLS]
    context: tuple  # (min, max) context length (bytes, one replaced by [MASK])
    n_spans: tuple  # (min, max) number of spans
    span_bytes: tuple  # (min, max) bytes inside each [SPAN] .. [ES]


CONFIG3_LAYOUT = CocktailLayout((32, 128), (256, 512), (4, 8), (16, 64))
CONFIG4_LAYOUT = CocktailLayout((256, 256), (2048, 2048), (32, 32), (64, 192))


def _randint(g, lo, hi):
    """Uniform integer in [lo, hi] inclusive."""
    return int(torch.randint(lo, hi + 1, (1,), generator=g).item())


def cocktail_sequence(g: torch.Generator, L: int, layout: CocktailLayout, max_tries: int = 1000):
    """One token row of length L (redrawn until the layout fits) and its metadata.

    Returns ``(tokens, in_span, span_id, is_prefix)`` as lists of length L.  The
    metadata is marked as the pieces are placed, as data_builder.py:606-643
    does: the prefix and its [CLS] (:609-611), each span from its [SPAN] through
    its [ES] with id 1 + its index in placement order (:620-634), and -1 at the
    [MASKQ] (:637-643).
    """
    for _ in range(max_tries):
        npre = _randint(g, *layout.prefix_bytes)
        nctx = _randint(g, *layout.context)
        nsp = _randint(g, *layout.n_spans)
        lens = [_randint(g, *layout.span_bytes) for _ in range(nsp)]
        total = npre + 1 + nctx + sum(n + 2 for n in lens) + 1
        if total <= L:
            break
    else:  # pragma: no cover - layouts above always fit within a few draws
        raise RuntimeError("cocktail layout does not fit in L")
    def byte_tokens(n):
        return (torch.randint(0, 256, (n,), generator=g) + NUM_SPECIAL).tolist()
    toks = byte_tokens(npre) + [CLS]
    is_prefix = [True] * len(toks)
    ctx = byte_tokens(nctx)
    ctx[_randint(g, 0, nctx - 1)] = MASK
    toks += ctx
    in_span = [False] * len(toks)
    span_id = [0] * len(toks)
    for sid, n in enumerate(lens, start=1):
        piece = [SPAN] + byte_tokens(n) + [ES]
        toks += piece
        in_span += [True] * len(piece)
        span_id += [sid] * len(piece)
    toks += [MASKQ]
    in_span.append(False)
    span_id.append(-1)
    pad = L - len(toks)
    toks += [PAD] * pad
    in_span += [False] * pad
    span_id += [0] * pad
    is_prefix += [False] * (L - len(is_prefix))
    return toks, in_span, span_id, is_prefix


def cocktail_batch(B: int, L: int, layout: CocktailLayout, seed: int):
    """Tokens ``[B, L]`` int64 plus the construction-time collate metadata
    (in_span bool, span_id int64, is_prefix bool), as cocktail_sequence marks it."""
    g = torch.Generator("cpu").manual_seed(seed)
    rows = [cocktail_sequence(g, L, layout) for _ in range(B)]
    tokens = torch.tensor([r[0] for r in rows], dtype=torch.int64)
    in_span = torch.tensor([r[1] for r in rows], dtype=torch.bool)
    span_id = torch.tensor([r[2] for r in rows], dtype=torch.int64)
    is_prefix = torch.tensor([r[3] for r in rows], dtype=torch.bool)
    return tokens, in_span, span_id, is_prefix


def qkvdo(B, H, L, d, seed, dtype=torch.bfloat16, scale=1.0, outlier_frac=0.0, outlier_mult=20.0):
    """Q, K, V, dO ~ N(0, 1) * scale drawn on the CPU in fp32, then cast.

    ``outlier_frac`` > 0 picks ``ceil(frac * d)`` seeded channels per head of
    Q, K and V and multiplies them by ``outlier_mult`` (config 4).
    """
    g = torch.Generator("cpu").manual_seed(seed)
    out = []
    for idx in range(4):
        x = torch.randn(B, H, L, d, generator=g, dtype=torch.float32) * scale
        if outlier_frac > 0 and idx < 3:
            n_out = math.ceil(outlier_frac * d)
            for h in range(H):
                ch = torch.randperm(d, generator=g)[:n_out]
                x[:, h, :, ch] *= outlier_mult
        out.append(x.to(dtype))
    return tuple(out)


def config_inputs(cfg: int, seed: int = 0, dtype=None):
    """Inputs of BASELINE configs 1-4 (CPU tensors).

    Returns a dict with q, k, v, do, the metadata (None for causal configs),
    ``causal`` and a short ``name``.
    """
    if cfg == 1:
        q, k, v, do = qkvdo(2, 4, 256, 64, seed, dtype=dtype or torch.float32)
        return dict(name="causal B2 H4 L256 d64", q=q, k=k, v=v, do=do, in_span=None,
                    span_id=None, is_prefix=None, causal=True)
    if cfg == 2:
        q, k, v, do = qkvdo(8, 16, 2048, 64, seed, dtype=dtype or torch.bfloat16, scale=64 ** -0.5)
        return dict(name="causal B8 H16 L2048 d64", q=q, k=k, v=v, do=do, in_span=None,
                    span_id=None, is_prefix=None, causal=True)
    if cfg == 3:
        tokens, in_span, span_id, is_prefix = cocktail_batch(16, 1024, CONFIG3_LAYOUT, seed)
        q, k, v, do = qkvdo(16, 12, 1024, 64, seed + 1, dtype=dtype or torch.bfloat16)
        return dict(name="cocktail B16 H12 L1024 d64", q=q, k=k, v=v, do=do, in_span=in_span,
                    span_id=span_id, is_prefix=is_prefix, causal=True, tokens=tokens)
    if cfg == 4:
        tokens, in_span, span_id, is_prefix = cocktail_batch(2, 8192, CONFIG4_LAYOUT, seed)
        q, k, v, do = qkvdo(2, 32, 8192, 128, seed + 1, dtype=dtype or torch.bfloat16,
                            outlier_frac=0.01)
        return dict(name="cocktail B2 H32 L8192 d128", q=q, k=k, v=v, do=do, in_span=in_span,
                    span_id=span_id, is_prefix=is_prefix, causal=True, tokens=tokens)
    raise ValueError(f"unknown config {cfg}")
