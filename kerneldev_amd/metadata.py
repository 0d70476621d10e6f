"""Token ids -> hierarchical-mask metadata, vectorised (no host syncs).

Three derivations exist in the reference and they disagree on [ES]:

* ``"collate"`` -- the data builder (``data_builder.py:603-643``), used on the
  training path (``train_loop.py:381`` -> ``model.py:197-201``): prefix
  through the first [CLS]; ``[SPAN] .. [ES]`` INCLUSIVE with ids 1..n;
  ``span_id = -1`` at the first [MASKQ].
* ``"fallback"`` -- the model's standalone fallback (``model.py:209-240``):
  ``in_span = cumsum([SPAN]) - cumsum([ES]) > 0`` EXCLUDES [ES] (it becomes a
  context token with span_id 0); every [MASKQ] gets -1.
* ``"teacher_forcing"`` -- ``train_loop.py:406-435``: prefix only.

All three run as a handful of cumulative sums on the tokens' device.
"""
from __future__ import annotations

import torch

PAD, CLS, MASK, SPAN, ES, MASKQ = 0, 1, 2, 3, 4, 5


def _prefix_through_first(tokens: torch.Tensor, tok: int) -> torch.Tensor:
    hit = (tokens == tok).to(torch.int32)
    before = torch.cumsum(hit, dim=1) - hit  # number of hits strictly before t
    has = hit.any(dim=1, keepdim=True)
    return (before == 0) & has


def _first_only(tokens: torch.Tensor, tok: int) -> torch.Tensor:
    hit = tokens == tok
    c = torch.cumsum(hit.to(torch.int32), dim=1)
    return hit & (c == 1)


def derive_metadata(tokens: torch.Tensor, rule: str = "collate"):
    """Return ``(in_span bool, span_id int64, is_prefix bool)``, each ``[B, L]``."""
    if tokens.dim() != 2:
        raise ValueError("tokens must be [B, L]")
    is_prefix = _prefix_through_first(tokens, CLS)
    if rule == "teacher_forcing":
        z = torch.zeros_like(tokens, dtype=torch.bool)
        return z, torch.zeros_like(tokens, dtype=torch.int64), is_prefix
    n_span = torch.cumsum((tokens == SPAN).to(torch.int64), dim=1)
    es = (tokens == ES).to(torch.int64)
    n_es = torch.cumsum(es, dim=1)
    if rule == "collate":
        in_span = (n_span - (n_es - es)) > 0  # [ES] closes AFTER itself
        span_id = torch.where(in_span, n_span, torch.zeros_like(n_span))
        span_id = torch.where(_first_only(tokens, MASKQ), torch.full_like(span_id, -1), span_id)
    elif rule == "fallback":
        in_span = (n_span - n_es) > 0
        span_id = torch.where(in_span, n_span, torch.zeros_like(n_span))
        span_id = torch.where(tokens == MASKQ, torch.full_like(span_id, -1), span_id)
    else:
        raise ValueError(f"unknown metadata rule {rule!r}")
    return in_span, span_id, is_prefix
