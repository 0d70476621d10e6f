"""Cocktail-party head on the CPU (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

``reference_scores`` restates ``model.py:263-296`` statement by statement: the
first ``[MASK]`` per row through ``torch.unique`` counts (:264-271), the
``nonzero`` position lists of ``[SPAN]`` and ``[ES]`` (:273-274), the Python
double loop that zips each row's lists and averages ``h[i, st+1:ed]`` when
``st + 1 < ed`` (:287-293), and the ``einsum`` scores (:296).  It keeps the
reference's indexing of ``span_ends`` with the START list's row mask
(``span_ends[batch_indices == i, 1]``, :289), so it fails like the reference
when the batch's total [SPAN] and [ES] counts differ.

``scores`` is the per-row form the kernel implements: each row's j-th
``[SPAN]`` with the same row's j-th ``[ES]``.  The two agree whenever every
row holds as many ``[SPAN]`` as ``[ES]`` tokens (then the reference's mask
selects exactly the row's own ends); tests pin that, and pin ``scores`` by
hand-computed cases.

Both evaluate in the dtype of ``h`` (use float64) and are differentiable in
``h`` through torch autograd.
"""
from __future__ import annotations

import torch

MASK, SPAN, ES = 2, 3, 4  # data_builder.py:44-52


def reference_scores(tokens: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """``model.py:263-296`` as written (``x`` = tokens, ``x_embed`` = h)."""
    x, x_embed = tokens, h
    B, T = x.shape
    D = x_embed.size(-1)
    mask_positions = (x == MASK).nonzero(as_tuple=True)  # :264
    h_context = x_embed.new_zeros(B, D)  # :265
    unique_batch_idx, counts = torch.unique(mask_positions[0], return_counts=True)  # :267
    first_mask_indices = torch.cat((x.new_zeros(1, dtype=torch.long), torch.cumsum(counts, 0)[:-1]))  # :268
    if unique_batch_idx.numel() > 0:  # :269-270
        h_context = h_context.index_put((unique_batch_idx,), x_embed[unique_batch_idx,
                                                                     mask_positions[1][first_mask_indices]])
    span_starts = (x == SPAN).nonzero()  # :273
    span_ends = (x == ES).nonzero()  # :274
    if span_starts.numel() == 0:  # :276-277
        return torch.empty(0)
    batch_indices = span_starts[:, 0]  # :280
    max_spans = int((x == SPAN).sum(dim=1).max())  # :283
    rows = []
    for i in range(B):  # :287
        st_indices = span_starts[batch_indices == i, 1]  # :288
        ed_indices = span_ends[batch_indices == i, 1]  # :289 (the start list's row mask)
        row = [x_embed.new_zeros(D) for _ in range(max_spans)]  # :285
        for j, (st, ed) in enumerate(zip(st_indices.tolist(), ed_indices.tolist())):  # :291
            if st + 1 < ed:  # :292
                row[j] = x_embed[i, st + 1:ed].mean(dim=0)  # :293
        rows.append(torch.stack(row))
    h_spans = torch.stack(rows)
    return torch.einsum("bd,bnd->bn", h_context, h_spans)  # :296


def scores(tokens: torch.Tensor, h: torch.Tensor, n_spans: int | None = None) -> torch.Tensor:
    """Per-row zip: row i's j-th [SPAN] with row i's j-th [ES]; ``[B, n_spans]``."""
    B, T = tokens.shape
    D = h.shape[-1]
    counts = (tokens == SPAN).sum(dim=1)
    n = int(counts.max()) if n_spans is None else n_spans
    out = []
    for i in range(B):
        t = tokens[i].tolist()
        first = next((p for p, v in enumerate(t) if v == MASK), None)
        ctx = h[i, first] if first is not None else h.new_zeros(D)
        sts = [p for p, v in enumerate(t) if v == SPAN]
        eds = [p for p, v in enumerate(t) if v == ES]
        row = []
        for j in range(n):
            if j < len(sts) and j < len(eds) and sts[j] + 1 < eds[j]:
                row.append((h[i, sts[j] + 1:eds[j]].mean(dim=0) * ctx).sum())
            else:
                row.append(h.new_zeros(()))
        out.append(torch.stack(row))
    return torch.stack(out)
