"""Token -> mask metadata, restated as plain per-token loops (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Token ids follow ``data_builder.py:44-52``: [PAD]=0, [CLS]=1, [MASK]=2,
[SPAN]=3, [ES]=4, [MASKQ]=5; bytes are ``byte + 6``.
"""
from __future__ import annotations

import numpy as np

PAD, CLS, MASK, SPAN, ES, MASKQ = 0, 1, 2, 3, 4, 5


def collate_metadata(tokens: np.ndarray):
    """The data-builder rule (``data_builder.py:603-643``) read off the tokens.

    * ``is_prefix``: positions ``[0, cls_idx]`` of the first [CLS] (:609-611);
      none when there is no [CLS] (task_prefix = [] at :498-501).
    * ``in_span`` / ``span_id``: each ``[SPAN] ... [ES]`` run INCLUSIVE of both
      markers, ids 1, 2, ... in order (:624-634).
    * ``span_id = -1`` at the first [MASKQ] (:637-643), which is not in a span.
    """
    tokens = np.asarray(tokens)
    B, T = tokens.shape
    in_span = np.zeros((B, T), bool)
    span_id = np.zeros((B, T), np.int64)
    is_prefix = np.zeros((B, T), bool)
    for b in range(B):
        row = [int(x) for x in tokens[b]]
        if CLS in row:
            c = row.index(CLS)
            for t in range(c + 1):
                is_prefix[b, t] = True
        sid = 0
        inside = False
        for t in range(T):
            if row[t] == SPAN and not inside:
                sid += 1
                inside = True
            if inside:
                in_span[b, t] = True
                span_id[b, t] = sid
                if row[t] == ES:
                    inside = False
        if MASKQ in row:
            span_id[b, row.index(MASKQ)] = -1
    return in_span, span_id, is_prefix


def fallback_metadata(tokens: np.ndarray):
    """The model's token fallback (``model.py:209-240``).

    ``in_span = cumsum([SPAN]) - cumsum([ES]) > 0`` -- this EXCLUDES the [ES]
    marker itself (:219); ``span_id = cumsum([SPAN])`` inside spans else 0
    (:220-221); every [MASKQ] gets -1 (:224-225); prefix up to and including
    the first [CLS] (:228-233).  Written as a running counter per token.
    """
    tokens = np.asarray(tokens)
    B, T = tokens.shape
    in_span = np.zeros((B, T), bool)
    span_id = np.zeros((B, T), np.int64)
    is_prefix = np.zeros((B, T), bool)
    for b in range(B):
        n_span = 0
        n_es = 0
        cls_seen = False
        for t in range(T):
            tok = int(tokens[b, t])
            if tok == SPAN:
                n_span += 1
            if tok == ES:
                n_es += 1
            inside = (n_span - n_es) > 0
            in_span[b, t] = inside
            span_id[b, t] = n_span if inside else 0
            if tok == MASKQ:
                span_id[b, t] = -1
            if not cls_seen:
                is_prefix[b, t] = True
                if tok == CLS:
                    cls_seen = True
        if not cls_seen:
            is_prefix[b, :] = False
    return in_span, span_id, is_prefix


def teacher_forcing_metadata(tokens: np.ndarray):
    """``train_loop.py:406-435``: prefix through the first [CLS], no spans."""
    tokens = np.asarray(tokens)
    B, T = tokens.shape
    in_span = np.zeros((B, T), bool)
    span_id = np.zeros((B, T), np.int64)
    is_prefix = np.zeros((B, T), bool)
    for b in range(B):
        row = [int(x) for x in tokens[b]]
        if CLS in row:
            is_prefix[b, : row.index(CLS) + 1] = True
    return in_span, span_id, is_prefix
