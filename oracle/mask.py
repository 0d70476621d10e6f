"""Dense restatement of the reference's attention-mask formula (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

The formula is ``original_kernel.py:478-517`` (forward; the dQ and dK/dV
kernels repeat it at ``:1289-1328`` and ``:1475-1514``).  Inputs are numpy
arrays; missing metadata uses the defaults of ``:449-470`` (``in_span`` and
``is_prefix`` all False, ``span_id`` all 0, and MASKQ / same-span detection
switched off when ``span_id`` is None).
"""
from __future__ import annotations

import numpy as np


def _np(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.asarray(x)


def mask_mode(in_span, span_id, is_prefix, attention_mask_given: bool, causal: bool) -> str:
    """Which branch of the reference's forward mask code applies.

    ``original_kernel.py:401`` sets FAST_PATH_NO_RULES when attention_mask and
    all metadata are None; then ``:512-515`` use ``i >= j`` (causal) or all
    True.  Otherwise the 7-term formula runs with defaults for missing tensors
    (so attention_mask with no metadata degenerates to ``i >= j``).
    """
    if in_span is None and span_id is None and is_prefix is None and not attention_mask_given:
        return "causal" if causal else "all"
    return "formula"


def dense_mask(T: int, B: int = 1, in_span=None, span_id=None, is_prefix=None,
               lens=None, causal: bool = True, attention_mask_given: bool = False) -> np.ndarray:
    """Boolean ``[B, T, T]`` mask, ``allow[b, i, j]`` = query i may see key j.

    Literal broadcast restatement of ``original_kernel.py:478-517``:

    * ``prefix_to_prefix  = q_pre & k_pre``                        (:484)
    * ``context_causal    = q_ctx & k_ctx & (i >= j)``             (:488-489)
    * ``context_to_prefix = q_ctx & k_pre``                        (:490)
    * ``same_span = q_span & k_span & (q_sid == k_sid) & span_id_given & (q_sid > 0)`` (:493-495)
    * ``span_to_context   = q_span & k_ctx``                       (:496)
    * ``maskq_to_spans    = q_mq & k_span``                        (:499)
    * ``maskq_to_cls      = q_mq & k_pre``                         (:500)

    with ``mq = (span_id == -1)`` only when span_id is given (:475, :481) and
    ``ctx = ~span & ~pre & ~mq`` (:476, :487).  Finally
    ``& (i < seq_len) & (j < seq_len)`` with ``seq_len = min(lens[b], T)``
    (:299-303, :517).
    """
    in_span, span_id, is_prefix, lens = _np(in_span), _np(span_id), _np(is_prefix), _np(lens)
    for t in (in_span, span_id, is_prefix):
        if t is not None:
            B = t.shape[0]
    if lens is not None:
        B = lens.shape[0]
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    mode = mask_mode(in_span, span_id, is_prefix, attention_mask_given, causal)
    if mode == "causal":
        m = np.broadcast_to(i >= j, (B, T, T)).copy()
    elif mode == "all":
        m = np.ones((B, T, T), dtype=bool)
    else:
        span = in_span.astype(bool) if in_span is not None else np.zeros((B, T), bool)
        pre = is_prefix.astype(bool) if is_prefix is not None else np.zeros((B, T), bool)
        sid = span_id.astype(np.int64) if span_id is not None else np.zeros((B, T), np.int64)
        if span_id is not None:
            mq = sid == -1
        else:
            mq = np.zeros((B, T), bool)
        ctx = ~span & ~pre & ~mq
        q_pre, k_pre = pre[:, :, None], pre[:, None, :]
        q_ctx, k_ctx = ctx[:, :, None], ctx[:, None, :]
        q_span, k_span = span[:, :, None], span[:, None, :]
        q_sid, k_sid = sid[:, :, None], sid[:, None, :]
        q_mq = mq[:, :, None]
        prefix_to_prefix = q_pre & k_pre
        context_causal = q_ctx & k_ctx & (i >= j)[None]
        context_to_prefix = q_ctx & k_pre
        same_span = q_span & k_span & (q_sid == k_sid) & (span_id is not None) & (q_sid > 0)
        span_to_context = q_span & k_ctx
        maskq_to_spans = q_mq & k_span
        maskq_to_cls = q_mq & k_pre
        m = (prefix_to_prefix | context_causal | context_to_prefix | same_span
             | span_to_context | maskq_to_spans | maskq_to_cls)
    if lens is not None:
        sl = np.minimum(lens.astype(np.int64), T)
        valid = np.arange(T)[None, :] < sl[:, None]
        m = m & valid[:, :, None] & valid[:, None, :]
    return m


def dense_mask_bruteforce(T, B=1, in_span=None, span_id=None, is_prefix=None, lens=None,
                          causal=True, attention_mask_given=False) -> np.ndarray:
    """Element-by-element Python evaluation of the same rules (tiny T only).

    Written as the nested conditionals a reader of ``original_kernel.py:478-517``
    would hand-evaluate, independent of the broadcasting above.
    """
    in_span, span_id, is_prefix, lens = _np(in_span), _np(span_id), _np(is_prefix), _np(lens)
    mode = mask_mode(in_span, span_id, is_prefix, attention_mask_given, causal)
    out = np.zeros((B, T, T), dtype=bool)
    for b in range(B):
        sl = T if lens is None else min(int(lens[b]), T)
        for i in range(T):
            for j in range(T):
                if i >= sl or j >= sl:
                    continue
                if mode == "causal":
                    out[b, i, j] = i >= j
                    continue
                if mode == "all":
                    out[b, i, j] = True
                    continue
                sp_i = bool(in_span[b, i]) if in_span is not None else False
                sp_j = bool(in_span[b, j]) if in_span is not None else False
                pr_i = bool(is_prefix[b, i]) if is_prefix is not None else False
                pr_j = bool(is_prefix[b, j]) if is_prefix is not None else False
                id_i = int(span_id[b, i]) if span_id is not None else 0
                id_j = int(span_id[b, j]) if span_id is not None else 0
                mq_i = span_id is not None and id_i == -1
                mq_j = span_id is not None and id_j == -1
                cx_i = not sp_i and not pr_i and not mq_i
                cx_j = not sp_j and not pr_j and not mq_j
                ok = False
                if pr_i and pr_j:
                    ok = True
                if cx_i and (pr_j or (cx_j and i >= j)):
                    ok = True
                if sp_i and cx_j:
                    ok = True
                if sp_i and sp_j and span_id is not None and id_i == id_j and id_i > 0:
                    ok = True
                if mq_i and (sp_j or pr_j):
                    ok = True
                out[b, i, j] = ok
    return out
