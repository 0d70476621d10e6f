"""CPU pinning of the oracle's mask formula (original_kernel.py:478-517).

The reference ships no tests or vectors for the mask, so the oracle is pinned
by hand-evaluated truth tables, the closed-form special cases of the
formula, brute force on tiny inputs and invariants of the cocktail layout.
"""
import numpy as np
import pytest
import torch
from hypothesis import given, settings, strategies as st

from oracle.mask import dense_mask, dense_mask_bruteforce
from oracle.metadata import collate_metadata, fallback_metadata

PAD, CLS, MASK, SPAN, ES, MASKQ = 0, 1, 2, 3, 4, 5
B1 = 100  # a byte token


def _rows_to_mask(T, rows):
    m = np.zeros((T, T), bool)
    for i, cols in rows.items():
        m[i, list(cols)] = True
    return m


def test_hand_built_cocktail_sequence():
    # 0 1 2   | 3 4 5      | 6  7  8  | 9 10 11 | 12    | 13
    # p p CLS | c MASK c   | SPAN s ES| SPAN s ES| MASKQ | PAD
    toks = np.array([[B1, B1, CLS, B1, MASK, B1, SPAN, B1, ES, SPAN, B1, ES, MASKQ, PAD]])
    in_span, span_id, is_prefix = collate_metadata(toks)
    assert in_span[0].tolist() == [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 0, 0]
    assert span_id[0].tolist() == [0, 0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 2, -1, 0]
    assert is_prefix[0].tolist() == [1, 1, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0]
    pre = {0, 1, 2}
    ctx = [3, 4, 5, 13]
    expected = {
        0: pre, 1: pre, 2: pre,                                   # prefix: bidirectional within prefix
        3: pre | {3}, 4: pre | {3, 4}, 5: pre | {3, 4, 5},        # context: prefix + causal context
        6: {6, 7, 8, *ctx}, 7: {6, 7, 8, *ctx}, 8: {6, 7, 8, *ctx},        # span 1 island + context
        9: {9, 10, 11, *ctx}, 10: {9, 10, 11, *ctx}, 11: {9, 10, 11, *ctx},  # span 2 island + context
        12: pre | {6, 7, 8, 9, 10, 11},                            # MASKQ: spans + prefix
        13: pre | {3, 4, 5, 13},                                   # trailing PAD is context
    }
    m = dense_mask(14, in_span=in_span, span_id=span_id, is_prefix=is_prefix)[0]
    np.testing.assert_array_equal(m, _rows_to_mask(14, expected))
    assert not m[:, 12].any()  # nobody sees MASKQ (F9)
    np.testing.assert_array_equal(
        m, dense_mask_bruteforce(14, in_span=in_span, span_id=span_id, is_prefix=is_prefix)[0])


def test_fallback_metadata_drops_es_from_span():
    toks = np.array([[B1, CLS, B1, SPAN, B1, ES, MASKQ]])
    in_span, span_id, _ = fallback_metadata(toks)
    assert in_span[0].tolist() == [0, 0, 0, 1, 1, 0, 0]
    assert span_id[0].tolist() == [0, 0, 0, 1, 1, 0, -1]
    ci, cs, _ = collate_metadata(toks)
    assert ci[0].tolist() == [0, 0, 0, 1, 1, 1, 0]
    assert cs[0].tolist() == [0, 0, 0, 1, 1, 1, -1]


@pytest.mark.parametrize("T", [1, 5, 17])
def test_no_metadata_fallbacks(T):
    tril = np.tril(np.ones((T, T), bool))
    np.testing.assert_array_equal(dense_mask(T, causal=True)[0], tril)
    np.testing.assert_array_equal(dense_mask(T, causal=False)[0], np.ones((T, T), bool))
    # attention_mask given without metadata: formula with defaults = i >= j even if not causal
    np.testing.assert_array_equal(dense_mask(T, causal=False, attention_mask_given=True)[0], tril)


def test_all_zero_metadata_is_tril_whatever_causal():
    T = 9
    z = np.zeros((1, T), bool)
    for causal in (True, False):
        m = dense_mask(T, in_span=z, span_id=np.zeros((1, T), np.int64), is_prefix=z, causal=causal)
        np.testing.assert_array_equal(m[0], np.tril(np.ones((T, T), bool)))


def test_pure_prefix_is_all_ones():
    T = 8
    m = dense_mask(T, is_prefix=np.ones((1, T), bool))
    assert m.all()


def test_span_id_missing_disables_maskq_and_same_span():
    T = 6
    in_span = np.array([[0, 1, 1, 0, 1, 1]], bool)
    m = dense_mask(T, in_span=in_span)
    # without span_id, spans see only context (never each other or themselves)
    for i in (1, 2, 4, 5):
        assert m[0, i].tolist() == [True, False, False, True, False, False]


def test_lens_masks_rows_and_columns():
    T = 10
    lens = np.array([6, 10], np.int32)
    m = dense_mask(T, B=2, lens=lens, causal=False)
    assert m[0, :6, :6].all() and not m[0, 6:].any() and not m[0, :, 6:].any()
    assert m[1].all()


meta_strategy = st.integers(min_value=1, max_value=11).flatmap(
    lambda T: st.tuples(
        st.just(T),
        st.lists(st.booleans(), min_size=T, max_size=T),
        st.lists(st.integers(min_value=-2, max_value=3), min_size=T, max_size=T),
        st.lists(st.booleans(), min_size=T, max_size=T),
        st.integers(min_value=0, max_value=T + 2),
        st.sampled_from(["all", "no_span_id", "no_in_span", "no_prefix"]),
    ))


@settings(max_examples=150, deadline=None)
@given(meta_strategy)
def test_broadcast_equals_bruteforce(case):
    T, sp, sid, pre, ln, which = case
    in_span = np.array([sp], bool)
    span_id = np.array([sid], np.int64)
    is_prefix = np.array([pre], bool)
    if which == "no_span_id":
        span_id = None
    elif which == "no_in_span":
        in_span = None
    elif which == "no_prefix":
        is_prefix = None
    lens = np.array([ln], np.int32)
    a = dense_mask(T, in_span=in_span, span_id=span_id, is_prefix=is_prefix, lens=lens)
    b = dense_mask_bruteforce(T, in_span=in_span, span_id=span_id, is_prefix=is_prefix, lens=lens)
    np.testing.assert_array_equal(a, b)


def test_cocktail_layout_invariants():
    """On generator rows with their construction-time metadata
    (tests/golden/cocktail_rows.npz, config-3 layout)."""
    import os
    fx = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cocktail_rows.npz"))
    tokens, in_span = fx["c3_tokens"].astype(np.int64), fx["c3_in_span"]
    span_id, is_prefix = fx["c3_span_id"].astype(np.int64), fx["c3_is_prefix"]
    B, T = tokens.shape
    m = dense_mask(T, B=B, in_span=in_span, span_id=span_id, is_prefix=is_prefix)
    for b in range(B):
        toks = tokens[b]
        mq = int(np.nonzero(toks == MASKQ)[0][0])
        assert not m[b, :, mq].any()  # MASKQ column empty
        assert m[b].any(axis=1).all()  # every row sees something (prefix exists)
        sid = span_id[b]
        spans = [s for s in np.unique(sid) if s > 0]
        for s1 in spans:
            for s2 in spans:
                if s1 != s2:
                    assert not m[b][np.ix_(sid == s1, sid == s2)].any()  # span isolation
        pre = is_prefix[b]
        assert m[b][np.ix_(pre, pre)].all()
        assert not m[b][np.ix_(pre, ~pre)].any()
