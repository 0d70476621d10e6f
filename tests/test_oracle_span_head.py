"""CPU: the cocktail-party head oracle (``oracle/span_head.py``).

``scores`` (the per-row pairing the kernel implements) is pinned by hand-built
cases with known answers and checked against ``reference_scores``, the
statement-by-statement restatement of ``model.py:263-296``, wherever the
reference is well defined (every row holds as many [SPAN] as [ES] tokens).
The cases where the reference's ``span_ends[batch_indices == i]`` indexing
(:289) pairs across rows or raises are pinned too, as documented differences.
"""
import os

import numpy as np
import pytest
import torch

from oracle import span_head as ref

MASK, SPAN, ES, X = 2, 3, 4, 100


def _h(B, T, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, T, D, generator=g, dtype=torch.float64)


def test_hand_case():
    # pos: 0  1     2     3  4  5   6     7   8     9  10  11
    toks = [X, MASK, SPAN, X, X, ES, SPAN, ES, MASK, SPAN, X, ES]
    t = torch.tensor([toks])
    h = torch.arange(12 * 2, dtype=torch.float64).view(1, 12, 2)
    ctx = h[0, 1]                       # first [MASK] only
    s0 = (h[0, 3:5].mean(0) * ctx).sum()  # interior of the first pair
    s2 = (h[0, 10:11].mean(0) * ctx).sum()
    want = torch.tensor([[s0, 0.0, s2]], dtype=torch.float64)  # the second pair is empty
    assert torch.equal(ref.scores(t, h), want)
    assert torch.equal(ref.reference_scores(t, h), want)


def test_row_without_mask_scores_zero_and_padding_columns():
    t = torch.tensor([[X, SPAN, X, ES, X, X],
                      [MASK, SPAN, X, X, ES, X]])
    h = _h(2, 6, 3)
    got = ref.scores(t, h)
    assert got.shape == (2, 1)
    assert got[0, 0] == 0                                    # no [MASK]: zero context
    assert torch.allclose(got[1, 0], (h[1, 2:4].mean(0) * h[1, 0]).sum())
    # more columns than spans: the extra ones are zero
    assert torch.equal(ref.scores(t, h, n_spans=3)[:, 1:], torch.zeros(2, 2, dtype=torch.float64))


@pytest.mark.parametrize("layout", ["c3", "c4"])
def test_matches_reference_on_generator_batches(layout):
    """Generator rows (tests/golden/cocktail_rows.npz): config-3 and config-4 layouts."""
    fx = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cocktail_rows.npz"))
    tokens = torch.from_numpy(fx[f"{layout}_tokens"].astype(np.int64))
    B, T = tokens.shape
    h = _h(B, T, 16, B)
    a, b = ref.scores(tokens, h), ref.reference_scores(tokens, h)
    assert a.shape == b.shape
    assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_matches_reference_on_balanced_malformed_rows():
    # equal [SPAN] / [ES] counts per row, in odd orders: nested, inverted, adjacent
    t = torch.tensor([[MASK, SPAN, SPAN, X, ES, X, ES, X],
                      [X, ES, X, MASK, SPAN, X, X, X],
                      [SPAN, ES, MASK, X, X, X, X, X]])
    h = _h(3, 8, 4, 3)
    a, b = ref.scores(t, h), ref.reference_scores(t, h)
    assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)
    # row 0 nests: pair 0 = (1, 4) -> interior 2..3 (includes the second [SPAN]), pair 1 = (2, 6)
    assert torch.allclose(a[0, 0], (h[0, 2:4].mean(0) * h[0, 0]).sum())
    assert torch.allclose(a[0, 1], (h[0, 3:6].mean(0) * h[0, 0]).sum())
    assert a[1, 0] == 0 and a[2, 0] == 0  # inverted pair; empty interior


def test_documented_differences_from_reference_indexing():
    # equal totals but per-row counts differ: the reference takes row 1's [ES]
    # for row 0's [SPAN] (span_ends[batch_indices == i]); the oracle keeps rows apart
    t = torch.tensor([[MASK, SPAN, X, X, X, X],
                      [MASK, X, ES, SPAN, X, ES]])
    h = _h(2, 6, 2, 5)
    got = ref.scores(t, h)
    assert got[0, 0] == 0                              # row 0 has no [ES]
    assert torch.allclose(got[1, 0], torch.zeros((), dtype=torch.float64))  # (3, 2) inverted
    r = ref.reference_scores(t, h)
    assert not torch.allclose(r, got)
    # different totals: the reference's boolean index has the wrong length
    t2 = torch.tensor([[MASK, SPAN, X, ES, ES, X]])
    with pytest.raises(IndexError):
        ref.reference_scores(t2, _h(1, 6, 2))
    assert ref.scores(t2, _h(1, 6, 2)).shape == (1, 1)


def test_gradient_is_the_spread_rule():
    # d score_j / d h[t] = ctx / n_j on the interior, sum_j ds_j mean_j at the [MASK] row
    t = torch.tensor([[X, MASK, SPAN, X, X, X, ES, SPAN, X, ES]])
    h = _h(1, 10, 3, 7).requires_grad_(True)
    ds = torch.tensor([[0.5, -2.0]], dtype=torch.float64)
    (ref.scores(t, h) * ds).sum().backward()
    ctx = h.detach()[0, 1]
    m0, m1 = h.detach()[0, 3:6].mean(0), h.detach()[0, 8:9].mean(0)
    want = torch.zeros(10, 3, dtype=torch.float64)
    want[3:6] = 0.5 * ctx / 3
    want[8] = -2.0 * ctx
    want[1] = 0.5 * m0 - 2.0 * m1
    assert torch.allclose(h.grad[0], want, rtol=1e-12, atol=1e-12)
