"""CPU: the product's token -> metadata derivation (kerneldev_amd.metadata,
vectorised torch) against the metadata the generator marks while it builds
each row, and against the oracle's per-token restatement of all three rules
(oracle/metadata.py: data_builder.py:603-643, model.py:209-240,
train_loop.py:406-435)."""
import os

import numpy as np
import pytest
import torch

from kerneldev_amd.metadata import derive_metadata
from kerneldev_amd.synth import CONFIG3_LAYOUT, CONFIG4_LAYOUT, cocktail_batch
from oracle import metadata as ref_meta

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cocktail_rows.npz")


def test_generator_reproduces_the_committed_rows():
    """cocktail_batch is deterministic: it regenerates the fixture's rows and metadata."""
    fx = np.load(GOLDEN)
    for name, (B, L, layout, seed) in {"c3": (6, 1024, CONFIG3_LAYOUT, 5), "c4": (2, 8192, CONFIG4_LAYOUT, 0)}.items():
        tokens, in_span, span_id, is_prefix = cocktail_batch(B, L, layout, seed)
        np.testing.assert_array_equal(tokens.numpy(), fx[f"{name}_tokens"])
        np.testing.assert_array_equal(in_span.numpy(), fx[f"{name}_in_span"])
        np.testing.assert_array_equal(span_id.numpy(), fx[f"{name}_span_id"])
        np.testing.assert_array_equal(is_prefix.numpy(), fx[f"{name}_is_prefix"])


@pytest.mark.parametrize("layout,B,L,seed", [(CONFIG3_LAYOUT, 16, 1024, 0), (CONFIG4_LAYOUT, 2, 8192, 0),
                                              (CONFIG3_LAYOUT, 8, 2048, 1), (CONFIG3_LAYOUT, 5, 1170, 77)])
def test_collate_derivation_equals_construction_and_oracle(layout, B, L, seed):
    tokens, in_span, span_id, is_prefix = cocktail_batch(B, L, layout, seed)
    d_in, d_sid, d_pre = derive_metadata(tokens, rule="collate")
    assert torch.equal(d_in, in_span) and torch.equal(d_sid, span_id) and torch.equal(d_pre, is_prefix)
    o_in, o_sid, o_pre = ref_meta.collate_metadata(tokens.numpy())
    np.testing.assert_array_equal(d_in.numpy(), o_in)
    np.testing.assert_array_equal(d_sid.numpy(), o_sid)
    np.testing.assert_array_equal(d_pre.numpy(), o_pre)


@pytest.mark.parametrize("rule", ["fallback", "teacher_forcing"])
def test_other_rules_against_oracle_on_generator_rows(rule):
    tokens, *_ = cocktail_batch(6, 1024, CONFIG3_LAYOUT, seed=5)
    fn = {"fallback": ref_meta.fallback_metadata, "teacher_forcing": ref_meta.teacher_forcing_metadata}[rule]
    for got, want in zip(derive_metadata(tokens, rule=rule), fn(tokens.numpy())):
        np.testing.assert_array_equal(got.numpy(), want)


def test_hand_rows_with_two_and_three_spans():
    CLS, SPAN, ES, MASKQ, PAD = 1, 3, 4, 5, 0
    rows = torch.tensor([[6, CLS, 7, SPAN, 8, ES, SPAN, 9, 10, ES, MASKQ, PAD, PAD],
                         [CLS, 7, SPAN, ES, SPAN, 11, ES, 12, SPAN, 13, 14, ES, MASKQ]])
    i, s, p = derive_metadata(rows, rule="collate")
    assert s.tolist() == [[0, 0, 0, 1, 1, 1, 2, 2, 2, 2, -1, 0, 0], [0, 0, 1, 1, 2, 2, 2, 0, 3, 3, 3, 3, -1]]
    assert i.tolist() == [[bool(x > 0) for x in r] for r in s.tolist()]
    assert p.tolist() == [[True, True] + [False] * 11, [True] + [False] * 12]
