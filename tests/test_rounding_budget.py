"""CPU: which form each product's 16-bit operand (P or dS) needs on config-4
data, from the emulation of the kernels' roundings (tests/rounding_emulation.py)
on two config-4 heads with Hadamard (the benchmarked configuration).

The per-element bar is max |x - ref| beyond one bf16 ulp <= 2e-2; a form is
taken only where it holds with a 2x margin (<= 1e-2).  What the table pins:

* the split (bf16 hi + lo, the kernels' default) holds every product with that
  margin;
* a single bf16 rounding (the reference's numerics) fails every product;
* a single fp16 rounding holds P V alone, but not dQ on either head, nor dV
  and dK with the margin on both;
* and a forward whose P V took P rounded once to fp16 breaks dQ even with a
  split backward: its O enters Delta = rowsum(dO O), and dS = P (dP - Delta)
  cancels.  So the forward stays split whenever a backward follows.
"""
import pytest

from rounding_emulation import FORMS, PRODUCTS, config4_head, emulate_head

BAR, MARGIN = 2e-2, 2.0
HEADS = [(1, 17), (0, 1)]


@pytest.fixture(scope="module")
def table():
    out = {}
    for b, h in HEADS:
        r = emulate_head(*config4_head(b, h, hadamard=True))
        out[(b, h)] = r
        for p in PRODUCTS:
            row = "  ".join(f"{f}={r['excess'][(p, f)]:.2e}" for f in FORMS)
            print(f"head ({b},{h}) {p:>2}: {row}  coupled={r['coupled'].get(p, float('nan')):.2e}")
    return out


def _worst(table, product, form):
    return max(r["excess"][(product, form)] for r in table.values())


def test_split_holds_every_product_with_margin(table):
    for p in PRODUCTS:
        assert _worst(table, p, "bf16x2") <= BAR / MARGIN, p


def test_single_bf16_rounding_fails_every_product(table):
    for p in PRODUCTS:
        assert _worst(table, p, "bf16") > BAR, p


def test_single_fp16_rounding_only_for_pv(table):
    assert _worst(table, "O", "fp16") <= BAR / MARGIN
    assert _worst(table, "dQ", "fp16") > BAR
    assert _worst(table, "dV", "fp16") > BAR / MARGIN
    assert _worst(table, "dK", "fp16") > BAR / MARGIN


def test_fp16_forward_breaks_dq_through_delta(table):
    worst = max(r["coupled"]["dQ"] for r in table.values())
    assert worst > BAR / MARGIN
    # ... although P V's own error was within the margin
    assert _worst(table, "O", "fp16") <= BAR / MARGIN
