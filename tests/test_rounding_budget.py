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
import numpy as np
import pytest
import torch

from oracle import attention as oracle_attention
from rounding_emulation import FORMS, LOG2E, PRODUCTS, as_form, bf16_round, config4_head, emulate_head, head_qkvdo

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


def test_bf16_round_is_torchs_round_to_nearest_even():
    """The emulation's bf16 rounding equals torch's fp32 -> bf16 cast, ties included."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(20000) * np.exp2(rng.integers(-40, 40, 20000))).astype(np.float32)
    ties = (rng.integers(1 << 23, 1 << 30, 4000, dtype=np.uint32) & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
    x = np.concatenate([x, ties.view(np.float32), -ties.view(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(bf16_round(x).view(np.uint32), want.view(np.uint32))
    # the split's two parts carry what one rounding drops: |x - (hi + lo)| <= 2^-16 |x|
    # (where x - hi is still a normal fp32 number)
    x = x[np.abs(x) >= 2.0 ** -100]
    rel = np.abs(as_form(x, "bf16x2") - x.astype(np.float64)) / np.abs(x.astype(np.float64))
    assert rel.max() <= 2.0 ** -16


def test_emulation_reference_is_the_oracle():
    """The fp64 results the excesses are measured against are the oracle's attention
    (original_kernel.py:550-579, :1239-1335, :1425-1524 restated in oracle/attention.py),
    over several query blocks, with a fully masked row and a row with one key."""
    rng = np.random.default_rng(3)
    T, d = 150, 32
    q, k, v, do = (bf16_round(rng.standard_normal((T, d)).astype(np.float32)) for _ in range(4))
    mask = rng.random((T, T)) < 0.3
    mask[5] = False
    mask[9] = False
    mask[9, 40] = True
    sm_scale = 0.125 / LOG2E  # sm_scale log2(e) exact in fp32, as the kernels hold it
    refs = emulate_head(q, k, v, do, mask, sm_scale, block=64)["refs"]
    t = [torch.from_numpy(x.astype(np.float64))[None, None] for x in (q, k, v, do)]
    m = torch.from_numpy(mask)[None]
    o, _ = oracle_attention.forward(t[0], t[1], t[2], m, sm_scale)
    dq, dk, dv, _ = oracle_attention.backward(t[0], t[1], t[2], o, t[3], m, sm_scale)
    for name, want in (("O", o), ("dQ", dq), ("dK", dk), ("dV", dv)):
        np.testing.assert_allclose(refs[name], want[0, 0].numpy(), rtol=1e-9, atol=1e-12, err_msg=name)


def test_head_generator_is_the_config_generator():
    """head_qkvdo (config4_head's inputs, one head at a time) equals the head
    of synth.qkvdo, outlier channels included, here on a small shape."""
    from kerneldev_amd.synth import qkvdo

    full = qkvdo(2, 3, 96, 64, seed=5, outlier_frac=0.05)
    for b, h in ((0, 0), (1, 2), (0, 1)):
        for x, y in zip(full, head_qkvdo(b, h, 2, 3, 96, 64, seed=5, outlier_frac=0.05)):
            assert torch.equal(x[b, h], y)
