"""CPU: the parity metric in tests/helpers.py (what the GPU tests assert with)."""
import torch

from helpers import REF_ZERO, assert_close, errors, single_key_rows


def test_relative_error_and_ulp_excess():
    ref = torch.tensor([1.0, -2.0, 0.5, 4.0], dtype=torch.float64)
    x = ref + torch.tensor([1e-3, 0.0, -1e-3, 0.0], dtype=torch.float64)
    ma, rr, ex = errors(x, ref, out_dtype=torch.float32)
    assert abs(ma - 1e-3) < 1e-12 and abs(ex - (1e-3 - 2.0 ** -24)) < 1e-12  # ulp of 0.5 in fp32
    assert abs(rr - (2e-6 / 4) ** 0.5 / ((1 + 4 + 0.25 + 16) / 4) ** 0.5) < 1e-9
    # one bf16 ulp at 4.0 is 2^-5: an error of 0.03 there is within it
    _, _, ex = errors(torch.tensor([4.03], dtype=torch.float64), torch.tensor([4.0], dtype=torch.float64),
                      out_dtype=torch.bfloat16)
    assert ex == 0.0


def test_zero_reference_has_no_relative_scale():
    """A reference that is 0 to fp64 rounding (dQ with one allowed key per row) is checked by
    the absolute bar only, when the caller says the exact result is zero; a real error there
    still fails it, and without that flag a tiny reference keeps the relative bar."""
    ref = torch.full((4, 8), 3e-16, dtype=torch.float64)
    assert ref.pow(2).mean().sqrt().item() <= REF_ZERO
    x = ref + 2e-7
    ma, rr, _ = errors(x, ref, out_dtype=torch.float32, zero_ref_ok=True)
    assert rr == 0.0 and ma < 3e-7
    assert_close("dq", x, ref, out_dtype=torch.float32, zero_ref_ok=True)
    for bad, flag in ((ref + 0.5, True), (x, False)):
        try:
            assert_close("dq", bad, ref, out_dtype=torch.float32, zero_ref_ok=flag)
        except AssertionError:
            pass
        else:
            raise AssertionError(f"error {float((bad - ref).abs().max()):.1e} passed (zero_ref_ok={flag})")
    # a tiny but genuine reference (inputs scaled by 1e-14) is held to the relative bar
    small = torch.linspace(-1, 1, 32, dtype=torch.float64) * 1e-14
    _, rr, _ = errors(small * 1.1, small, out_dtype=torch.float32)
    assert abs(rr - 0.1) < 1e-9


def test_single_key_rows():
    eye = torch.eye(5, dtype=torch.bool)[None]
    assert single_key_rows(eye) and single_key_rows(torch.zeros(1, 3, 3, dtype=torch.bool))
    assert not single_key_rows(torch.ones(1, 2, 2, dtype=torch.bool).tril())
