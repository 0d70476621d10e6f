"""CPU model of the forward kernel's lazy rescale: the packed P stays finite.

``k_fwd`` (kd_fwd.hip) keeps a per-row reference max ``m_ref`` and rescales O
and l only when a key tile raises the row max by more than ``R`` log2 units.
Between rescales it forms ``P = exp2(fma(S, c, -m_ref c))`` in fp32 and packs
P to the input type for the P V product.  This models that sequence in numpy,
with ``v_exp_f32`` taken one fp32 ulp high (its documented error), and checks:

* with fp16 and ``R = 16`` a jump of 15.9998 log2 units (no rescale) rounds P
  to +inf -- the failure the fp16 threshold of 15 removes;
* with the thresholds the kernel uses (16 for bf16, 15 for fp16) no jump that
  escapes the rescale, over the whole window up to the threshold and a range
  of score magnitudes, gives a non-finite packed P.
"""
import numpy as np
import pytest
import torch

THRESHOLD = {torch.bfloat16: 16.0, torch.float16: 15.0}  # rescale_log2<E> in kd_fwd.hip


def packed_p(s, c, m_ref, dtype):
    """P as k_fwd packs it: exp2 of the fp32 fma, one ulp high, rounded to dtype."""
    s, c, m_ref = (np.float32(x) for x in (s, c, m_ref))
    ms = np.float32(m_ref * c)                       # ms = m_ref * sl2 (fp32)
    e = np.float32(np.float64(s) * c - ms)           # fma: one rounding
    p = np.exp2(e.astype(np.float32))
    p = np.nextafter(p, np.float32(np.inf))          # v_exp_f32: <= 1 ulp
    return torch.from_numpy(np.atleast_1d(p)).to(dtype).float().numpy()


def escapes_rescale(m_new, m_ref, c, dtype):
    """The kernel's test: rescale iff (m_new - m_ref) * c > R."""
    return not (np.float32(np.float32(m_new) - np.float32(m_ref)) * np.float32(c) > THRESHOLD[dtype])


def test_fp16_with_threshold_16_overflows():
    # the failure the fp16 threshold removes: a jump of 15.9998 log2 units
    c = np.float32(1.0)
    s = np.float32(15.9998)
    p = packed_p(s, c, 0.0, torch.float16)
    assert np.isinf(p).all()
    assert not (np.float32(s - 0.0) * c > 16.0)  # R = 16 would not have rescaled


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scale", [1.0 / 64, 0.125, 1.0, 8.0, 700.0])
def test_unrescaled_p_is_finite_over_the_window(dtype, scale):
    R = THRESHOLD[dtype]
    c = np.float32(scale)
    for m_ref in (-5000.0, -3.0, 0.0, 0.7, 400.0):
        m_ref = np.float32(m_ref / scale)
        # jumps from R - 0.01 up to just past R, in steps far below fp32's
        # spacing at the threshold
        jumps = np.linspace(R - 0.01, R + 0.001, 4001, dtype=np.float64)
        for j in jumps:
            m_new = np.float32(np.float64(m_ref) + j / np.float64(c))
            if not escapes_rescale(m_new, m_ref, c, dtype):
                continue
            p = packed_p(m_new, c, m_ref, dtype)
            assert np.isfinite(p).all(), (dtype, scale, float(m_ref), j, p)
            assert p.max() <= 2.0 ** R * (1 + 2.0 ** -8), (dtype, scale, float(m_ref), j, p)
