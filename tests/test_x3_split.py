"""CPU: the operand layout of the bf16x3 path for fp32 inputs, and which kernels
flash_attention picks per dtype and head dim (kerneldev_amd.attention).

The kernels see Q' = [Qh, Qh, Ql], K' = [Kh, Kl, Kh], V' = [Vh, Vl, Vh],
dO' = [dOh, dOh, dOl] (zero-padded) and compute every product of the
attention on them; the results are combined column-block-wise.  Here each
product is formed exactly (fp64) on the expanded operands, as the kernels'
fp32 accumulation approximates it, and must match the same product of the
fp32 operands to the split's ~2^-16 -- a wrong pattern or a wrong combining
block (the mistakes this layout invites) is off by O(1) or by 2^-8.
"""
import pytest
import torch

from kerneldev_amd.attention import X3_HEAD_DIMS, _hi_lo, _x3


def _rel(x, ref):
    return ((x - ref).norm() / ref.norm()).item()


@pytest.mark.parametrize("d", sorted(X3_HEAD_DIMS))
def test_every_product_through_the_expanded_operands(d):
    g = torch.Generator().manual_seed(d)
    T, Dp = 48, X3_HEAD_DIMS[d]
    q, k, v, do = (torch.randn(1, 1, T, d, generator=g) * 3 for _ in range(4))
    p = torch.softmax(torch.randn(T, T, generator=g, dtype=torch.float64), dim=-1)
    ds = torch.randn(T, T, generator=g, dtype=torch.float64)
    qx, kx, vx, dox = (_x3(x, pat, Dp)[0, 0].double() for x, pat in ((q, "hhl"), (k, "hlh"), (v, "hlh"), (do, "hhl")))
    q, k, v, do = (x[0, 0].double() for x in (q, k, v, do))
    assert qx.shape == (T, Dp) and (qx[:, 3 * d:] == 0).all()
    bound = 2.0 ** -15
    # scores and dP: one product over the expanded head dim
    assert _rel(qx @ kx.T, q @ k.T) < bound
    assert _rel(dox @ vx.T, do @ v.T) < bound
    zero = torch.zeros(T, Dp, dtype=torch.float64)
    # outputs: O = P V' in blocks [0, d) + [d, 2d); dQ = dS K' in [0, d) + [d, 2d);
    # dK = dS^T Q' and dV = P^T dO' in [0, d) + [2d, 3d)
    assert _rel(_hi_lo(p @ vx, zero, d, 1), p @ v) < bound
    assert _rel(_hi_lo(ds @ kx, zero, d, 1), ds @ k) < bound
    assert _rel(_hi_lo(ds.T @ qx, zero, d, 2), ds.T @ q) < bound
    assert _rel(_hi_lo(p.T @ dox, zero, d, 2), p.T @ do) < bound


def test_hi_lo_adds_the_residual():
    x = torch.randn(2, 3, 5, 64, dtype=torch.float32)
    hi = x.to(torch.bfloat16)
    lo = (x - hi.float()).to(torch.bfloat16)
    got = _hi_lo(hi, lo, 16, 2)
    want = (hi.float() + lo.float())[..., :16] + (hi.float() + lo.float())[..., 32:48]
    assert torch.equal(got, want)
    assert _rel(got.double(), (x[..., :16] + x[..., 32:48]).double()) < 2.0 ** -15


def test_head_dim_route():
    """flash_attention's choice of kernels per dtype, head dim and precision."""
    from kerneldev_amd.attention import head_dim_route

    bf, f32 = torch.bfloat16, torch.float32
    # 16-bit inputs go to the MFMA kernels unpadded at every head dim
    assert not any(head_dim_route(bf, d, p) for d in (16, 32, 64, 128, 256) for p in ("tf32", "ieee", "bf16"))
    assert not head_dim_route(torch.float16, 128, "ieee")
    # fp32: bf16x3 at "tf32" and d = 16, 32; the fp32 MFMA kernels, unpadded, otherwise
    assert head_dim_route(f32, 16, "tf32") and head_dim_route(f32, 32, "tf32")
    assert not head_dim_route(f32, 64, "tf32") and not head_dim_route(f32, 128, "tf32")
    assert not any(head_dim_route(f32, d, "ieee") for d in (16, 32, 64, 128, 256))
