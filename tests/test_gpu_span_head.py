"""GPU: the cocktail-party head kernels (kd_span_scores / kd_span_scores_bwd)
against the CPU oracle (``oracle/span_head.py``, fp64 on the same bf16 / fp16
values).

Bars: span bounds and the [MASK] position exact; scores within fp32 summation
error (|err| <= 1e-5 * sum_d |mean_d ctx_d| + 1e-6); dh within the rounding of
the output dtype (|err| <= 2^-8 |ref| + 1e-6 max |ref| for bf16, 2^-11 for
fp16).
"""
import pytest
import torch

from kerneldev_amd.span_head import _span_fwd_op, max_spans, span_scores
from kerneldev_amd.synth import CONFIG3_LAYOUT, cocktail_batch
from oracle import span_head as ref

pytestmark = pytest.mark.gpu

MASK, SPAN, ES, X = 2, 3, 4, 100


def _bounds(tokens, n):
    """Oracle interiors and first-[MASK] positions from the token lists."""
    B = tokens.shape[0]
    lo = torch.zeros(B, n, dtype=torch.int32)
    hi = torch.zeros(B, n, dtype=torch.int32)
    mp = torch.full((B,), -1, dtype=torch.int32)
    for i in range(B):
        t = tokens[i].tolist()
        sts = [p for p, v in enumerate(t) if v == SPAN]
        eds = [p for p, v in enumerate(t) if v == ES]
        for j in range(min(len(sts), len(eds), n)):
            if sts[j] + 1 < eds[j]:
                lo[i, j], hi[i, j] = sts[j] + 1, eds[j]
        if MASK in t:
            mp[i] = t.index(MASK)
    return lo, hi, mp


def _check(tokens, h, dev, seed=0, strided=False):
    """strided: h [B, T, D] is handed over as slice 1 of a [B, T, 3, D] tensor (t stride 3 D)."""
    print(f"span head B={h.shape[0]} T={h.shape[1]} D={h.shape[2]} {h.dtype} tokens {tokens.dtype} "
          f"strided={strided}", flush=True)
    n = max_spans(tokens)
    if strided:
        leaf = torch.zeros(h.shape[0], h.shape[1], 3, h.shape[2], dtype=h.dtype, device=dev)
        leaf[:, :, 1] = h.to(dev)
        leaf.requires_grad_(True)
        hd = leaf[:, :, 1, :]
    else:
        leaf = h.to(dev).requires_grad_(True)
        hd = leaf
    scores, h_ctx, h_spans, lo, hi, mp = _span_fwd_op(tokens.to(dev), hd, n)
    g = torch.Generator().manual_seed(seed)
    ds = torch.randn(scores.shape, generator=g, dtype=torch.float32)
    (scores * ds.to(dev)).sum().backward()
    torch.cuda.synchronize()
    grad = leaf.grad[:, :, 1, :] if strided else leaf.grad
    wlo, whi, wmp = _bounds(tokens.cpu(), n)
    assert torch.equal(lo.cpu(), wlo) and torch.equal(hi.cpu(), whi) and torch.equal(mp.cpu(), wmp)
    h64 = h.detach().cpu().double().requires_grad_(True)
    want = ref.scores(tokens.cpu().long(), h64, n)
    (want * ds.double()).sum().backward()
    # |sum_d mean_d ctx_d| error bound from the magnitudes of the terms
    ctx = torch.stack([h64.detach()[i, m] if m >= 0 else torch.zeros(h.shape[2], dtype=torch.float64)
                       for i, m in enumerate(wmp.tolist())])
    mag = torch.zeros_like(want)
    for i in range(want.shape[0]):
        for j in range(n):
            if whi[i, j] > wlo[i, j]:
                mag[i, j] = (h64.detach()[i, wlo[i, j]:whi[i, j]].mean(0) * ctx[i]).abs().sum()
    err = (scores.detach().cpu().double() - want.detach()).abs()
    assert bool((err <= 1e-5 * mag + 1e-6).all()), f"score error {err.max().item():.3e}"
    got, wg = grad.cpu().double(), h64.grad
    ulp = 2.0 ** -8 if h.dtype == torch.bfloat16 else 2.0 ** -11
    bad = (got - wg).abs() > ulp * wg.abs() + 1e-6 * wg.abs().max()
    assert not bool(bad.any()), f"{int(bad.sum())} dh entries off; max err {(got - wg).abs().max().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config5_batch(dev, dtype):
    tokens, *_ = cocktail_batch(8, 2048, CONFIG3_LAYOUT, 3)
    g = torch.Generator().manual_seed(1)
    h = torch.randn(8, 2048, 768, generator=g).to(dtype)
    _check(tokens, h, dev)


def test_malformed_rows_int32_tokens_strided_h(dev):
    T = 40
    rows = [[MASK, SPAN, SPAN, X, ES, X, ES] + [X] * (T - 7),            # nested pairs
            [X, ES, X, MASK, SPAN, X, X] + [X] * (T - 7),                # [ES] before [SPAN]
            [SPAN, ES, MASK, SPAN, X, X, ES, MASK, SPAN] + [X] * (T - 9),  # empty, normal, unpaired
            [X] * 5 + [SPAN, X, X, ES] + [X] * (T - 9),                  # no [MASK]: zero scores
            [MASK] + [X] * (T - 1)]                                      # no spans in the row
    tokens = torch.tensor(rows, dtype=torch.int32)
    g = torch.Generator().manual_seed(2)
    h = torch.randn(5, T, 96, generator=g).to(torch.bfloat16)
    _check(tokens, h, dev, seed=4, strided=True)


def test_many_overlapping_spans_odd_width(dev):
    """100 spans in a row (the backward's span ballot runs in two chunks of 64), a row
    of 70 nested [SPAN]s then 70 [ES]s whose zipped interiors all overlap (a token
    in up to 70 spans, added in ascending span order across the chunk boundary),
    and widths that are not multiples of the kernels' 64- and 256-column chunks."""
    T = 420
    r0 = [MASK] + [SPAN, X, X, ES] * 100
    r1 = [MASK] + [SPAN] * 70 + [X] * 5 + [ES] * 70
    r2 = [X] * 3 + [MASK] + [SPAN, X, ES] * 40
    rows = [r + [X] * (T - len(r)) for r in (r0, r1, r2)]
    tokens = torch.tensor(rows, dtype=torch.int64)
    g = torch.Generator().manual_seed(6)
    for D in (300, 600):
        h = torch.randn(3, T, D, generator=g).to(torch.bfloat16)
        _check(tokens, h, dev, seed=D)


def test_public_entry_and_errors(dev):
    tokens = torch.tensor([[MASK, SPAN, X, X, ES, X]], device=dev)
    h = torch.randn(1, 6, 64, device=dev).to(torch.bfloat16)
    s = span_scores(tokens, h)
    torch.cuda.synchronize()
    want = (h[0, 2:4].float().mean(0) * h[0, 0].float()).sum()
    assert torch.allclose(s[0, 0], want, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        span_scores(torch.tensor([[MASK, X, X]], device=dev), torch.randn(1, 3, 8, device=dev).bfloat16())
    with pytest.raises(ValueError):
        span_scores(tokens, h.float())
