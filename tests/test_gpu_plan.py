"""GPU: the tile classifier, work lists and dense mask are bit-exact.

Compares the device plan (``kd_plan_build``) and ``return_attention_mask``
output against the oracle's dense mask (``original_kernel.py:478-517``) and
its exhaustive tile reduction, on the benchmark configurations and on
ragged / fuzzed metadata.
"""
import numpy as np
import pytest
import torch

from kerneldev_amd import build_plan, build_plan_from_tokens, derive_metadata, flash_attention, plan_views
from kerneldev_amd.attention import mask_mode, tile_masks
from kerneldev_amd.synth import CONFIG3_LAYOUT, CONFIG4_LAYOUT, cocktail_batch
from oracle import metadata, tilemap
from oracle.mask import dense_mask

pytestmark = pytest.mark.gpu


def _views(plan, B, T, D):
    """The plan's sections, plus every tile's row / column masks as the kernels build them."""
    out = {k: (v.cpu().numpy() if torch.is_tensor(v) else v) for k, v in plan_views(plan, B, T, D).items()}
    rows, cols = tile_masks(plan, B, T, D)
    torch.cuda.synchronize()
    out["qbits"], out["kbits"] = rows.cpu().numpy(), cols.cpu().numpy()
    return out


def _device_plan(dev, B, T, D, in_span=None, span_id=None, is_prefix=None, lens=None, causal=True,
                 attention_mask_given=False):
    to = lambda t: None if t is None else t.to(dev)
    mode = mask_mode(in_span, span_id, is_prefix, True if attention_mask_given else None, causal)
    plan = build_plan(B, T, D, dev, mode, to(in_span), to(span_id), to(is_prefix), to(lens))
    torch.cuda.synchronize()
    return _views(plan, B, T, D)


def _check_plan(p, mask):
    B, T, _ = mask.shape
    L = p["layout"]
    cls = tilemap.classify(mask, 64)
    np.testing.assert_array_equal(p["cls"], cls)
    n = L["nT"]
    pad = np.zeros((B, n * 64, n * 64), bool)
    pad[:, :T, :T] = mask
    cnt = pad.reshape(B, n, 64, n, 64).sum(axis=(2, 4))
    np.testing.assert_array_equal(p["nnz"], cnt)
    for name, group, fn in (("fwd", L["fwd_group"], tilemap.q_lists), ("dq", L["dq_group"], tilemap.q_lists),
                            ("dkdv", L["dkdv_group"], tilemap.k_lists)):
        ent, counts = fn(cls, group)
        np.testing.assert_array_equal(p[f"{name}_count"], counts, err_msg=name)
        np.testing.assert_array_equal(p[f"{name}_list"].view(np.uint32), ent, err_msg=name)
        # work order: descending count, ties by ascending item (a stable sort of -count)
        flat = np.asarray(counts).reshape(-1)
        np.testing.assert_array_equal(p[f"{name}_order"], np.argsort(-flat, kind="stable"), err_msg=name)
    # row / column bit masks as the kernels build them from the codes (kd_tile_masks),
    # bit-exact on every tile (the kernels use them on PARTIAL tiles)
    qbits, kbits = tilemap.tile_bits(mask, 64)
    np.testing.assert_array_equal(p["qbits"].view(np.uint64), qbits, err_msg="row masks")
    np.testing.assert_array_equal(p["kbits"].view(np.uint64), kbits, err_msg="column masks")


@pytest.mark.parametrize("T,causal", [(256, True), (2048, True), (200, False), (1, True), (77, True)])
def test_plan_no_metadata(dev, T, causal):
    B = 2
    print(f"plan no-metadata T={T} causal={causal}", flush=True)
    p = _device_plan(dev, B, T, 64, causal=causal)
    _check_plan(p, dense_mask(T, B=B, causal=causal))


def test_plan_attention_mask_defaults_to_tril(dev):
    T = 300
    p = _device_plan(dev, 1, T, 128, causal=False, attention_mask_given=True)
    _check_plan(p, dense_mask(T, B=1, causal=False, attention_mask_given=True))


def test_plan_config3(dev):
    tokens, in_span, span_id, is_prefix = cocktail_batch(16, 1024, CONFIG3_LAYOUT, seed=0)
    print("plan config3", flush=True)
    p = _device_plan(dev, 16, 1024, 64, in_span, span_id, is_prefix)
    m = dense_mask(1024, in_span=in_span.numpy(), span_id=span_id.numpy(), is_prefix=is_prefix.numpy())
    _check_plan(p, m)


def test_plan_config4(dev):
    tokens, in_span, span_id, is_prefix = cocktail_batch(2, 8192, CONFIG4_LAYOUT, seed=0)
    print("plan config4", flush=True)
    p = _device_plan(dev, 2, 8192, 128, in_span, span_id, is_prefix)
    m = dense_mask(8192, in_span=in_span.numpy(), span_id=span_id.numpy(), is_prefix=is_prefix.numpy())
    _check_plan(p, m)


@pytest.mark.parametrize("seed", range(6))
def test_plan_fuzzed_metadata(dev, seed):
    rng = np.random.default_rng(seed)
    B = 3
    T = int(rng.integers(1, 400))
    in_span = torch.from_numpy(rng.random((B, T)) < 0.4)
    is_prefix = torch.from_numpy(rng.random((B, T)) < 0.2)
    # large, repeated and negative span ids; non-contiguous spans sharing an id
    pool = np.array([-1, 0, 1, 2, 7, 2 ** 40 + 3, 2 ** 40 + 3 + 2 ** 32, -5], np.int64)
    span_id = torch.from_numpy(pool[rng.integers(0, len(pool), (B, T))])
    lens = torch.from_numpy(rng.integers(0, T + 3, (B,)).astype(np.int32))
    which = seed % 3
    if which == 1:
        span_id = span_id.to(torch.int32).clamp(-5, 7)  # int32 path
    kw = dict(in_span=in_span, span_id=span_id, is_prefix=is_prefix)
    if which == 2:
        kw["is_prefix"] = None
    print(f"plan fuzz seed={seed} T={T}", flush=True)
    p = _device_plan(dev, B, T, 64, lens=lens, **kw)
    m = dense_mask(T, B=B, lens=lens.numpy(), **{k: (None if v is None else v.numpy()) for k, v in kw.items()})
    _check_plan(p, m)


def test_plan_spans_across_rounds(dev):
    """Rows longer than the codes kernel's 8192-token round, with a span running across the
    boundary: row 0's ids increase from span to span (each token's own run is its group's
    first), row 1 reuses a few ids in separate spans (the first run with the id is earlier)."""
    T, B = 8192 + 333, 2
    rng = np.random.default_rng(5)
    in_span = np.zeros((B, T), bool)
    span_id = np.zeros((B, T), np.int64)
    is_prefix = np.zeros((B, T), bool)
    is_prefix[:, :40] = True
    for b in range(B):
        t, sid = 40, 0
        while t < T:
            t += int(rng.integers(1, 30))
            n = int(rng.integers(1, 120))
            sid = sid + 1 if b == 0 else int(rng.integers(1, 6))
            in_span[b, t:t + n] = True
            span_id[b, t:t + n] = sid
            t += n
        in_span[b, 8192 - 5:8192 + 5] = True
        span_id[b, 8192 - 5:8192 + 5] = span_id[b, 8192 - 5] if span_id[b, 8192 - 5] > 0 else 3
    kw = dict(in_span=torch.from_numpy(in_span), span_id=torch.from_numpy(span_id),
              is_prefix=torch.from_numpy(is_prefix))
    print(f"plan spans across rounds T={T}", flush=True)
    p = _device_plan(dev, B, T, 64, **kw)
    _check_plan(p, dense_mask(T, in_span=in_span, span_id=span_id, is_prefix=is_prefix))


@pytest.mark.parametrize("rule", ["collate", "fallback"])
def test_plan_from_tokens_long_row(dev, rule):
    """Token rows longer than the codes kernel's 8192-token round: a well-formed
    cocktail-party row (config 4's layout, collate rule) and a random row over the
    special ids (fallback rule), against the oracle's metadata, mask and tiles."""
    T = 8192 + 500
    if rule == "collate":
        tokens, _, _, _ = cocktail_batch(1, T, CONFIG4_LAYOUT, seed=41)
    else:
        rng = np.random.default_rng(42)
        tokens = torch.from_numpy(rng.choice(np.array([0, 1, 2, 3, 4, 5, 40, 41, 42]), size=(1, T),
                                             p=[.1, .01, .01, .03, .03, .01, .35, .38, .08]))
    print(f"plan from tokens, long row, rule={rule} T={T}", flush=True)
    got = build_plan_from_tokens(tokens.to(dev), 64, rule=rule)
    torch.cuda.synchronize()
    in_span, span_id, is_prefix = ORACLE_RULES[rule](tokens.numpy())
    _check_plan(_views(got.tensor, 1, T, 64),
                dense_mask(T, B=1, in_span=in_span, span_id=span_id, is_prefix=is_prefix))


def test_plan_strided_metadata(dev):
    rng = np.random.default_rng(11)
    T = 333
    base_span = torch.from_numpy(rng.random((2, 2 * T)) < 0.5)
    base_sid = torch.from_numpy(rng.integers(-1, 4, (2, 2 * T)))
    base_pre = torch.from_numpy(rng.random((2, 2 * T)) < 0.3)
    kw = dict(in_span=base_span[:, ::2], span_id=base_sid[:, ::2], is_prefix=base_pre[:, ::2])
    p = _device_plan(dev, 2, T, 64, **kw)
    m = dense_mask(T, B=2, **{k: v.numpy() for k, v in kw.items()})
    _check_plan(p, m)


@pytest.mark.parametrize("T", [64, 130])
def test_return_attention_mask_bit_exact(dev, T):
    tokens, in_span, span_id, is_prefix = cocktail_batch(2, 512, CONFIG3_LAYOUT, seed=7)
    in_span, span_id, is_prefix = in_span[:, :T], span_id[:, :T], is_prefix[:, :T]
    q = torch.randn(2, 3, T, 64, device=dev, dtype=torch.bfloat16)
    _, mask = flash_attention(q, q, q, in_span=in_span.to(dev), span_id=span_id.to(dev),
                              is_prefix=is_prefix.to(dev), return_attention_mask=True)
    ref = dense_mask(T, in_span=in_span.numpy(), span_id=span_id.numpy(), is_prefix=is_prefix.numpy())
    got = mask.cpu().numpy()
    for h in range(3):
        np.testing.assert_array_equal(got[:, h], ref)


def _token_batches():
    """Well-formed cocktail rows, and random rows over the special ids (nested
    [SPAN]s, [ES] before [SPAN], several [CLS] / [MASKQ], none at all)."""
    tokens, _, _, _ = cocktail_batch(3, 1024, CONFIG3_LAYOUT, seed=31)
    rng = np.random.default_rng(32)
    rand = rng.choice(np.array([0, 1, 2, 3, 4, 5, 40, 41, 42]), size=(3, 777), p=[.1, .02, .02, .08, .08, .02, .3, .3, .08])
    rand[2, :] = 50  # no special token at all
    return [tokens, torch.from_numpy(rand).to(torch.int32)]


ORACLE_RULES = {"collate": metadata.collate_metadata, "fallback": metadata.fallback_metadata,
                "teacher_forcing": metadata.teacher_forcing_metadata}


@pytest.mark.parametrize("rule", ["collate", "fallback", "teacher_forcing"])
def test_plan_from_tokens_against_oracle(dev, rule):
    """kd_plan_build_tokens against the oracle: metadata by the rule's per-token
    restatement (oracle/metadata.py), dense mask, exhaustive tile reduction.

    The collate rule (data_builder.py:603-643) marks spans from the builder's
    own span list, so it is defined on well-formed rows only; the fallback
    (model.py:209-240) and teacher-forcing (train_loop.py:406-435) rules are
    token scans and are checked on the malformed rows too."""
    batches = _token_batches()
    if rule == "collate":
        batches = batches[:1]
    for tokens in batches:
        print(f"plan from tokens vs oracle rule={rule} shape={tuple(tokens.shape)} {tokens.dtype}", flush=True)
        tk = tokens.to(dev)
        B, T = tk.shape
        in_span, span_id, is_prefix = ORACLE_RULES[rule](tokens.numpy())
        for D in (64, 128):
            lens = np.array([T, T // 2, 1][:B], dtype=np.int32)
            for ln in (None, lens):
                got = build_plan_from_tokens(tk, D, rule=rule, lens=None if ln is None else torch.from_numpy(ln).to(dev))
                torch.cuda.synchronize()
                p = _views(got.tensor, B, T, D)
                m = dense_mask(T, B=B, in_span=in_span, span_id=span_id, is_prefix=is_prefix, lens=ln)
                _check_plan(p, m)


def test_flash_attention_with_shared_plan(dev):
    """flash_attention(plan=...) == flash_attention(metadata) bit for bit, forward and backward."""
    tokens, in_span, span_id, is_prefix = cocktail_batch(2, 1024, CONFIG3_LAYOUT, seed=33)
    from kerneldev_amd.synth import qkvdo

    q0, k0, v0, do = (x.to(dev) for x in qkvdo(2, 3, 1024, 64, seed=34))
    plan = build_plan_from_tokens(tokens.to(dev), 64, rule="collate")
    meta = [x.to(dev) for x in derive_metadata(tokens.to(dev), rule="collate")]
    res = []
    for use_plan in (False, True):
        q, k, v = (x.detach().requires_grad_(True) for x in (q0, k0, v0))
        if use_plan:
            o = flash_attention(q, k, v, plan=plan)
        else:
            o = flash_attention(q, k, v, in_span=meta[0], span_id=meta[1], is_prefix=meta[2])
        o.backward(do)
        torch.cuda.synchronize()
        res.append((o.detach(), q.grad, k.grad, v.grad))
    for x, y in zip(*res):
        assert torch.equal(x, y)
    with pytest.raises(ValueError, match="plan replaces"):
        flash_attention(q0, k0, v0, plan=plan, in_span=meta[0])
    with pytest.raises(ValueError, match="plan is for"):
        flash_attention(q0[:, :, :512], k0[:, :, :512], v0[:, :, :512], plan=plan)
