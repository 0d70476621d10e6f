"""GPU: one config-5 training step (GPTModel, d_model 768, 12 layers, 12 heads of
64, SwiGLU 2048, vocab 262) through the MI355X attention, against the same
bf16 weights with a dense fp32 masked reference attention.

Only the attention differs between the two runs: the reference upcasts q/k/v
to fp32, applies torch SDPA with the dense hierarchical mask (the oracle's
formula) and casts back.  Compared: the final hidden states, the
cocktail-party span scores, and -- for a well-conditioned objective -- the
next-token loss through the tied head and every parameter's gradient.  (At
random init the span scores are O(500) and equal to within a few units, so
the cocktail-party cross entropy is decided by differences far below the
bf16 spacing of the hidden states; its gradient is not a useful comparison.)
"""
import copy

import pytest
import torch
import torch.nn.functional as F

from kerneldev_amd.gpt import GPTModel, config5_batch, span_scores
from oracle.mask import dense_mask

pytestmark = pytest.mark.gpu


def dense_reference_attention(q, k, v, lens=None, causal=True, attention_mask=None, in_span=None, span_id=None,
                              is_prefix=None):
    B, H, T, D = q.shape
    m = torch.from_numpy(dense_mask(T, B=B, in_span=in_span.cpu().numpy(), span_id=span_id.cpu().numpy(),
                                    is_prefix=is_prefix.cpu().numpy())).to(q.device)
    o = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), attn_mask=m[:, None],
                                                         scale=D ** -0.5)
    return o.to(q.dtype)


def _rel(a, b):
    a, b = a.float(), b.float()
    return ((a - b).pow(2).mean().sqrt() / b.pow(2).mean().sqrt().clamp_min(1e-30)).item()


def _step(model, batch, dev):
    tokens, in_span, span_id, is_prefix, correct = (x.to(dev) for x in batch)
    model.zero_grad(set_to_none=True)
    h = model.hidden(tokens, in_span, span_id, is_prefix)
    scores = span_scores(tokens, h)
    logits = model.head(h).float()
    loss = F.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]), tokens[:, 1:].reshape(-1), ignore_index=0)
    loss.backward()
    torch.cuda.synchronize()
    return (h.detach(), scores.detach(), loss.detach(),
            {n: p.grad.detach().float() for n, p in model.named_parameters()})


def test_config5_training_step_matches_dense_reference(dev):
    torch.manual_seed(0)
    model = GPTModel().to(dev).to(torch.bfloat16)
    ref = copy.deepcopy(model)
    for blk in ref.blocks:
        blk.attn.attention = dense_reference_attention
    batch = config5_batch(B=2, L=2048, seed=3)
    print("config5 step: kdattn", flush=True)
    h, sc, loss, grads = _step(model, batch, dev)
    print("config5 step: dense fp32 reference attention", flush=True)
    h_r, sc_r, loss_r, grads_r = _step(ref, batch, dev)
    rel_h = _rel(h, h_r)
    sc_err = (sc - sc_r).abs().max().item()
    print(f"  hidden rel-RMS {rel_h:.3e}; span scores max|diff| {sc_err:.3e} of max {sc_r.abs().max().item():.1f}; "
          f"loss {loss.item():.6f} ref {loss_r.item():.6f}")
    assert rel_h <= 1e-2
    assert sc_err <= 2e-2 * max(1.0, sc_r.abs().max().item())
    assert torch.isfinite(loss) and abs(loss.item() - loss_r.item()) <= 1e-3 * abs(loss_r.item())
    worst, worst_name = 0.0, ""
    for name, g in grads.items():
        rel = _rel(g, grads_r[name])
        if rel > worst:
            worst, worst_name = rel, name
    print(f"  worst per-parameter grad rel-RMS {worst:.3e} ({worst_name})")
    assert worst <= 2e-2, f"{worst_name}: grad rel-RMS {worst:.3e}"


def test_config5_full_batch_step_runs(dev):
    """The full config-5 batch (8 x 2048): cocktail-party loss, fwd+bwd."""
    torch.manual_seed(1)
    model = GPTModel().to(dev).to(torch.bfloat16)
    tokens, in_span, span_id, is_prefix, correct = (x.to(dev) for x in config5_batch(B=8, L=2048, seed=4))

    def step():
        model.zero_grad(set_to_none=True)
        _, loss = model(tokens, correct_idx=correct, in_span=in_span, span_id=span_id, is_prefix=is_prefix)
        loss.backward()
        return loss

    step()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    loss = step()
    end.record()
    torch.cuda.synchronize()
    print(f"  config5 step (B=8, L=2048): {start.elapsed_time(end):.1f} ms, loss {loss.item():.4f}")
    assert torch.isfinite(loss)
    assert all(torch.isfinite(p.grad).all() for p in model.parameters())
