"""GPT training-step harness through the MI355X attention.

A restatement of KernelDev's ``GPTModel`` (``model.py:31-117`` blocks,
``:127-314`` model), the hot path's only caller: token + position embeddings,
pre-norm blocks of weightless RMSNorm -> ``MultiHeadAttention`` -> residual and
RMSNorm -> SwiGLU -> residual, a final RMSNorm, a head tied to the token
embedding, N(0, 0.02) init (``:174-178``).  Attention goes through
``flash_attention`` with the mask metadata, exactly as ``model.py:73-96``
calls it; the q/k/v projections are handed over as strided ``[B, H, L, d]``
views of ``[B, L, H, d]``, without copies, and O comes back in ``[B, L, H, d]``
memory (``out_layout="bthd"``), so ``o_proj`` reads it without a copy either.

The cocktail-party head (``model.py:250-298``) scores the hidden state at the
first ``[MASK]`` against the mean hidden state of each span's interior
(``[SPAN] x.. [ES]`` minus the markers) and takes the cross entropy against
``correct_idx``; spans a row does not have score 0, as the reference's
zero-padded ``h_spans`` do.  The pooling and the scores run in the
``kd_span_scores`` kernels (``span_head.py``) instead of the reference's Python
double loop, and the scores are fp32.

``attention`` is injectable so a test can run the same weights through a
dense fp32 reference attention.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import AttentionPlan, build_plan, build_plan_from_tokens, flash_attention, mask_mode
from .metadata import CLS, MASKQ, SPAN, derive_metadata
from .span_head import has_cocktail_layout, span_scores

VOCAB = 256 + 6  # byte tokens + [PAD] [CLS] [MASK] [SPAN] [ES] [MASKQ] (data_builder.py:44-52)


class RMSNorm(nn.Module):
    """x / rms(x), no weight (model.py:31-39)."""

    def __init__(self, eps: float = 1e-6):
        super().__init__()
        self.eps = eps

    def forward(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)


class SwiGLU(nn.Module):
    """w2(silu(w1 x) * w3 x) (model.py:42-52)."""

    def __init__(self, dim: int, hidden: int):
        super().__init__()
        self.w1 = nn.Linear(dim, hidden, bias=False)
        self.w2 = nn.Linear(hidden, dim, bias=False)
        self.w3 = nn.Linear(dim, hidden, bias=False)

    def forward(self, x):
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class MultiHeadAttention(nn.Module):
    """q/k/v projections -> flash_attention -> o_proj (model.py:58-96)."""

    def __init__(self, dim: int, n_heads: int, causal: bool = True, attention=None):
        super().__init__()
        self.n_heads, self.head_dim, self.causal = n_heads, dim // n_heads, causal
        self.q_proj = nn.Linear(dim, dim, bias=False)
        self.k_proj = nn.Linear(dim, dim, bias=False)
        self.v_proj = nn.Linear(dim, dim, bias=False)
        self.o_proj = nn.Linear(dim, dim, bias=False)
        self.attention = attention or flash_attention

    def forward(self, x, in_span, span_id, is_prefix, plan=None):
        B, L, _ = x.shape
        shape = (B, L, self.n_heads, self.head_dim)
        q = self.q_proj(x).view(shape).transpose(1, 2)
        k = self.k_proj(x).view(shape).transpose(1, 2)
        v = self.v_proj(x).view(shape).transpose(1, 2)
        if plan is not None:  # the model's shared plan stands for the metadata
            # flash_attention writes O straight into [B, L, H, d] memory, so the
            # transpose + reshape below is a view rather than model.py:95's copy
            out = flash_attention(q, k, v, causal=self.causal, plan=plan, out_layout="bthd")
        else:
            out = self.attention(q, k, v, lens=None, causal=self.causal, attention_mask=None,
                                 in_span=in_span, span_id=span_id, is_prefix=is_prefix)
        return self.o_proj(out.transpose(1, 2).reshape(B, L, -1))


class Block(nn.Module):
    def __init__(self, dim, n_heads, hidden, causal=True, attention=None):
        super().__init__()
        self.norm1, self.norm2 = RMSNorm(), RMSNorm()
        self.attn = MultiHeadAttention(dim, n_heads, causal, attention)
        self.mlp = SwiGLU(dim, hidden)

    def forward(self, x, in_span, span_id, is_prefix, plan=None):
        x = x + self.attn(self.norm1(x), in_span, span_id, is_prefix, plan)
        return x + self.mlp(self.norm2(x))


class GPTModel(nn.Module):
    """Config 5: d_model 768, 12 layers, 12 heads of 64, SwiGLU 2048, vocab 262."""

    def __init__(self, vocab_size=VOCAB, dim=768, n_layers=12, n_heads=12, max_seq_len=2048, mlp_hidden=2048,
                 causal=True, attention=None):
        super().__init__()
        self.token_emb = nn.Embedding(vocab_size, dim)
        self.pos_emb = nn.Embedding(max_seq_len, dim)
        self.blocks = nn.ModuleList(Block(dim, n_heads, mlp_hidden, causal, attention) for _ in range(n_layers))
        self.norm_out = RMSNorm()
        self.head = nn.Linear(dim, vocab_size, bias=False)
        self.head.weight = self.token_emb.weight  # tied (model.py:170)
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, mean=0.0, std=0.02)

    def hidden(self, tokens, in_span, span_id, is_prefix, plan=None):
        pos = torch.arange(tokens.shape[1], device=tokens.device)
        h = self.token_emb(tokens) + self.pos_emb(pos)[None]
        for blk in self.blocks:
            h = blk(h, in_span, span_id, is_prefix, plan)
        return self.norm_out(h)

    def plan(self, tokens, in_span=None, span_id=None, is_prefix=None) -> AttentionPlan | None:
        """One tile plan for every layer: from the given metadata (the training
        path's collate metadata, model.py:197-201), else straight from the tokens
        by the model's fallback rule (model.py:209-240) on the device.  None when
        the blocks run an injected reference attention."""
        attn = self.blocks[0].attn
        if attn.attention is not flash_attention:
            return None
        B, T = tokens.shape
        if in_span is None or span_id is None or is_prefix is None:
            return build_plan_from_tokens(tokens, attn.head_dim, rule="fallback")
        mode = mask_mode(in_span, span_id, is_prefix, None, attn.causal)
        return AttentionPlan(build_plan(B, T, attn.head_dim, tokens.device, mode, in_span, span_id, is_prefix),
                             B, T, attn.head_dim)

    def forward(self, tokens, correct_idx=None, in_span=None, span_id=None, is_prefix=None, targets=None):
        """Cocktail-party scores and loss, or LM logits and loss (model.py:180-314)."""
        plan = self.plan(tokens, in_span, span_id, is_prefix)
        if plan is None and (in_span is None or span_id is None or is_prefix is None):
            in_span, span_id, is_prefix = derive_metadata(tokens, rule="fallback")
        h = self.hidden(tokens, in_span, span_id, is_prefix, plan)
        if has_cocktail_layout(tokens):
            scores = span_scores(tokens, h)
            loss = F.cross_entropy(scores, correct_idx) if correct_idx is not None else None
            return scores, loss
        logits = self.head(h)
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1), ignore_index=0)
        return logits, loss


def config5_batch(B=8, L=2048, seed=0):
    """Config-3-generator sequences at L, collate metadata, seeded correct_idx."""
    from .synth import CONFIG3_LAYOUT, cocktail_batch

    tokens, in_span, span_id, is_prefix = cocktail_batch(B, L, CONFIG3_LAYOUT, seed)
    n_spans = (tokens == SPAN).sum(dim=1)
    g = torch.Generator("cpu").manual_seed(seed + 7)
    correct = (torch.rand(B, generator=g) * n_spans.to(torch.float32)).to(torch.int64)
    return tokens, in_span, span_id, is_prefix, correct


__all__ = ["GPTModel", "span_scores", "config5_batch", "VOCAB", "CLS", "MASKQ"]
