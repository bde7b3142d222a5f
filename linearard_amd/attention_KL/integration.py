"""Autograd boundary: ``AttnKLAlignFn`` / ``attn_kl_align`` (mirrors integration.py:6-73).

``attn_kl_align(qs, ks, qt, kt, attn_mask=None, causal=True,
sm_scale_s=None, sm_scale_t=None)`` returns the 0-d float32 SUM over rows of
KL(P_t || P_s), P_x = softmax of the (masked, causal) relation logits
sm_scale_x * q_x . k_x.  Gradients flow to qs and ks only; the teacher,
mask, causal flag and scales get None (integration.py:67).
"""

from __future__ import annotations

import torch

from .kernel_A import lse_stats
from .kernel_B import kl_forward
from .kernel_C import kl_backward

__all__ = ["AttnKLAlignFn", "attn_kl_align"]


class AttnKLAlignFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qs, ks, qt, kt, attn_mask, causal: bool, sm_scale_s, sm_scale_t):
        """Stage A for both relations, then stage B (integration.py:8-45)."""
        lse_s = lse_stats(qs, ks, attn_mask=attn_mask, causal=causal, sm_scale=sm_scale_s)
        lse_t = lse_stats(qt, kt, attn_mask=attn_mask, causal=causal, sm_scale=sm_scale_t)
        kl = kl_forward(qs, ks, lse_s, qt, kt, lse_t, attn_mask=attn_mask, causal=causal,
                        sm_scale_s=sm_scale_s, sm_scale_t=sm_scale_t)
        if attn_mask is None:
            saved_mask = torch.empty(0, device=qs.device)
            has_mask = False
        else:
            saved_mask = attn_mask
            has_mask = True
        ctx.save_for_backward(qs, ks, lse_s, qt, kt, lse_t, saved_mask)
        ctx.has_mask = has_mask
        ctx.causal = causal
        ctx.sm_scale_s = sm_scale_s
        ctx.sm_scale_t = sm_scale_t
        return kl

    @staticmethod
    def backward(ctx, dloss):
        """Stage C, then the chain rule with dloss (integration.py:48-67)."""
        qs, ks, lse_s, qt, kt, lse_t, saved_mask = ctx.saved_tensors
        attn_mask = saved_mask if ctx.has_mask else None
        dqs, dks = kl_backward(qs, ks, lse_s, qt, kt, lse_t, attn_mask=attn_mask, causal=ctx.causal,
                               sm_scale_s=ctx.sm_scale_s, sm_scale_t=ctx.sm_scale_t)
        dqs = dqs * dloss
        dks = dks * dloss
        return dqs, dks, None, None, None, None, None, None


def attn_kl_align(qs, ks, qt, kt, attn_mask=None, causal=True, sm_scale_s=None, sm_scale_t=None):
    """Drop-in for integration.py:70-73."""
    return AttnKLAlignFn.apply(qs, ks, qt, kt, attn_mask, causal, sm_scale_s, sm_scale_t)
