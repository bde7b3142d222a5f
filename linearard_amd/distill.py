"""The loss side of the reference's distillation step (train.py:360-423).

Per micro-batch the reference computes, from the captured per-layer
projections of the student (qs, ks, vs) and the teacher (qt, kt, vt) and the
kept-position logits of both models:

    for each aligned layer:                                  # train.py:369-409
        Q += attn_kl_align(qs, qs, qt, qt) / denom           # causal self relations
        K += attn_kl_align(ks, ks, kt, kt) / denom
        V += attn_kl_align(vs, vs, vt, vt) / denom
    attn_loss = (Q + K + V) / max(1, L)                      # train.py:410
    logits_loss = mean KL(softmax(t_logits/T) || softmax(s_logits/T))   # :412-420
    loss = lam_A * attn_loss + lam_L * logits_loss           # :423

with ``denom = B * Hq * T`` without a mask and ``mask.sum().clamp_min(1) *
Hq`` with one (Hq = the layer's query heads, used for all three relations,
train.py:403-406).  ``distillation_loss`` computes the same quantities with
the batched relation launches (one launch per 8 relations of one kind, so
that Q, K and V stay separate for logging) and the logits-KL kernels, and
returns them all (train.py logs Q_loss, K_loss, V_loss, attn, logits and the
total, train.py:440-458).

When ``lam_L == 0`` (the scripts' default, scripts/train_linearard_*.sh)
the reference still evaluates the logits KL for its log and back-propagates
zeros through it; here the logits KL is evaluated without a graph in that
case, so the logged value is the same and no zero gradient pass runs.
"""

from __future__ import annotations

from typing import NamedTuple, Optional, Sequence

import torch

from .attention_KL import attn_kl_align_batched
from .attention_KL._checks import require
from .logits_kl import logits_kl

__all__ = ["DistillLoss", "distillation_loss"]


class DistillLoss(NamedTuple):
    loss: torch.Tensor          # lam_A * attn + lam_L * logits (train.py:423)
    attn_loss: torch.Tensor     # (Q + K + V) / max(1, L)  (train.py:410)
    logits_loss: torch.Tensor   # mean per-position KL (train.py:419), or None without logits
    Q_loss: torch.Tensor        # sum over layers of the Q/Q KL / denom (train.py:407)
    K_loss: torch.Tensor
    V_loss: torch.Tensor


def _denoms(xs: Sequence[torch.Tensor], attn_mask, dev):
    """denom of every layer (train.py:403-406), as float32 device scalars."""
    out = []
    for q in xs:
        B, Hq, T, _ = q.shape
        if attn_mask is None:  # a device fill, not a host tensor (no synchronising copy)
            out.append(torch.full((), float(B * Hq * T), device=dev, dtype=torch.float32))
        else:
            out.append(attn_mask.sum().clamp_min(1).to(torch.float32) * Hq)
    return out


def distillation_loss(qs: Sequence[torch.Tensor], ks: Sequence[torch.Tensor], vs: Sequence[torch.Tensor],
                      qt: Sequence[torch.Tensor], kt: Sequence[torch.Tensor], vt: Sequence[torch.Tensor],
                      t_logits: Optional[torch.Tensor] = None, s_logits: Optional[torch.Tensor] = None,
                      attn_mask: Optional[torch.Tensor] = None, lam_A: float = 1.0, lam_L: float = 0.0,
                      temperature: float = 1.0, sm_scale_s=None, sm_scale_t=None) -> DistillLoss:
    """The losses of train.py:360-423 for one micro-batch.

    ``qs``..``vt``: one [B, H, T, D] tensor per aligned layer (any views with
    a unit last stride, e.g. the attention hook's [B, T, H, D] projections
    permuted); gradients flow to the student tensors.  ``t_logits`` /
    ``s_logits``: [B, K, V] logits of the kept positions, or both None (no
    output alignment: ``logits_loss`` is None and ``loss = lam_A * attn``).
    ``attn_mask``: [B, T] or None.  ``lam_A``, ``lam_L``, ``temperature`` as
    train.py's --lam-a, --lam-l, --temperature (defaults 1.0, 0.0, 1.0).
    """
    L = len(qs)
    require(L > 0 and all(len(x) == L for x in (ks, vs, qt, kt, vt)), "one tensor per layer for each of Q, K, V")
    require((t_logits is None) == (s_logits is None), "t_logits and s_logits must be given together")
    dev = qs[0].device
    if attn_mask is not None and attn_mask.device != dev:
        attn_mask = attn_mask.to(dev)
    w = torch.stack(_denoms(qs, attn_mask, dev)).reciprocal()   # 1 / denom per layer

    def kind(xs_, xt_):
        return attn_kl_align_batched(list(xs_), list(xt_), w, attn_mask=attn_mask, causal=True,
                                     sm_scale_s=sm_scale_s, sm_scale_t=sm_scale_t)

    Q = kind(qs, qt)
    K = kind(ks, kt)
    V = kind(vs, vt)
    attn = (Q + K + V) / max(1, L)
    if t_logits is None:
        return DistillLoss(lam_A * attn, attn, None, Q, K, V)
    if lam_L == 0.0:
        with torch.no_grad():
            lg = logits_kl(t_logits, s_logits, temperature=temperature)
        return DistillLoss(lam_A * attn + 0.0 * lg, attn, lg, Q, K, V)
    lg = logits_kl(t_logits, s_logits, temperature=temperature)
    return DistillLoss(lam_A * attn + lam_L * lg, attn, lg, Q, K, V)
