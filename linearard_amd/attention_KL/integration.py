"""Autograd boundary: ``AttnKLAlignFn`` / ``attn_kl_align`` (mirrors integration.py:6-73).

``attn_kl_align(qs, ks, qt, kt, attn_mask=None, causal=True,
sm_scale_s=None, sm_scale_t=None)`` returns the 0-d float32 SUM over rows of
KL(P_t || P_s), P_x = softmax of the (masked, causal) relation logits
sm_scale_x * q_x . k_x.  Gradients flow to qs and ks only; the teacher,
mask, causal flag and scales get None (integration.py:67).

Forward (``lard_attn_kl_forward``): one pass over the key tiles yields both
LSE vectors, the per-row KL and, when a gradient is needed, the row-side
gradient dq = sm_scale_s (P_s - P_t) K_s.  Backward
(``lard_attn_kl_backward``): one column-owner pass yields
dk = sm_scale_s sum_h D^T Q_s.  For the train.py call ``attn_kl_align(x, x,
y, y)`` (q is k), the backward adds the saved dq and returns the whole
gradient of ``x`` as the first output (and None for the second), so autograd
accumulates it once.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ._checks import check_mask, check_relations, check_scale

__all__ = ["AttnKLAlignFn", "attn_kl_align"]


class AttnKLAlignFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qs, ks, qt, kt, attn_mask, causal: bool, sm_scale_s, sm_scale_t):
        """integration.py:8-45 (stage A x2 + stage B), fused in the library."""
        B, Hq, T, Ds, Dt = check_relations(qs, ks, qt, kt)
        attn_mask = check_mask(attn_mask, qs.device, B, T)
        ss = check_scale(sm_scale_s, Ds, "sm_scale_s")
        st = check_scale(sm_scale_t, Dt, "sm_scale_t")
        want_grad = bool(ctx.needs_input_grad[0] or ctx.needs_input_grad[1])

        L = _lib.lib()
        dev = qs.device
        lse_s = torch.empty((B, Hq, T), device=dev, dtype=torch.float32)
        lse_t = torch.empty((B, Hq, T), device=dev, dtype=torch.float32)
        loss = torch.empty((), device=dev, dtype=torch.float32)
        dq_row = torch.empty((B, Hq, T, Ds), device=dev, dtype=torch.float32) if want_grad else None
        ws_bytes = L.lard_attn_kl_forward_workspace_bytes(B, Hq, T)
        ws = torch.empty((ws_bytes // 4 if ws_bytes >= 4 else 1,), device=dev, dtype=torch.float32)
        d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
        md = _lib.mask_desc(attn_mask)
        rc = L.lard_attn_kl_forward(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), ctypes.byref(d[3]),
                                    ctypes.byref(md), int(bool(causal)), ss, st, lse_s.data_ptr(), lse_t.data_ptr(),
                                    loss.data_ptr(), dq_row.data_ptr() if dq_row is not None else None,
                                    ws.data_ptr(), ws_bytes, _lib.stream_of(qs))
        _lib.check(rc, "lard_attn_kl_forward")

        saved_mask = attn_mask if attn_mask is not None else torch.empty(0, device=dev)
        saved_dq = dq_row if dq_row is not None else torch.empty(0, device=dev)
        ctx.save_for_backward(qs, ks, lse_s, qt, kt, lse_t, saved_mask, saved_dq)
        ctx.has_mask = attn_mask is not None
        ctx.causal = bool(causal)
        ctx.sm_scale_s = ss
        ctx.sm_scale_t = st
        ctx.self_relation = qs is ks
        return loss

    @staticmethod
    def backward(ctx, dloss):
        """integration.py:48-67: stage C and the chain rule with dloss."""
        qs, ks, lse_s, qt, kt, lse_t, saved_mask, dq_row = ctx.saved_tensors
        attn_mask = saved_mask if ctx.has_mask else None
        dloss = dloss.detach().to(torch.float32).contiguous()
        B, Hq, T, Ds = qs.shape
        dk = torch.empty((B, ks.shape[1], T, Ds), device=qs.device, dtype=torch.float32)
        d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
        md = _lib.mask_desc(attn_mask)
        rc = _lib.lib().lard_attn_kl_backward(
            ctypes.byref(d[0]), ctypes.byref(d[1]), lse_s.data_ptr(), ctypes.byref(d[2]), ctypes.byref(d[3]),
            lse_t.data_ptr(), ctypes.byref(md), int(ctx.causal), ctx.sm_scale_s, ctx.sm_scale_t,
            dq_row.data_ptr(), dloss.data_ptr(), int(ctx.self_relation), dk.data_ptr(), _lib.stream_of(qs))
        _lib.check(rc, "lard_attn_kl_backward")
        if ctx.self_relation:
            return dk, None, None, None, None, None, None, None
        dq = dq_row * dloss
        return dq, dk, None, None, None, None, None, None


def attn_kl_align(qs, ks, qt, kt, attn_mask=None, causal=True, sm_scale_s=None, sm_scale_t=None):
    """Drop-in for integration.py:70-73."""
    return AttnKLAlignFn.apply(qs, ks, qt, kt, attn_mask, causal, sm_scale_s, sm_scale_t)
