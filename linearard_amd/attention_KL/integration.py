"""Autograd boundary: ``AttnKLAlignFn`` / ``attn_kl_align`` (mirrors integration.py:6-73).

``attn_kl_align(qs, ks, qt, kt, attn_mask=None, causal=True,
sm_scale_s=None, sm_scale_t=None)`` returns the 0-d float32 SUM over rows of
KL(P_t || P_s), P_x = softmax of the (masked, causal) relation logits
sm_scale_x * q_x . k_x.  Gradients flow to qs and ks only; the teacher,
mask, causal flag and scales get None (integration.py:67).

Forward (``lard_attn_kl_forward``): stage A for both relations and stage B in
one pass over the key tiles; only the two LSE vectors are saved (O(n), as in
integration.py:40).  Backward (``lard_attn_kl_backward``): stage C as a
row-owner pass (dq) and a column-owner pass (dk), both with D = P_s - P_t cast
to the input dtype before the product like kernel_C.py:233.  For the train.py
call ``attn_kl_align(x, x, y, y)`` (q is k) the library sums dq + dk in place
and the Function returns that whole gradient of ``x`` once (None for the
second input) instead of two float32 tensors for autograd to add.

When the student needs a gradient and the operands take the throughput
kernels, the forward is ``lard_attn_kl_forward_rowgrad`` instead: the same
pass also forms the row side of the gradient (dq before dloss, a float32
[B, Hq, T, Ds] buffer kept for the backward, O(n d) like the gradient
itself), and the backward runs only the column side
(``lard_attn_kl_backward_colgrad``), which adds itself to that buffer in
place.  A second backward through the same graph (retain_graph) finds the
buffer consumed and runs the full ``lard_attn_kl_backward``.
"""

from __future__ import annotations

import ctypes
import warnings

import torch

from .. import _lib
from ._checks import check_mask, check_relations, check_scale

__all__ = ["AttnKLAlignFn", "attn_kl_align"]


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty((nbytes if nbytes > 0 else 1,), device=device, dtype=torch.uint8)


PATH_NAMES = {0: "throughput", 1: "fused-forward", 2: "stage", 3: "float32"}
_WARNED = set()


def kernel_path(d, ss: float, st: float):
    """(path name, condition) of lard_attn_kl_path for the four operand descriptors."""
    L = _lib.lib()
    rc = L.lard_attn_kl_path(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), ctypes.byref(d[3]), ss, st)
    if rc < 0:  # a path code otherwise, not a status
        _lib.check(rc, "lard_attn_kl_path")
    return PATH_NAMES[rc], L.lard_last_error().decode()


def _warn_slow_path(d, ss: float, st: float) -> None:
    """One RuntimeWarning per condition that moves a call off the throughput
    kernels (the stage composition is about 4x slower at d=128)."""
    name, why = kernel_path(d, ss, st)
    if name != "throughput" and why not in _WARNED:
        _WARNED.add(why)
        warnings.warn(f"attn_kl_align: {why}: these inputs run the {name} kernels, not the throughput "
                      f"kernels (several times slower)", RuntimeWarning, stacklevel=3)


class AttnKLAlignFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qs, ks, qt, kt, attn_mask, causal: bool, sm_scale_s, sm_scale_t):
        """integration.py:8-45: stage A x2 + stage B."""
        B, Hq, T, Ds, Dt = check_relations(qs, ks, qt, kt)
        attn_mask = check_mask(attn_mask, qs.device, B, T)
        ss = check_scale(sm_scale_s, Ds, "sm_scale_s")
        st = check_scale(sm_scale_t, Dt, "sm_scale_t")

        L = _lib.lib()
        dev = qs.device
        lse_s = torch.empty((B, Hq, T), device=dev, dtype=torch.float32)
        lse_t = torch.empty((B, Hq, T), device=dev, dtype=torch.float32)
        loss = torch.empty((), device=dev, dtype=torch.float32)
        ws_bytes = L.lard_attn_kl_forward_workspace_bytes(B, Hq, T)
        ws = _workspace(ws_bytes, dev)
        d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
        path = "throughput"
        if B * Hq * T > 0:
            _warn_slow_path(d, ss, st)
            path = kernel_path(d, ss, st)[0]
        md = _lib.mask_desc(attn_mask)
        dq_row = None
        if path == "throughput" and B * Hq * T > 0 and (ctx.needs_input_grad[0] or ctx.needs_input_grad[1]):
            dq_row = torch.empty((B, Hq, T, Ds), device=dev, dtype=torch.float32)
            ws_bytes = L.lard_attn_kl_forward_rowgrad_workspace_bytes(B, Hq, ks.shape[1], kt.shape[1], T, Ds)
            ws = _workspace(ws_bytes, dev)
            rc = L.lard_attn_kl_forward_rowgrad(
                ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), ctypes.byref(d[3]), ctypes.byref(md),
                int(bool(causal)), ss, st, lse_s.data_ptr(), lse_t.data_ptr(), loss.data_ptr(), dq_row.data_ptr(),
                ws.data_ptr(), ws_bytes, _lib.stream_of(qs))
            _lib.check(rc, "lard_attn_kl_forward_rowgrad")
        else:
            rc = L.lard_attn_kl_forward(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]),
                                        ctypes.byref(d[3]), ctypes.byref(md), int(bool(causal)), ss, st,
                                        lse_s.data_ptr(), lse_t.data_ptr(), loss.data_ptr(), ws.data_ptr(), ws_bytes,
                                        _lib.stream_of(qs))
            _lib.check(rc, "lard_attn_kl_forward")

        saved_mask = attn_mask if attn_mask is not None else torch.empty(0, device=dev)
        ctx.has_row_grad = dq_row is not None
        ctx.row_grad_used = False
        ctx.save_for_backward(qs, ks, lse_s, qt, kt, lse_t, saved_mask,
                              dq_row if dq_row is not None else torch.empty(0, device=dev))
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
        self_rel = ctx.self_relation
        dev = qs.device
        L = _lib.lib()
        ws_bytes = L.lard_attn_kl_backward_workspace_bytes(B, Hq, ks.shape[1], T, Ds, int(self_rel))
        ws = _workspace(ws_bytes, dev)
        d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
        md = _lib.mask_desc(attn_mask)
        if ctx.has_row_grad and not ctx.row_grad_used:
            # the row side came with the forward: the column side adds itself
            # to it in place (self relation) or dq_row becomes dq
            ctx.row_grad_used = True
            dk = dq_row if self_rel else torch.empty((B, ks.shape[1], T, Ds), device=dev, dtype=torch.float32)
            rc = L.lard_attn_kl_backward_colgrad(
                ctypes.byref(d[0]), ctypes.byref(d[1]), lse_s.data_ptr(), ctypes.byref(d[2]), ctypes.byref(d[3]),
                lse_t.data_ptr(), ctypes.byref(md), int(ctx.causal), ctx.sm_scale_s, ctx.sm_scale_t,
                dloss.data_ptr(), int(self_rel), dq_row.data_ptr(), dk.data_ptr(), ws.data_ptr(), ws_bytes,
                _lib.stream_of(qs))
            _lib.check(rc, "lard_attn_kl_backward_colgrad")
            if self_rel:
                return dk, None, None, None, None, None, None, None
            return dq_row, dk, None, None, None, None, None, None
        dk = torch.empty((B, ks.shape[1], T, Ds), device=dev, dtype=torch.float32)
        dq = None if self_rel else torch.empty((B, Hq, T, Ds), device=dev, dtype=torch.float32)
        rc = L.lard_attn_kl_backward(
            ctypes.byref(d[0]), ctypes.byref(d[1]), lse_s.data_ptr(), ctypes.byref(d[2]), ctypes.byref(d[3]),
            lse_t.data_ptr(), ctypes.byref(md), int(ctx.causal), ctx.sm_scale_s, ctx.sm_scale_t, dloss.data_ptr(),
            int(self_rel), None if dq is None else dq.data_ptr(), dk.data_ptr(), ws.data_ptr(), ws_bytes,
            _lib.stream_of(qs))
        _lib.check(rc, "lard_attn_kl_backward")
        if self_rel:
            return dk, None, None, None, None, None, None, None
        return dq, dk, None, None, None, None, None, None


def attn_kl_align(qs, ks, qt, kt, attn_mask=None, causal=True, sm_scale_s=None, sm_scale_t=None):
    """Drop-in for integration.py:70-73."""
    return AttnKLAlignFn.apply(qs, ks, qt, kt, attn_mask, causal, sm_scale_s, sm_scale_t)
