"""Batched relation loss: the caller's loop over layers and Q/K/V relations.

The reference caller (train.py:369-410) computes, per aligned layer, three
self relations -- ``attn_kl_align(x_s, x_s, x_t, x_t)`` for x in Q, K, V --
divides each by ``denom`` (``B*Hq*T`` without a mask, ``mask.sum()*Hq``
with one, Hq the layer's query heads, train.py:403-406), sums them and
divides by the number of layers (train.py:410).  That is 3 L calls and
12 L kernel launches per micro-batch.

``attn_kl_align_batched(xs, xt, weights)`` computes
``sum_r weights[r] * attn_kl_align(xs[r], xs[r], xt[r], xt[r])`` with one
launch per 8 relations (``lard_attn_kl_batched_forward`` / ``_backward``):
the relations' row blocks share one grid even when their head counts differ
(Q/Q 32 heads next to K/K 8).  When the students need gradients the forward
is ``lard_attn_kl_batched_forward_rowgrad``, which also leaves the row side
of every gradient in the float32 buffers the backward returns, and the
backward (``lard_attn_kl_batched_backward_colgrad``) adds the column side in
place; a second backward through the same graph runs the full
``lard_attn_kl_batched_backward``.  ``relation_kl_loss`` builds the weights of
the train.py formula from the layers' tensors.  Batches outside the batched
kernels (different head dims, D = 256, extreme scales) go relation by
relation through the single-relation entry points inside the same autograd
Function, so the result is the same either way.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ._checks import check_mask, check_relations, check_scale, require

__all__ = ["AttnKLBatchedFn", "attn_kl_align_batched", "relation_kl_loss"]


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty((nbytes if nbytes > 0 else 1,), device=device, dtype=torch.uint8)


def _relations(xs, xt, lse_s, lse_t, dxs=None):
    arr = (_lib.Relation * len(xs))()
    for r in range(len(xs)):
        arr[r].xs = _lib.tensor4(xs[r])
        arr[r].xt = _lib.tensor4(xt[r])
        arr[r].lse_s = lse_s[r].data_ptr()
        arr[r].lse_t = lse_t[r].data_ptr()
        arr[r].dxs = None if dxs is None else dxs[r].data_ptr()
    return arr


class AttnKLBatchedFn(torch.autograd.Function):
    """Forward: sum_r w_r KL_r.  Backward: the gradient of every student
    tensor xs[r] (teachers, weights, mask, flags and scales get None)."""

    @staticmethod
    def forward(ctx, weights, attn_mask, causal: bool, sm_scale_s, sm_scale_t, n: int, *tensors):
        xs, xt = list(tensors[:n]), list(tensors[n:])
        dev = xs[0].device
        B, _, T, _ = xs[0].shape
        for r in range(n):
            check_relations(xs[r], xs[r], xt[r], xt[r], strided_ok=True)
            require(xs[r].shape[0] == B and xs[r].shape[2] == T, "batched relations must share B and T")
        attn_mask = check_mask(attn_mask, dev, B, T)
        ss = [check_scale(sm_scale_s, x.shape[3], "sm_scale_s") for x in xs]
        st = [check_scale(sm_scale_t, x.shape[3], "sm_scale_t") for x in xt]
        weights = weights.detach().to(device=dev, dtype=torch.float32).contiguous()
        require(weights.shape == (n,), "weights must hold one value per relation")

        L = _lib.lib()
        lse_s = [torch.empty(x.shape[:3], device=dev, dtype=torch.float32) for x in xs]
        lse_t = [torch.empty(x.shape[:3], device=dev, dtype=torch.float32) for x in xs]
        loss = torch.empty((), device=dev, dtype=torch.float32)
        md = _lib.mask_desc(attn_mask)
        stream = _lib.stream_of(xs[0])
        batched = len(set(ss)) == 1 and len(set(st)) == 1
        row_grad = None
        if batched:
            want_grad = any(ctx.needs_input_grad[6:6 + n])
            if want_grad:
                row_grad = [torch.empty(x.shape, device=dev, dtype=torch.float32) for x in xs]
            rels = _relations(xs, xt, lse_s, lse_t, row_grad)
            ws_bytes = (L.lard_attn_kl_batched_rowgrad_workspace_bytes(rels, n) if want_grad
                        else L.lard_attn_kl_batched_workspace_bytes(rels, n))
            ws = _workspace(ws_bytes, dev)
            fn = L.lard_attn_kl_batched_forward_rowgrad if want_grad else L.lard_attn_kl_batched_forward
            rc = fn(rels, n, ctypes.byref(md), int(bool(causal)), ss[0], st[0], weights.data_ptr(), loss.data_ptr(),
                    ws.data_ptr(), ws_bytes, stream)
            if rc == _lib.LARD_ERR_UNSUPPORTED:
                batched = False
                row_grad = None
            else:
                _lib.check(rc, "lard_attn_kl_batched_forward_rowgrad" if want_grad else "lard_attn_kl_batched_forward")
        if not batched:
            # relation by relation (same kernels as attn_kl_align), summed on the device
            losses = torch.empty((n,), device=dev, dtype=torch.float32)
            for r in range(n):
                B_, H_, T_, _ = xs[r].shape
                ws_bytes = L.lard_attn_kl_forward_workspace_bytes(B_, H_, T_)
                ws = _workspace(ws_bytes, dev)
                d = [_lib.tensor4(x) for x in (xs[r], xt[r])]
                rc = L.lard_attn_kl_forward(ctypes.byref(d[0]), ctypes.byref(d[0]), ctypes.byref(d[1]),
                                            ctypes.byref(d[1]), ctypes.byref(md), int(bool(causal)), ss[r], st[r],
                                            lse_s[r].data_ptr(), lse_t[r].data_ptr(), losses[r:r + 1].data_ptr(),
                                            ws.data_ptr(), ws_bytes, stream)
                _lib.check(rc, "lard_attn_kl_forward")
            loss = (losses * weights).sum()

        saved_mask = attn_mask if attn_mask is not None else torch.empty(0, device=dev)
        ctx.has_row_grad = row_grad is not None
        ctx.row_grad_used = False
        ctx.save_for_backward(weights, saved_mask, *xs, *xt, *lse_s, *lse_t, *(row_grad or []))
        ctx.n = n
        ctx.has_mask = attn_mask is not None
        ctx.causal = bool(causal)
        ctx.ss, ctx.st = ss, st
        ctx.batched = batched
        return loss

    @staticmethod
    def backward(ctx, dloss):
        n = ctx.n
        saved = ctx.saved_tensors
        weights, saved_mask = saved[0], saved[1]
        xs, xt = saved[2:2 + n], saved[2 + n:2 + 2 * n]
        lse_s, lse_t = saved[2 + 2 * n:2 + 3 * n], saved[2 + 3 * n:2 + 4 * n]
        attn_mask = saved_mask if ctx.has_mask else None
        dloss = dloss.detach().to(torch.float32).contiguous()
        dev = xs[0].device
        L = _lib.lib()
        md = _lib.mask_desc(attn_mask)
        stream = _lib.stream_of(xs[0])
        if ctx.has_row_grad and not ctx.row_grad_used:
            ctx.row_grad_used = True
            dxs = list(saved[2 + 4 * n:2 + 5 * n])
            rels = _relations(xs, xt, lse_s, lse_t, dxs)
            ws_bytes = L.lard_attn_kl_batched_workspace_bytes(rels, n)
            ws = _workspace(ws_bytes, dev)
            rc = L.lard_attn_kl_batched_backward_colgrad(rels, n, ctypes.byref(md), int(ctx.causal), ctx.ss[0],
                                                         ctx.st[0], weights.data_ptr(), dloss.data_ptr(),
                                                         ws.data_ptr(), ws_bytes, stream)
            _lib.check(rc, "lard_attn_kl_batched_backward_colgrad")
            return (None, None, None, None, None, None, *dxs, *([None] * n))
        dxs = [torch.empty(x.shape, device=dev, dtype=torch.float32) for x in xs]
        if ctx.batched:
            rels = _relations(xs, xt, lse_s, lse_t, dxs)
            ws_bytes = L.lard_attn_kl_batched_workspace_bytes(rels, n)
            ws = _workspace(ws_bytes, dev)
            rc = L.lard_attn_kl_batched_backward(rels, n, ctypes.byref(md), int(ctx.causal), ctx.ss[0], ctx.st[0],
                                                 weights.data_ptr(), dloss.data_ptr(), ws.data_ptr(), ws_bytes,
                                                 stream)
            _lib.check(rc, "lard_attn_kl_batched_backward")
        else:
            scaled = (dloss * weights).contiguous()  # dloss * w_r, one device scalar per relation
            for r in range(n):
                B_, H_, T_, D_ = xs[r].shape
                ws_bytes = L.lard_attn_kl_backward_workspace_bytes(B_, H_, H_, T_, D_, 1)
                ws = _workspace(ws_bytes, dev)
                d = [_lib.tensor4(x) for x in (xs[r], xt[r])]
                rc = L.lard_attn_kl_backward(
                    ctypes.byref(d[0]), ctypes.byref(d[0]), lse_s[r].data_ptr(), ctypes.byref(d[1]),
                    ctypes.byref(d[1]), lse_t[r].data_ptr(), ctypes.byref(md), int(ctx.causal), ctx.ss[r], ctx.st[r],
                    scaled[r:r + 1].data_ptr(), 1, None, dxs[r].data_ptr(), ws.data_ptr(), ws_bytes, stream)
                _lib.check(rc, "lard_attn_kl_backward")
        return (None, None, None, None, None, None, *dxs, *([None] * n))


def attn_kl_align_batched(xs, xt, weights=None, attn_mask=None, causal=True, sm_scale_s=None, sm_scale_t=None):
    """``sum_r weights[r] * attn_kl_align(xs[r], xs[r], xt[r], xt[r], ...)``.

    ``xs``, ``xt``: sequences of [B, H_r, T, D] student / teacher tensors
    (one self relation each, as train.py:380-402 calls it), any views with a
    unit last stride (the attention hook's [B, T, H, D] projections seen as
    [B, H, T, D] need no .contiguous() copy, unlike train.py:133-142);
    ``weights``: a float32 tensor (or sequence) of one value per relation,
    default all 1.  Returns a 0-d float32 tensor; gradients flow to the
    ``xs`` tensors.
    """
    xs, xt = list(xs), list(xt)
    require(len(xs) > 0 and len(xs) == len(xt), "xs and xt must hold the same number (>= 1) of relations")
    dev = xs[0].device
    if weights is None:
        weights = torch.ones((len(xs),), device=dev, dtype=torch.float32)
    elif not isinstance(weights, torch.Tensor):
        weights = torch.tensor([float(w) for w in weights], device=dev, dtype=torch.float32)
    return AttnKLBatchedFn.apply(weights, attn_mask, causal, sm_scale_s, sm_scale_t, len(xs), *xs, *xt)


def relation_kl_loss(qs, ks, vs, qt, kt, vt, attn_mask=None, sm_scale_s=None, sm_scale_t=None):
    """The attention-relation loss of train.py:360-410 in batched launches.

    ``qs``, ``ks``, ``vs`` (student) and ``qt``, ``kt``, ``vt`` (teacher) are
    sequences over the aligned layers of [B, H, T, D] tensors.  Per layer:
    Q/Q + K/K + V/V self relations (causal), each divided by ``denom`` =
    B * Hq * T (no mask) or mask.sum().clamp_min(1) * Hq, with Hq the layer's
    query-head count for all three (train.py:403-406); the layer sum is
    divided by max(1, L) (train.py:410).  No host synchronisation: the
    weights stay on the device.
    """
    L = len(qs)
    require(L > 0 and all(len(x) == L for x in (ks, vs, qt, kt, vt)), "one tensor per layer for each of Q, K, V")
    dev = qs[0].device
    if attn_mask is not None and attn_mask.device != dev:
        attn_mask = attn_mask.to(dev)
    xs, xt, w = [], [], []
    for layer in range(L):
        B, Hq, T, _ = qs[layer].shape
        if attn_mask is None:  # a fill on the device: a host tensor here would be a synchronising copy
            denom = torch.full((), float(B * Hq * T), device=dev, dtype=torch.float32)
        else:
            denom = attn_mask.sum().clamp_min(1).to(torch.float32) * Hq
        wl = 1.0 / (denom * max(1, L))
        for s_, t_ in ((qs[layer], qt[layer]), (ks[layer], kt[layer]), (vs[layer], vt[layer])):
            xs.append(s_)
            xt.append(t_)
            w.append(wl)
    weights = torch.stack(w).to(torch.float32)
    return attn_kl_align_batched(xs, xt, weights, attn_mask=attn_mask, causal=True, sm_scale_s=sm_scale_s,
                                 sm_scale_t=sm_scale_t)
