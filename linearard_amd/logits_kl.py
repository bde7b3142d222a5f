"""Logits KL over the kept positions (the output-alignment term).

The reference's distillation step (train.py:412-420) computes, over the
[B, K, V] logits of the last K = ``--logits-keep-k`` positions of the
teacher and the student (``logits_to_keep``, train.py:343, :355):

    t_logp = F.log_softmax(t_logits / T, dim=-1)
    s_logp = F.log_softmax(s_logits / T, dim=-1)
    kl_per_tok = (t_logp.exp() * (t_logp - s_logp)).sum(dim=-1)
    logits_kl = kl_per_tok.mean()

``logits_kl(t_logits, s_logits, temperature)`` gives the same quantity from
two HBM-bound HIP kernels (``lard_logits_kl_forward``: one pass over both
logits tensors, no [B, K, V] intermediates; ``lard_logits_kl_backward``: one
pass writing the gradients).  The scaled logits are rounded to the logits
dtype as ``t_logits / T`` rounds them; the log-softmax, exponentials,
products and sums are float32, where the reference rounds each of its
intermediates to the logits dtype (the parity tests bound that difference).
The result is a float32 scalar (``reduction="mean"``) or the float32
per-position KL [B, K] (``reduction="none"``, ``kl_per_tok``).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

__all__ = ["LogitsKLFn", "logits_kl"]

_LOGITS_TYPES = (torch.float16, torch.bfloat16, torch.float32)


def _require(cond, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def _aligned(x: torch.Tensor) -> torch.Tensor:
    """x itself when its rows start on 16-byte boundaries, else a copy into a
    padded buffer (viewed back to x's shape)."""
    vec = 16 // x.element_size()
    if x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and all(
            x.stride(i) % vec == 0 or x.shape[i] <= 1 for i in range(x.ndim - 1)):
        return x
    return _padded_empty(x.shape, x.dtype, x.device).copy_(x)


def _padded_empty(shape, dtype, device) -> torch.Tensor:
    """Uninitialised tensor of `shape` whose rows are 16-byte aligned."""
    vec = 16 // torch.empty((), dtype=dtype).element_size()
    V = shape[-1]
    Vp = (V + vec - 1) // vec * vec
    buf = torch.empty((*shape[:-1], Vp), device=device, dtype=dtype)
    return buf[..., :V] if Vp != V else buf


def _as3(x: torch.Tensor) -> torch.Tensor:
    return x.unsqueeze(0) if x.ndim == 2 else x


class LogitsKLFn(torch.autograd.Function):
    """Forward: mean (or per-position) KL(p_t || p_s) of the tempered logits.
    Backward: gradients of both logits tensors (each only when required)."""

    @staticmethod
    def forward(ctx, t_logits, s_logits, temperature: float, reduction: str):
        _require(reduction in ("mean", "none"), "reduction must be 'mean' or 'none'")
        for name, x in (("t_logits", t_logits), ("s_logits", s_logits)):
            _require(isinstance(x, torch.Tensor) and x.is_cuda, f"{name} must be a CUDA tensor")
            _require(x.ndim in (2, 3), f"{name} must be [B, K, V] or [K, V]")
            _require(x.dtype in _LOGITS_TYPES, f"{name} dtype supports only fp16/bf16/fp32")
        _require(t_logits.shape == s_logits.shape, "t_logits and s_logits must have the same shape")
        _require(t_logits.dtype == s_logits.dtype, "t_logits and s_logits must have the same dtype")
        _require(t_logits.device == s_logits.device, "t_logits and s_logits must be on one device")
        T = float(temperature)
        t = _aligned(_as3(t_logits.detach()))
        s = _aligned(_as3(s_logits.detach()))
        B, K, V = t.shape
        rows = B * K
        dev = t.device
        lse_t = torch.empty((rows,), device=dev, dtype=torch.float32)
        lse_s = torch.empty((rows,), device=dev, dtype=torch.float32)
        kl_rows = torch.empty((rows,), device=dev, dtype=torch.float32)
        loss = torch.empty((), device=dev, dtype=torch.float32)
        L = _lib.lib()
        ws_bytes = L.lard_logits_kl_workspace_bytes(rows, V)
        ws = torch.empty((max(ws_bytes, 16),), device=dev, dtype=torch.uint8)
        dt, ds = _lib.logits_desc(t), _lib.logits_desc(s)
        rc = L.lard_logits_kl_forward(ctypes.byref(dt), ctypes.byref(ds), T, lse_t.data_ptr(), lse_s.data_ptr(),
                                      kl_rows.data_ptr(), loss.data_ptr(), ws.data_ptr(), ws_bytes,
                                      _lib.stream_of(t))
        _lib.check(rc, "lard_logits_kl_forward")
        ctx.save_for_backward(t, s, lse_t, lse_s, kl_rows)
        ctx.temperature = T
        ctx.reduction = reduction
        ctx.in_shape = t_logits.shape
        if reduction == "mean":
            return loss
        return kl_rows.view(t_logits.shape[:-1]).clone()  # not the saved tensor: callers may modify it

    @staticmethod
    def backward(ctx, g):
        t, s, lse_t, lse_s, kl_rows = ctx.saved_tensors
        need_t, need_s = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_t or need_s):
            return None, None, None, None
        B, K, V = t.shape
        rows = B * K
        g = g.detach().to(torch.float32).contiguous()
        if ctx.reduction == "mean":
            per_row, row_scale = 0, (1.0 / rows if rows > 0 else 0.0)
        else:
            per_row, row_scale = 1, 1.0
        gt = _padded_empty(t.shape, t.dtype, t.device) if need_t else None
        gs = _padded_empty(s.shape, s.dtype, s.device) if need_s else None
        dgt = _lib.logits_desc(gt) if gt is not None else None
        dgs = _lib.logits_desc(gs) if gs is not None else None
        L = _lib.lib()
        dt, ds = _lib.logits_desc(t), _lib.logits_desc(s)
        rc = L.lard_logits_kl_backward(
            ctypes.byref(dt), ctypes.byref(ds), ctx.temperature, lse_t.data_ptr(), lse_s.data_ptr(),
            kl_rows.data_ptr(), g.data_ptr(), per_row, row_scale,
            ctypes.byref(dgt) if dgt is not None else None, ctypes.byref(dgs) if dgs is not None else None,
            _lib.stream_of(t))
        _lib.check(rc, "lard_logits_kl_backward")
        shape = ctx.in_shape
        return (gt.reshape(shape) if gt is not None else None, gs.reshape(shape) if gs is not None else None,
                None, None)


def logits_kl(t_logits: torch.Tensor, s_logits: torch.Tensor, temperature: float = 1.0,
              reduction: str = "mean") -> torch.Tensor:
    """KL(softmax(t_logits / T) || softmax(s_logits / T)) per kept position,
    averaged (``"mean"``, the reference's ``logits_kl``, train.py:419) or
    not (``"none"``, ``kl_per_tok`` [B, K], train.py:417).

    t_logits, s_logits: [B, K, V] (or [K, V]) CUDA tensors of one dtype
    (bf16 as the reference's models produce them, fp16 or fp32).  The result
    is float32; gradients flow to whichever of the two requires them.
    """
    return LogitsKLFn.apply(t_logits, s_logits, temperature, reduction)
