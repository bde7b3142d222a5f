"""CPU oracle for the logits KL over the kept positions (numpy, float64).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` (and ``bench.py``'s CPU
baseline) as the checker, never by the product package.

Restates the output-alignment lines of the reference's distillation step
(train.py:412-419) on [B, K, V] logits of the kept positions:

* scaled logits ``q = R(x * (1/T))``: ``t_logits / T`` with T a Python float
  is a tensor-by-host-scalar division; in the reference's runtime (torch
  2.9.0+cu128, requirement.txt:1) CUDA's true-division kernel turns a
  division by a host scalar into a product with the float32 reciprocal
  ``1.0f / float(T)`` (aten/src/ATen/native/cuda/BinaryDivTrueKernel.cu),
  and the float32 product is rounded to the tensor dtype (R);
* ``log_softmax`` of q, ``p_t = exp(l_t)``, ``kl = sum_v p_t (l_t - l_s)``
  per kept position (train.py:413-417) and its mean (train.py:419), here in
  float64 (the reference rounds each of these intermediates to the logits
  dtype; the tests bound that difference separately);
* the gradients autograd forms for ``loss.backward()`` (train.py:424):
  ``d/dx_s = c (p_s - p_t) / T`` and ``d/dx_t = c p_t (l_t - l_s - kl) / T``
  with ``c`` the upstream gradient of the row (``dloss / rows`` for the
  mean), in exact arithmetic (autograd's log_softmax backward multiplies
  ``p_s`` by ``sum_v p_t``, which is 1).

Pinned in tests/test_oracle_logits_kl.py against scipy's ``log_softmax`` /
``rel_entr``, closed forms (a two-word vocabulary, identical and
row-shifted logits), central finite differences of the loss for both
gradients, and the reference's own lines evaluated by torch on the CPU.
"""

from __future__ import annotations

import numpy as np

from .attn_kl import round_to

__all__ = ["scale_logits", "logits_kl", "logits_kl_grads"]


def scale_logits(x, temperature, dtype):
    """``x / T`` as the reference's tensor op rounds it (see the module
    docstring): float32 values of the dtype."""
    x = np.asarray(x, dtype=np.float32)
    inv = np.float32(1.0) / np.float32(temperature)
    if inv == np.float32(1.0):
        return x
    return round_to(x * inv, dtype)


def _log_softmax(q):
    if q.shape[-1] == 0:  # an empty vocabulary: log-sum-exp -inf, no terms
        return q, np.full(q.shape[:-1], -np.inf)
    m = np.max(q, axis=-1, keepdims=True)
    lse = m + np.log(np.sum(np.exp(q - m), axis=-1, keepdims=True))
    return q - lse, lse[..., 0]


def logits_kl(t_logits, s_logits, temperature=1.0, dtype="bf16"):
    """Return (loss, kl [B, K], lse_t [B, K], lse_s [B, K]) in float64.

    ``t_logits`` / ``s_logits``: float32 arrays holding values of ``dtype``
    (``"bf16"``, ``"f16"`` or ``"f32"``), shape [B, K, V] (or [K, V])."""
    qt = scale_logits(t_logits, temperature, dtype).astype(np.float64)
    qs = scale_logits(s_logits, temperature, dtype).astype(np.float64)
    lt, lse_t = _log_softmax(qt)
    ls, lse_s = _log_softmax(qs)
    kl = np.sum(np.exp(lt) * (lt - ls), axis=-1)
    loss = float(np.mean(kl)) if kl.size else float("nan")
    return loss, kl, lse_t, lse_s


def logits_kl_grads(t_logits, s_logits, temperature=1.0, dtype="bf16", dloss=1.0, reduction="mean"):
    """Return (grad_t, grad_s) in float64 for ``reduction`` "mean" (scalar
    ``dloss``) or "none" (``dloss`` of shape [B, K])."""
    qt = scale_logits(t_logits, temperature, dtype).astype(np.float64)
    qs = scale_logits(s_logits, temperature, dtype).astype(np.float64)
    lt, _ = _log_softmax(qt)
    ls, _ = _log_softmax(qs)
    pt, ps = np.exp(lt), np.exp(ls)
    kl = np.sum(pt * (lt - ls), axis=-1, keepdims=True)
    rows = int(np.prod(qt.shape[:-1]))
    inv = float(np.float32(1.0) / np.float32(temperature))
    if reduction == "mean":
        c = np.full(qt.shape[:-1] + (1,), float(dloss) / rows)
    else:
        c = np.asarray(dloss, dtype=np.float64).reshape(qt.shape[:-1] + (1,))
    c = c * inv
    return c * pt * ((lt - ls) - kl), c * (ps - pt)
