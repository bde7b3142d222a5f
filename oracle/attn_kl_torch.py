"""The reference math as float32 eager PyTorch on the CPU (bench.py's CPU baseline).

TEST / MEASUREMENT INFRASTRUCTURE ONLY: imported by ``tests/`` (which pin
these functions against oracle/attn_kl.py) and by ``bench.py``'s
``cpu_baseline`` leg, never by the product package.

* ``materialized_kl`` -- the reference's own fp32 check of the op, the
  materialised n x n formula of integration.py:102-127 (log_softmax of both
  scaled relations, causal -inf mask, ``sum p_t (log p_t - log p_s)`` over
  the rows), differentiated by torch autograd for dX_s (BASELINE cfg1).
* ``self_relation_chunked`` -- the same loss and the q-is-k gradient
  ``dX = a_s (D + D^T) X_s`` (D = P_s - P_t; kernel_C.py:224-253 with q = k,
  train.py:380-402) over blocks of query rows, so memory stays O(chunk * n):
  the linear-memory restatement used for cfg4 (n = 32768), where the
  materialised form would need ~20 GiB of temporaries per head.
"""

from __future__ import annotations

import math

import torch

__all__ = ["materialized_kl", "self_relation_chunked"]


def materialized_kl(xs: torch.Tensor, xt: torch.Tensor, causal: bool = True, sm_scale_s=None, sm_scale_t=None):
    """Sum over (b, h, i) of KL(P_t || P_s) for the self relations of [B, H, n, d]
    float32 tensors (integration.py:102-127).  Differentiable in xs."""
    d = xs.shape[-1]
    a_s = 1.0 / math.sqrt(d) if sm_scale_s is None else sm_scale_s
    a_t = 1.0 / math.sqrt(xt.shape[-1]) if sm_scale_t is None else sm_scale_t
    ss = (xs @ xs.transpose(-1, -2)) * a_s
    st = (xt @ xt.transpose(-1, -2)) * a_t
    if causal:
        n = xs.shape[-2]
        keep = torch.ones((n, n), dtype=torch.bool, device=xs.device).tril()
        ss = ss.masked_fill(~keep, float("-inf"))
        st = st.masked_fill(~keep, float("-inf"))
    lps = torch.log_softmax(ss, dim=-1)
    lpt = torch.log_softmax(st, dim=-1)
    pt = lpt.exp()
    term = torch.where(pt > 0, pt * (lpt - lps), torch.zeros_like(pt))
    return term.sum()


@torch.no_grad()
def self_relation_chunked(xs: torch.Tensor, xt: torch.Tensor, causal: bool = True, sm_scale_s=None,
                          sm_scale_t=None, chunk: int = 1024):
    """(loss, dX) of one [n, d] float32 self relation, O(chunk * n) memory."""
    n, d = xs.shape
    a_s = 1.0 / math.sqrt(d) if sm_scale_s is None else sm_scale_s
    a_t = 1.0 / math.sqrt(xt.shape[1]) if sm_scale_t is None else sm_scale_t
    dx = torch.zeros_like(xs)
    loss = 0.0
    cols = torch.arange(n)
    for i0 in range(0, n, chunk):
        i1 = min(n, i0 + chunk)
        jmax = i1 if causal else n
        ss = (xs[i0:i1] @ xs[:jmax].T) * a_s
        st = (xt[i0:i1] @ xt[:jmax].T) * a_t
        if causal:
            keep = cols[None, :jmax] <= torch.arange(i0, i1)[:, None]
            ss = ss.masked_fill(~keep, float("-inf"))
            st = st.masked_fill(~keep, float("-inf"))
        lps = torch.log_softmax(ss, dim=-1)
        lpt = torch.log_softmax(st, dim=-1)
        pt = lpt.exp()
        loss += float(torch.where(pt > 0, pt * (lpt - lps), torch.zeros_like(pt)).sum())
        dm = lps.exp() - pt
        dx[i0:i1] += a_s * (dm @ xs[:jmax])
        dx[:jmax] += a_s * (dm.T @ xs[i0:i1])
    return loss, dx
