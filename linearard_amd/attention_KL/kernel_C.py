"""Stage C: gradients of the summed KL w.r.t. the student q and k, given
both LSE vectors (mirrors kernel_C.py:293-449).

Returns (dq [B,Hq,T,Ds], dk [B,Hkv_s,T,Ds]) in float32 with
D = p_s - p_t cast to the student dtype (kernel_C.py:233),
dq = sm_scale_s * D @ K_s and dk = sm_scale_s * sum_{h in group} D^T @ Q_s.
dk has one owning workgroup per key tile inside the library
(``lard_kl_backward``), so it needs no atomics and no zero-initialisation.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ._checks import SUPPORTED_HEAD_DIMS, check_mask, check_scale, check_two_sided

__all__ = ["SUPPORTED_HEAD_DIMS", "kl_backward"]


def kl_backward(qs, ks, lse_s, qt, kt, lse_t, attn_mask=None, causal=True, sm_scale_s=None, sm_scale_t=None):
    """Stage C wrapper; preconditions follow kernel_C.py:307-380."""
    B, Hq, T, Ds, Dt = check_two_sided(qs, ks, lse_s, qt, kt, lse_t)
    attn_mask = check_mask(attn_mask, qs.device, B, T)
    sm_scale_s = check_scale(sm_scale_s, Ds, "sm_scale_s")
    sm_scale_t = check_scale(sm_scale_t, Dt, "sm_scale_t")

    dq = torch.empty((B, Hq, T, Ds), device=qs.device, dtype=torch.float32)
    dk = torch.empty((B, ks.shape[1], T, Ds), device=qs.device, dtype=torch.float32)
    d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
    md = _lib.mask_desc(attn_mask)
    rc = _lib.lib().lard_kl_backward(ctypes.byref(d[0]), ctypes.byref(d[1]), lse_s.data_ptr(), ctypes.byref(d[2]),
                                     ctypes.byref(d[3]), lse_t.data_ptr(), ctypes.byref(md), int(bool(causal)),
                                     sm_scale_s, sm_scale_t, dq.data_ptr(), dk.data_ptr(), _lib.stream_of(qs))
    _lib.check(rc, "lard_kl_backward")
    return dq, dk
