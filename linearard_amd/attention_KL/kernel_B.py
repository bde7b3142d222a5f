"""Stage B: KL(P_t || P_s) summed over rows, given both LSE vectors
(mirrors kernel_B.py:249-391).

Returns a 0-d float32 tensor holding sum_rows sum_j p_t (log p_t - log p_s).
The per-row terms are reduced in a fixed order inside the library
(``lard_kl_forward``), so repeated calls are bitwise identical.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ._checks import SUPPORTED_HEAD_DIMS, check_mask, check_scale, check_two_sided

__all__ = ["SUPPORTED_HEAD_DIMS", "kl_forward"]


def kl_forward(qs, ks, lse_s, qt, kt, lse_t, attn_mask=None, causal=True, sm_scale_s=None, sm_scale_t=None):
    """Stage B wrapper; preconditions follow kernel_B.py:262-333."""
    B, Hq, T, Ds, Dt = check_two_sided(qs, ks, lse_s, qt, kt, lse_t)
    attn_mask = check_mask(attn_mask, qs.device, B, T)
    sm_scale_s = check_scale(sm_scale_s, Ds, "sm_scale_s")
    sm_scale_t = check_scale(sm_scale_t, Dt, "sm_scale_t")

    L = _lib.lib()
    loss_sum = torch.empty((), device=qs.device, dtype=torch.float32)
    ws_bytes = L.lard_kl_forward_workspace_bytes(B, Hq, T)
    ws = torch.empty((ws_bytes // 4 if ws_bytes >= 4 else 1,), device=qs.device, dtype=torch.float32)
    d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
    md = _lib.mask_desc(attn_mask)
    rc = L.lard_kl_forward(ctypes.byref(d[0]), ctypes.byref(d[1]), lse_s.data_ptr(), ctypes.byref(d[2]),
                           ctypes.byref(d[3]), lse_t.data_ptr(), ctypes.byref(md), int(bool(causal)), sm_scale_s,
                           sm_scale_t, loss_sum.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_of(qs))
    _lib.check(rc, "lard_kl_forward")
    return loss_sum
