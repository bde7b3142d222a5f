"""Stage A: per-row log-sum-exp of one relation (mirrors kernel_A.py:190-265).

``lse_stats(q, k, attn_mask=None, causal=True, sm_scale=None)`` takes
q [B,Hq,T,D] and k [B,Hkv,T,D] (fp16/bf16 as the reference, or float32;
contiguous, on the GPU) and
returns lse [B,Hq,T] float32: log sum_j exp(sm_scale * q_i . k_j) over the
valid set (padding mask, causal), 0 for masked rows.  The work runs in
``lard_lse_stats`` of liblinearard_amd.so.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from ._checks import SUPPORTED_HEAD_DIMS, check_mask, check_scale, require

__all__ = ["SUPPORTED_HEAD_DIMS", "lse_stats"]


def lse_stats(q, k, attn_mask=None, causal=True, sm_scale=None):
    """Stage A wrapper; preconditions follow kernel_A.py:192-227."""
    require(isinstance(q, torch.Tensor), "q must be a torch.Tensor")
    require(isinstance(k, torch.Tensor), "k must be a torch.Tensor")
    require(q.is_cuda and k.is_cuda, "q/k must be on CUDA")
    require(q.dtype in (torch.float16, torch.bfloat16, torch.float32), "q dtype supports only fp16/bf16/fp32")
    require(k.dtype in (torch.float16, torch.bfloat16, torch.float32), "k dtype supports only fp16/bf16/fp32")
    require(q.dtype == k.dtype, "q/k dtype must match")
    require(q.ndim == 4 and k.ndim == 4, "q/k shape must be [B,H,T,D]")
    require(q.shape[0] == k.shape[0], "q/k B must match")
    require(q.shape[2] == k.shape[2], "q/k T must match")
    require(q.shape[3] == k.shape[3], "q/k D must match")
    require(q.is_contiguous() and k.is_contiguous(), "q/k must be contiguous")
    require(q.stride(-1) == 1 and k.stride(-1) == 1, "q/k last-dim stride must be 1")
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    require(D in SUPPORTED_HEAD_DIMS, "D is not in the supported set")
    require(Hkv > 0 and Hq % Hkv == 0, "Hq must be divisible by Hkv")
    attn_mask = check_mask(attn_mask, q.device, B, T)
    sm_scale = check_scale(sm_scale, D, "sm_scale")

    lse = torch.empty((B, Hq, T), device=q.device, dtype=torch.float32)
    qd, kd, md = _lib.tensor4(q), _lib.tensor4(k), _lib.mask_desc(attn_mask)
    rc = _lib.lib().lard_lse_stats(ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(md), int(bool(causal)),
                                   sm_scale, lse.data_ptr(), _lib.stream_of(q))
    _lib.check(rc, "lard_lse_stats")
    return lse
