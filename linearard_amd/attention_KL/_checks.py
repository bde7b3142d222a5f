"""Precondition checks shared by the stage wrappers.

They restate the reference wrappers' ``assert`` statements with the same
messages (kernel_A.py:192-220, kernel_B.py:262-322, kernel_C.py:307-368) but
raise ``AssertionError`` explicitly, so ``python -O`` cannot strip them.
"""

from __future__ import annotations

import math

import torch

SUPPORTED_HEAD_DIMS = (8, 16, 32, 64, 128, 256)  # kernel_A.py:18

# fp16 / bf16 as the reference (kernel_A.py:195-196), plus float32 (the
# library's float32 stage kernels; both sides must then be float32)
_INPUT_TYPES = (torch.float16, torch.bfloat16, torch.float32)
_MASK_TYPES = (torch.bool, torch.int32, torch.int64, torch.uint8)


def require(cond, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def check_mask(attn_mask, device, B, T):
    """kernel_B.py:311-322: a CPU mask is moved to the device first."""
    if attn_mask is None:
        return None
    require(isinstance(attn_mask, torch.Tensor), "attn_mask must be a torch.Tensor")
    if attn_mask.device.type == "cpu":
        require(attn_mask.is_contiguous(), "attn_mask must be contiguous")
        attn_mask = attn_mask.to(device=device)
    require(attn_mask.is_cuda, "attn_mask must be on CUDA")
    require(attn_mask.ndim == 2, "attn_mask shape must be [B,T]")
    require(attn_mask.shape[0] == B and attn_mask.shape[1] == T, "attn_mask shape must be [B,T]")
    require(attn_mask.dtype in _MASK_TYPES, "attn_mask dtype is invalid")
    require(attn_mask.is_contiguous(), "attn_mask must be contiguous")
    require(attn_mask.stride(-1) == 1, "attn_mask last-dim stride must be 1")
    return attn_mask


def check_scale(value, default_dim: int, name: str) -> float:
    """kernel_B.py:326-333: default 1/sqrt(D); must be a Python scalar."""
    if value is None:
        value = 1.0 / math.sqrt(default_dim)
    require(isinstance(value, float) or isinstance(value, int), f"{name} must be a scalar")
    return float(value)


def check_relations(qs, ks, qt, kt, strided_ok=False):
    """The q/k preconditions of kernel_B.py:262-309 (no lse involved).  With
    strided_ok (the batched caller API) any view with a unit last stride is
    accepted -- e.g. the [B,T,H,D] projections of train.py:133-142 seen as
    [B,H,T,D] -- and the library checks its alignment."""
    for t, n in ((qs, "qs"), (ks, "ks"), (qt, "qt"), (kt, "kt")):
        require(isinstance(t, torch.Tensor), f"{n} must be a torch.Tensor")
    require(qs.is_cuda and ks.is_cuda and qt.is_cuda and kt.is_cuda, "Q/K must be on CUDA")
    require(qs.dtype in _INPUT_TYPES, "qs dtype supports only fp16/bf16/fp32")
    require(ks.dtype in _INPUT_TYPES, "ks dtype supports only fp16/bf16/fp32")
    require(qt.dtype in _INPUT_TYPES, "qt dtype supports only fp16/bf16/fp32")
    require(kt.dtype in _INPUT_TYPES, "kt dtype supports only fp16/bf16/fp32")
    require((qs.dtype == torch.float32) == (qt.dtype == torch.float32),
            "float32 inputs need float32 on both sides")
    require(qs.dtype == ks.dtype, "qs/ks dtype must match")
    require(qt.dtype == kt.dtype, "qt/kt dtype must match")
    require(qs.ndim == 4 and ks.ndim == 4, "qs/ks shape must be [B,H,T,Ds]")
    require(qt.ndim == 4 and kt.ndim == 4, "qt/kt shape must be [B,H,T,Dt]")
    require(qs.shape[0] == ks.shape[0], "qs/ks B must match")
    require(qs.shape[2] == ks.shape[2], "qs/ks T must match")
    require(qs.shape[3] == ks.shape[3], "qs/ks Ds must match")
    require(qt.shape[0] == kt.shape[0], "qt/kt B must match")
    require(qt.shape[2] == kt.shape[2], "qt/kt T must match")
    require(qt.shape[3] == kt.shape[3], "qt/kt Dt must match")
    if not strided_ok:
        require(qs.is_contiguous() and ks.is_contiguous(), "qs/ks must be contiguous")
        require(qt.is_contiguous() and kt.is_contiguous(), "qt/kt must be contiguous")
    require(qs.stride(-1) == 1 and ks.stride(-1) == 1, "qs/ks last-dim stride must be 1")
    require(qt.stride(-1) == 1 and kt.stride(-1) == 1, "qt/kt last-dim stride must be 1")
    B, Hq, T, Ds = qs.shape
    B2, Hq2, T2, Dt = qt.shape
    Hkv_s = ks.shape[1]
    Hkv_t = kt.shape[1]
    require((B, Hq, T) == (B2, Hq2, T2), "student/teacher B/Hq/T must align")
    require(Hkv_s > 0 and Hq % Hkv_s == 0, "Hq must be divisible by Hkv_s")
    require(Hkv_t > 0 and Hq % Hkv_t == 0, "Hq must be divisible by Hkv_t")
    require(Ds in SUPPORTED_HEAD_DIMS, "Ds is not in the supported set")
    require(Dt in SUPPORTED_HEAD_DIMS, "Dt is not in the supported set")
    return B, Hq, T, Ds, Dt


def check_two_sided(qs, ks, lse_s, qt, kt, lse_t):
    """kernel_B.py:262-309 / kernel_C.py:307-354."""
    for t, n in ((qs, "qs"), (ks, "ks"), (qt, "qt"), (kt, "kt"), (lse_s, "lse_s"), (lse_t, "lse_t")):
        require(isinstance(t, torch.Tensor), f"{n} must be a torch.Tensor")
    require(qs.is_cuda and ks.is_cuda and qt.is_cuda and kt.is_cuda, "Q/K must be on CUDA")
    require(lse_s.is_cuda and lse_t.is_cuda, "lse must be on CUDA")
    require(lse_s.ndim == 3 and lse_t.ndim == 3, "lse shape must be [B,H,T]")
    require(lse_s.dtype == torch.float32 and lse_t.dtype == torch.float32, "lse must be float32")
    require(lse_s.is_contiguous() and lse_t.is_contiguous(), "lse must be contiguous")
    require(lse_s.stride(-1) == 1 and lse_t.stride(-1) == 1, "lse last-dim stride must be 1")
    dims = check_relations(qs, ks, qt, kt)
    B, Hq, T = dims[:3]
    require((B, Hq, T) == tuple(lse_s.shape), "lse_s shape must match [B,Hq,T]")
    require((B, Hq, T) == tuple(lse_t.shape), "lse_t shape must match [B,Hq,T]")
    return dims
