"""RoPE teacher/student pair producer (the step before the attention KL).

train.py captures q / k after each model's rotary embedding (train.py:133-142
via the record_qkv attention hook): the teacher's native RoPE and the
student's scaled one (``--student-rope-scaling``, train.py:206-213;
``{"rope_type": "linear", "factor": 8.0}`` for Llama-2, 4.0 for Llama-3 and
Mistral, scripts/train_linearard_*.sh:9).  ``rope_pair`` produces both from
one pre-RoPE tensor on the GPU with HF LLaMA's arithmetic (rotate_half
layout, cos / sin rounded to the tensor dtype, bf16 tensor ops), in one pass
over the input (``lard_rope_pair``).

The frequencies follow HF's ``_compute_default_rope_parameters`` (float32
``1 / base ** (arange(0, d, 2) / d)``) and, for ``linear`` scaling,
``inv_freq / factor``.
"""

from __future__ import annotations

import ctypes
import json

import torch

from . import _lib

__all__ = ["rope_inv_freq", "rope_pair"]

_FREQ_CACHE = {}  # (dim, base, scaling, device) -> device tensor: no host-to-device copy per call


def rope_inv_freq(dim: int, base: float, rope_scaling=None, device=None) -> torch.Tensor:
    """float32 [dim/2] inverse frequencies, computed like HF (on the CPU, then moved)."""
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.int64).to(dtype=torch.float) / dim))
    if rope_scaling is not None:
        kind = rope_scaling.get("rope_type", rope_scaling.get("type", "default"))
        if kind == "linear":
            inv = inv / float(rope_scaling["factor"])
        elif kind != "default":
            raise NotImplementedError(f"rope_type {kind!r}: only default and linear scaling are built")
    return inv.to(device) if device is not None else inv


def rope_pair(x: torch.Tensor, base: float, student_rope_scaling=None, position_ids=None):
    """(student, teacher) = (RoPE with the scaled frequencies, native RoPE) of x.

    x: pre-RoPE [B, H, T, D] bf16/fp16 on the GPU, any strides with a unit
    last stride (a permuted [B, T, H, D] tensor works without a copy), D a
    multiple of 16.  position_ids: optional int64 [B, T] (default 0..T-1).
    Returns two contiguous [B, H, T, D] tensors of x's dtype.
    """
    if not (isinstance(x, torch.Tensor) and x.is_cuda and x.ndim == 4):
        raise AssertionError("x must be a [B,H,T,D] CUDA tensor")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise AssertionError("x dtype supports only fp16/bf16")
    B, H, T, D = x.shape
    dev = x.device

    def freqs(scaling):
        key = (D, float(base), json.dumps(scaling, sort_keys=True), str(dev))
        if key not in _FREQ_CACHE:
            _FREQ_CACHE[key] = rope_inv_freq(D, base, scaling, dev)
        return _FREQ_CACHE[key]

    inv_t = freqs(None)
    inv_s = freqs(student_rope_scaling)
    out_t = torch.empty((B, H, T, D), device=dev, dtype=x.dtype)
    out_s = torch.empty((B, H, T, D), device=dev, dtype=x.dtype)
    pos_ptr, pos_sb = None, 0
    if position_ids is not None:
        if position_ids.dtype != torch.int64 or position_ids.shape != (B, T) or position_ids.stride(1) != 1:
            raise AssertionError("position_ids must be int64 [B,T] with a unit last stride")
        position_ids = position_ids.to(dev)
        pos_ptr, pos_sb = position_ids.data_ptr(), position_ids.stride(0)
    L = _lib.lib()
    d = _lib.tensor4(x)
    rc = L.lard_rope_pair(ctypes.byref(d), inv_t.data_ptr(), inv_s.data_ptr(), pos_ptr, pos_sb, out_t.data_ptr(),
                          out_s.data_ptr(), _lib.stream_of(x))
    _lib.check(rc, "lard_rope_pair")
    return out_s, out_t
