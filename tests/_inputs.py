"""Seeded CPU input generation shared by the GPU parity tests and the bench.

Inputs are drawn with numpy on the CPU (so every case is reproducible on
any host), rounded to the target 16-bit type, and only then copied to the
device: the oracle sees exactly the values the kernels see.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import attn_kl as O

TORCH_DTYPES = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def rounded(x, dtype):
    return O.round_to(np.asarray(x, np.float32), dtype)


def randn(rng, shape, dtype, scale=1.0):
    return rounded(rng.standard_normal(shape).astype(np.float32) * scale, dtype)


def make_mask(rng, B, T, ratio, kind="i32"):
    """``rand > ratio`` with column 0 forced valid, as test_kernel_A.py:238-239."""
    m = (rng.random((B, T)) > ratio)
    m[:, 0] = True
    return {"i32": m.astype(np.int32), "i64": m.astype(np.int64), "u8": m.astype(np.uint8), "bool": m}[kind]


def to_dev(x, dtype, requires_grad=False):
    t = torch.tensor(np.asarray(x, np.float32), dtype=TORCH_DTYPES[dtype], device="cuda")
    if requires_grad:
        t.requires_grad_(True)
    return t


def mask_to_dev(m):
    if m is None:
        return None
    return torch.from_numpy(np.ascontiguousarray(m)).cuda()
