"""CPU oracle for the RoPE pair producer (numpy).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` as the checker, never by the
product package.

Restates HF LLaMA's rotary embedding as the reference's models apply it to
the captured q / k (train.py:206-213 for the student's scaling, record_qkv
at train.py:116-142 capturing the rotated tensors):

* angles ``pos * inv_freq[i]`` as one float32 product (HF's float32
  ``inv_freq @ position_ids``), ``emb = cat(freqs, freqs)``;
* ``cos``, ``sin`` of the angles times the rope type's attention scaling (a
  float32 product; HF's ``emb.cos() * attention_scaling``), cast to the
  tensor dtype;
* ``q * cos + rotate_half(q) * sin`` in the tensor dtype, rotate_half =
  ``cat(-x2, x1)``: every product and the sum rounded to the dtype (bf16
  tensor arithmetic rounds each operation's float32 result).

The cosines and sines are evaluated in float64 and rounded to float32 (so
to within half an ulp of float32); a device library's float32 cos / sin may
differ by an ulp, which after the dtype rounding changes a value only when
it sits on a rounding boundary.  Pinned against torch's own CPU
implementation of the same formula in tests/test_oracle_rope.py.
"""

from __future__ import annotations

import numpy as np

from .attn_kl import round_to

__all__ = ["rope_apply"]


def rope_apply(x, inv_freq, positions, dtype, attention_scaling=1.0):
    """x: [..., T, D] float32 values of the dtype; inv_freq: float32 [D/2];
    positions: [T] (or broadcastable [..., T]) integer positions;
    attention_scaling: the cos / sin multiplier.  Returns the rotated tensor
    as float32 values of the dtype."""
    x = np.asarray(x, dtype=np.float32)
    D = x.shape[-1]
    half = D // 2
    pos = np.asarray(positions).astype(np.float32)
    ang = (pos[..., :, None] * np.asarray(inv_freq, dtype=np.float32)[None, :]).astype(np.float32)
    att = np.float32(attention_scaling)
    c = round_to((np.cos(ang.astype(np.float64)).astype(np.float32) * att).astype(np.float32), dtype)
    s = round_to((np.sin(ang.astype(np.float64)).astype(np.float32) * att).astype(np.float32), dtype)
    x1, x2 = x[..., :half], x[..., half:]
    o1 = round_to(round_to(x1 * c, dtype) + round_to(-x2 * s, dtype), dtype)
    o2 = round_to(round_to(x2 * c, dtype) + round_to(x1 * s, dtype), dtype)
    return np.concatenate([o1, o2], axis=-1)
