"""RoPE teacher/student pair producer (the step before the attention KL).

train.py captures q / k after each model's rotary embedding (train.py:133-142
via the record_qkv attention hook): the teacher's native RoPE and the
student's scaled one.  train.py:206-213 hands ``--student-rope-scaling`` to
the student's HF config unchanged (any HF rope type: ``linear`` with factor 8
for Llama-2 or 4 for Llama-3 and Mistral in scripts/train_linearard_*.sh:9,
and equally ``dynamic`` NTK, ``yarn``, ``longrope`` or ``llama3``).
``rope_pair`` produces both rotated tensors from one pre-RoPE tensor on the
GPU with HF LLaMA's arithmetic (rotate_half layout, cos / sin times the rope
type's attention scaling rounded to the tensor dtype, dtype tensor ops), in
one pass over the input (``lard_rope_pair``).  A student with a different
RoPE base (static NTK scaling, e.g. base x 8) takes ``student_base``.

``rope_parameters`` computes the inverse frequencies and the cos / sin
scaling of each rope type as HF's rope initialisation functions do (float32
torch arithmetic on the CPU, the same operations in the same order), so the
tables are bitwise HF's; the tests pin them against transformers' own
functions.
"""

from __future__ import annotations

import collections
import ctypes
import json
import math

import torch

from . import _lib

__all__ = ["rope_inv_freq", "rope_pair", "rope_parameters"]

# (dim, base, scaling, max_position_embeddings, length key, device) ->
# (device tensor, attention scaling); least recently used entries go first
_FREQ_CACHE = collections.OrderedDict()
_FREQ_CACHE_SIZE = 32


def _default_inv_freq(dim: int, base: float) -> torch.Tensor:
    return 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.int64).to(dtype=torch.float) / dim))


def rope_parameters(dim: int, base: float, rope_scaling=None, *, max_position_embeddings=None, seq_len=None):
    """(inv_freq float32 [dim/2] on the CPU, attention_scaling) of one rope type.

    rope_scaling: None or an HF rope-scaling dict (``rope_type`` or, as
    train.py:211-212 renames it, ``type``).  max_position_embeddings: the
    model's (needed by ``dynamic`` and by ``yarn`` / ``longrope`` without a
    ``factor``).  seq_len: the longest position + 1 of the call (``dynamic``
    and ``longrope`` choose their tables by it, as HF's forward-time update
    does for a fresh rotary module).
    """
    scaling = dict(rope_scaling or {})
    kind = scaling.get("rope_type", scaling.get("type", "default"))
    if float(scaling.get("partial_rotary_factor", 1.0)) != 1.0:
        raise NotImplementedError("partial_rotary_factor != 1 is not built")
    max_pos = scaling.get("max_position_embeddings", max_position_embeddings)
    if kind == "default":
        return _default_inv_freq(dim, base), 1.0
    if kind == "linear":
        return _default_inv_freq(dim, base) / float(scaling["factor"]), 1.0
    if kind == "dynamic":
        if max_pos is None:
            raise ValueError("dynamic rope scaling needs max_position_embeddings")
        factor = scaling["factor"]
        L = max_pos if seq_len is None else max(int(seq_len), max_pos)
        nb = base * ((factor * L / max_pos) - (factor - 1)) ** (dim / (dim - 2))
        return _default_inv_freq(dim, nb), 1.0
    if kind == "llama3":
        inv = _default_inv_freq(dim, base)
        factor = scaling["factor"]
        lo, hi = scaling["low_freq_factor"], scaling["high_freq_factor"]
        old = scaling["original_max_position_embeddings"]
        lo_wl, hi_wl = old / lo, old / hi
        wl = 2 * math.pi / inv
        out = torch.where(wl > lo_wl, inv / factor, inv)
        smooth = (old / wl - lo) / (hi - lo)
        smoothed = (1 - smooth) * out / factor + smooth * out
        medium = ~(wl < hi_wl) * ~(wl > lo_wl)
        return torch.where(medium, smoothed, out), 1.0
    if kind == "yarn":
        orig = scaling["original_max_position_embeddings"]
        factor = scaling.get("factor")
        if factor is None:
            factor = max_pos / orig
        att = scaling.get("attention_factor")
        mscale, mscale_all = scaling.get("mscale"), scaling.get("mscale_all_dim")

        def get_mscale(s, m=1):
            return 1.0 if s <= 1 else 0.1 * m * math.log(s) + 1.0

        if att is None:
            att = float(get_mscale(factor, mscale) / get_mscale(factor, mscale_all)) if mscale and mscale_all \
                else get_mscale(factor)
        beta_fast = scaling.get("beta_fast") or 32
        beta_slow = scaling.get("beta_slow") or 1

        def corr_dim(rot):
            return (dim * math.log(orig / (rot * 2 * math.pi))) / (2 * math.log(base))

        low, high = corr_dim(beta_fast), corr_dim(beta_slow)
        if scaling.get("truncate", True):
            low, high = math.floor(low), math.ceil(high)
        low, high = max(low, 0), min(high, dim - 1)
        if low == high:
            high += 0.001
        ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - low) / (high - low), 0, 1)
        pos_freqs = base ** (torch.arange(0, dim, 2).to(dtype=torch.float) / dim)
        extra = 1 - ramp
        inv = (1.0 / (factor * pos_freqs)) * (1 - extra) + (1.0 / pos_freqs) * extra
        return inv, float(att)
    if kind == "longrope":
        orig = scaling["original_max_position_embeddings"]
        factor = scaling.get("factor")
        if factor is None:
            factor = max_pos / orig
        att = scaling.get("attention_factor")
        if att is None:
            att = 1.0 if factor <= 1.0 else math.sqrt(1 + math.log(factor) / math.log(orig))
        ext = scaling["long_factor"] if seq_len and seq_len > orig else scaling["short_factor"]
        ext = torch.tensor(ext, dtype=torch.float32)
        shape = torch.arange(0, dim, 2, dtype=torch.int64).float() / dim
        return 1.0 / (ext * base ** shape), float(att)
    raise NotImplementedError(f"rope_type {kind!r} is not built")


def _length_key(rope_scaling, seq_len, max_position_embeddings):
    """The part of a call's length that changes a rope type's table: dynamic
    uses max(seq_len, max_position_embeddings), longrope only whether seq_len
    exceeds original_max_position_embeddings, the other types nothing."""
    scaling = dict(rope_scaling or {})
    kind = scaling.get("rope_type", scaling.get("type", "default"))
    if seq_len is None or kind not in ("dynamic", "longrope"):
        return None
    if kind == "dynamic":
        max_pos = scaling.get("max_position_embeddings", max_position_embeddings)
        return int(seq_len) if max_pos is None else max(int(seq_len), int(max_pos))
    orig = scaling.get("original_max_position_embeddings")
    return int(seq_len) if orig is None else bool(seq_len > orig)


def _cached_parameters(dim, base, rope_scaling, max_position_embeddings, seq_len, device):
    """rope_parameters with the table moved to `device`, from a bounded LRU cache."""
    key = (dim, float(base), json.dumps(rope_scaling, sort_keys=True), max_position_embeddings,
           _length_key(rope_scaling, seq_len, max_position_embeddings), str(device))
    hit = _FREQ_CACHE.get(key)
    if hit is not None:
        _FREQ_CACHE.move_to_end(key)
        return hit
    inv, att = rope_parameters(dim, base, rope_scaling, max_position_embeddings=max_position_embeddings,
                               seq_len=seq_len)
    _FREQ_CACHE[key] = hit = (inv.to(device), float(att))
    while len(_FREQ_CACHE) > _FREQ_CACHE_SIZE:
        _FREQ_CACHE.popitem(last=False)
    return hit


def rope_inv_freq(dim: int, base: float, rope_scaling=None, device=None, **kw) -> torch.Tensor:
    """float32 [dim/2] inverse frequencies, computed like HF (on the CPU, then moved)."""
    inv, _ = rope_parameters(dim, base, rope_scaling, **kw)
    return inv.to(device) if device is not None else inv


def rope_pair(x: torch.Tensor, base: float, student_rope_scaling=None, position_ids=None, *, student_base=None,
              max_position_embeddings=None):
    """(student, teacher) = (RoPE with the student's frequencies, native RoPE) of x.

    x: pre-RoPE [B, H, T, D] bf16/fp16 on the GPU, any strides with a unit
    last stride (a permuted [B, T, H, D] tensor works without a copy), D a
    multiple of 16.  base: the teacher's RoPE base (rope_theta); the student
    uses ``student_base`` (default: the same) with ``student_rope_scaling``
    on top.  position_ids: optional int64 [B, T] (default 0..T-1).
    Returns two contiguous [B, H, T, D] tensors of x's dtype.
    """
    if not (isinstance(x, torch.Tensor) and x.is_cuda and x.ndim == 4):
        raise AssertionError("x must be a [B,H,T,D] CUDA tensor")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise AssertionError("x dtype supports only fp16/bf16")
    B, H, T, D = x.shape
    dev = x.device
    if position_ids is not None:
        if position_ids.dtype != torch.int64 or position_ids.shape != (B, T) or position_ids.stride(1) != 1:
            raise AssertionError("position_ids must be int64 [B,T] with a unit last stride")
    sbase = base if student_base is None else student_base
    kind = (student_rope_scaling or {}).get("rope_type", (student_rope_scaling or {}).get("type", "default"))
    seq_len = None
    if kind in ("dynamic", "longrope"):  # their tables depend on the call's longest position
        seq_len = T if position_ids is None else int(position_ids.max().item()) + 1

    inv_t, att_t = _cached_parameters(D, base, None, max_position_embeddings, seq_len, dev)
    inv_s, att_s = _cached_parameters(D, sbase, student_rope_scaling, max_position_embeddings, seq_len, dev)
    out_t = torch.empty((B, H, T, D), device=dev, dtype=x.dtype)
    out_s = torch.empty((B, H, T, D), device=dev, dtype=x.dtype)
    pos_ptr, pos_sb = None, 0
    if position_ids is not None:
        position_ids = position_ids.to(dev)
        pos_ptr, pos_sb = position_ids.data_ptr(), position_ids.stride(0)
    L = _lib.lib()
    d = _lib.tensor4(x)
    rc = L.lard_rope_pair(ctypes.byref(d), inv_t.data_ptr(), inv_s.data_ptr(), att_t, att_s, pos_ptr, pos_sb,
                          out_t.data_ptr(), out_s.data_ptr(), _lib.stream_of(x))
    _lib.check(rc, "lard_rope_pair")
    return out_s, out_t
