"""Pins of the RoPE oracle (oracle/rope.py) against torch's own CPU
implementation of HF LLaMA's rotary embedding, and simple invariants."""

import numpy as np
import pytest
import torch

from oracle import rope as R
from oracle.attn_kl import round_to


def _hf_rope_torch(x, inv_freq, positions, dtype):
    """HF LlamaRotaryEmbedding + apply_rotary_pos_emb, written with torch ops
    (float32 angles and cos/sin, then dtype tensor arithmetic)."""
    freqs = positions.float()[:, None] * inv_freq.float()[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return (x * cos) + (rot * sin)


@pytest.mark.parametrize("dtype,tdtype", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_rope_oracle_matches_torch_hf_formula(dtype, tdtype):
    rng = np.random.default_rng(0)
    H, T, D = 3, 257, 64
    x = round_to(rng.standard_normal((H, T, D)).astype(np.float32) * 2, dtype)
    inv = (1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))) / 8.0
    pos = torch.arange(T) * 37  # large angles too
    got = R.rope_apply(x, inv.numpy(), pos.numpy(), dtype)
    ref = _hf_rope_torch(torch.tensor(x).to(tdtype), inv, pos, tdtype).float().numpy()
    diff = got != ref
    # float32 cos/sin of torch may differ from the float64-rounded ones by an
    # ulp: after the dtype rounding that shows as a one-ulp difference on a
    # handful of elements, never more
    assert diff.mean() < 2e-3
    ulp = np.abs(ref) * (2.0 ** -7 if dtype == "bf16" else 2.0 ** -10) + 1e-30
    assert np.all(np.abs(got - ref)[diff] <= 2 * ulp[diff])


def test_rope_oracle_invariants():
    rng = np.random.default_rng(1)
    x = round_to(rng.standard_normal((2, 16, 32)).astype(np.float32), "bf16")
    inv = np.float32(1.0) / (np.float32(10000.0) ** (np.arange(0, 32, 2, dtype=np.float32) / np.float32(32)))
    # position 0 is the identity
    out = R.rope_apply(x, inv, np.zeros(16, dtype=np.int64), "bf16")
    assert np.array_equal(out, x)
    # a rotation keeps each pair's norm (up to the dtype rounding)
    out = R.rope_apply(x, inv, np.arange(16), "f32")
    n0 = x[..., :16] ** 2 + x[..., 16:] ** 2
    n1 = out[..., :16] ** 2 + out[..., 16:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
    # a planted mistake (rotate_half with the wrong sign) is caught
    bad = x.copy()
    bad[..., :16], bad[..., 16:] = x[..., 16:], -x[..., :16]  # what cat(x2, -x1) would feed in
    assert not np.allclose(R.rope_apply(x, inv, np.arange(16), "f32")[..., :16],
                           x[..., :16] * np.cos(np.arange(16)[:, None] * inv) +
                           bad[..., :16] * np.sin(np.arange(16)[:, None] * inv), atol=1e-3)
