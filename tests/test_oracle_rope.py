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


_ROPE_TYPES = [
    (None, {}, None),
    ({"rope_type": "linear", "factor": 8.0}, {}, None),
    ({"type": "linear", "factor": 4.0}, {}, None),  # train.py:211-212 renames rope_type to type
    ({"rope_type": "dynamic", "factor": 4.0}, {"max_position_embeddings": 4096}, 32768),
    ({"rope_type": "dynamic", "factor": 2.0}, {"max_position_embeddings": 4096}, 1000),  # below max: unchanged
    ({"rope_type": "yarn", "factor": 8.0, "original_max_position_embeddings": 4096}, {}, None),
    ({"rope_type": "yarn", "factor": 4.0, "original_max_position_embeddings": 8192, "beta_fast": 16,
      "mscale": 0.7, "mscale_all_dim": 1.0}, {}, None),
    ({"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
      "original_max_position_embeddings": 8192}, {"max_position_embeddings": 131072}, None),
    ({"rope_type": "longrope", "long_factor": [1.0 + 0.05 * i for i in range(64)],
      "short_factor": [1.0 + 0.01 * i for i in range(64)], "original_max_position_embeddings": 4096},
     {"max_position_embeddings": 16384}, 32768),
    ({"rope_type": "longrope", "long_factor": [1.5] * 64, "short_factor": [1.1] * 64,
      "original_max_position_embeddings": 4096}, {"max_position_embeddings": 16384}, 2048),
]


@pytest.mark.parametrize("scaling,cfg,seq_len", _ROPE_TYPES,
                         ids=[f"{(s or {}).get('rope_type', (s or {}).get('type', 'default'))}-{i}"
                              for i, (s, _, _) in enumerate(_ROPE_TYPES)])
def test_rope_parameters_match_transformers(scaling, cfg, seq_len):
    """The product's frequency tables (linearard_amd.rope.rope_parameters) equal,
    bitwise, those of transformers' own rope initialisation functions -- what
    the student model of train.py:206-213 would compute for that rope type --
    and the attention scaling to float precision."""
    transformers = pytest.importorskip("transformers")
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    from linearard_amd.rope import rope_parameters

    base, dim = 500000.0, 128
    max_pos = cfg.get("max_position_embeddings", 4096)
    hf_scaling = None
    if scaling is not None:
        hf_scaling = dict(scaling)
        if "type" in hf_scaling:
            hf_scaling["rope_type"] = hf_scaling.pop("type")
    c = transformers.LlamaConfig(hidden_size=dim * 32, num_attention_heads=32, max_position_embeddings=max_pos,
                                 rope_theta=base, rope_scaling=hf_scaling)
    kind = (hf_scaling or {}).get("rope_type", "default")
    if kind == "default":
        ref_inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.int64).float() / dim))
        ref_att = 1.0
    else:
        kw = {"seq_len": seq_len} if seq_len is not None else {}
        ref_inv, ref_att = ROPE_INIT_FUNCTIONS[kind](c, "cpu", **kw)
    inv, att = rope_parameters(dim, base, scaling, max_position_embeddings=max_pos, seq_len=seq_len)
    assert inv.dtype == torch.float32 and inv.shape == (dim // 2,)
    assert torch.equal(inv, ref_inv.float()), (inv - ref_inv).abs().max()
    assert att == pytest.approx(float(ref_att), rel=1e-12)


def test_rope_parameters_rejects_unbuilt_types():
    from linearard_amd.rope import rope_parameters

    with pytest.raises(NotImplementedError):
        rope_parameters(128, 1e4, {"rope_type": "mrope", "factor": 2.0})
    with pytest.raises(NotImplementedError):
        rope_parameters(128, 1e4, {"rope_type": "linear", "factor": 2.0, "partial_rotary_factor": 0.5})
    with pytest.raises(ValueError):
        rope_parameters(128, 1e4, {"rope_type": "dynamic", "factor": 2.0})


def test_rope_oracle_attention_scaling_matches_torch():
    """cos / sin times the attention scaling (HF's float32 product, then the
    dtype cast), pinned against torch's arithmetic."""
    rng = np.random.default_rng(3)
    H, T, D = 2, 129, 64
    x = round_to(rng.standard_normal((H, T, D)).astype(np.float32), "bf16")
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))
    pos = torch.arange(T)
    att = 1.2079441541679836
    got = R.rope_apply(x, inv.numpy(), pos.numpy(), "bf16", attention_scaling=att)
    freqs = pos.float()[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = (emb.cos() * att).to(torch.bfloat16), (emb.sin() * att).to(torch.bfloat16)
    xt = torch.tensor(x).to(torch.bfloat16)
    ref = (xt * cos + torch.cat((-xt[..., D // 2:], xt[..., :D // 2]), dim=-1) * sin).float().numpy()
    diff = got != ref
    assert diff.mean() < 2e-3
    assert np.all(np.abs(got - ref)[diff] <= 2 * np.abs(ref)[diff] * 2.0 ** -7 + 1e-30)
    # a dropped scaling is caught
    plain = R.rope_apply(x, inv.numpy(), pos.numpy(), "bf16")
    assert (plain != ref).mean() > 0.5


def test_frequency_cache_keys_on_what_changes_the_table_and_stays_bounded():
    """rope_pair's table cache: a dynamic table is keyed on max(seq_len,
    max_position_embeddings) and a longrope one on seq_len > original length,
    so lengths that give the same table share one entry; the cache holds at
    most _FREQ_CACHE_SIZE entries, and every entry equals rope_parameters."""
    from linearard_amd import rope

    rope._FREQ_CACHE.clear()
    dyn = {"rope_type": "dynamic", "factor": 4.0}
    for n in (10, 100, 256):  # <= max_position_embeddings: one table
        inv, _ = rope._cached_parameters(64, 1e4, dyn, 256, n, "cpu")
    assert len(rope._FREQ_CACHE) == 1
    assert torch.equal(inv, rope.rope_parameters(64, 1e4, dyn, max_position_embeddings=256, seq_len=10)[0])
    inv_long, _ = rope._cached_parameters(64, 1e4, dyn, 256, 1000, "cpu")
    assert len(rope._FREQ_CACHE) == 2
    assert torch.equal(inv_long, rope.rope_parameters(64, 1e4, dyn, max_position_embeddings=256, seq_len=1000)[0])
    lr = {"rope_type": "longrope", "original_max_position_embeddings": 64, "factor": 4.0,
          "short_factor": [1.0] * 32, "long_factor": [2.0] * 32}
    for n in (3, 30, 64, 65, 500, 4000):
        got, att = rope._cached_parameters(64, 1e4, lr, 256, n, "cpu")
        want, att_w = rope.rope_parameters(64, 1e4, lr, max_position_embeddings=256, seq_len=n)
        assert torch.equal(got, want) and att == att_w
    assert len(rope._FREQ_CACHE) == 4  # short and long
    for n in range(300, 300 + 3 * rope._FREQ_CACHE_SIZE):  # distinct dynamic lengths
        rope._cached_parameters(64, 1e4, dyn, 256, n, "cpu")
    assert len(rope._FREQ_CACHE) == rope._FREQ_CACHE_SIZE
    other = {"rope_type": "linear", "factor": 8.0}
    a = rope._cached_parameters(128, 1e4, other, None, 5, "cpu")
    b = rope._cached_parameters(128, 1e4, other, None, 50000, "cpu")
    assert a is b  # the length does not enter the key of a fixed table
    rope._FREQ_CACHE.clear()
