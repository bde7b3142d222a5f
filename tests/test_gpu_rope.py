"""GPU parity of the RoPE pair producer (lard_rope_pair) with the oracle."""

import numpy as np
import pytest
import torch

from oracle import rope as R
from oracle.attn_kl import round_to

pytestmark = pytest.mark.gpu

TD = {"bf16": torch.bfloat16, "f16": torch.float16}


def _check(got, ref, x, dtype):
    """Equal, except where a float32 cos / sin of the device library and the
    oracle's correctly rounded one straddle a dtype rounding boundary: then c
    or s differs by one dtype ulp (<= eps for values <= 1), which moves the
    output by at most eps (|x_i| + |x_{i+D/2}|) plus its own rounding."""
    got = got.float().cpu().numpy()
    diff = got != ref
    assert diff.mean() <= 1e-3, diff.mean()
    eps = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    half = x.shape[-1] // 2
    pair = np.abs(x) + np.abs(np.concatenate([x[..., half:], x[..., :half]], axis=-1))
    bound = eps * pair + 2 * eps * np.abs(ref) + 1e-30
    assert np.all(np.abs(got - ref)[diff] <= bound[diff])


@pytest.mark.parametrize("dtype,B,H,T,D,factor,with_pos", [
    ("bf16", 2, 4, 300, 128, 8.0, False),
    ("f16", 1, 3, 77, 64, 4.0, True),
    ("bf16", 1, 2, 4096, 128, 8.0, False),  # large angles
    # cfg4's rotations: positions up to 32767 (angles up to 32767 rad for the
    # teacher), linear x8 student, base 1e4; in order and permuted
    ("bf16", 1, 4, 32768, 128, 8.0, False),
    ("bf16", 1, 2, 32768, 128, 8.0, True),
])
def test_rope_pair_matches_oracle(gpu_available, dtype, B, H, T, D, factor, with_pos):
    from linearard_amd.rope import rope_inv_freq, rope_pair

    rng = np.random.default_rng(T)
    x = round_to(rng.standard_normal((B, H, T, D)).astype(np.float32), dtype)
    pos = None
    pos_np = np.broadcast_to(np.arange(T), (B, T))
    if with_pos:
        pos_np = np.stack([rng.permutation(T) + 5 * b for b in range(B)])
        pos = torch.tensor(pos_np, dtype=torch.int64, device="cuda")
    xd = torch.tensor(x, device="cuda").to(TD[dtype])
    xs, xt = rope_pair(xd, 10000.0, {"rope_type": "linear", "factor": factor}, position_ids=pos)
    assert xs.shape == xt.shape == (B, H, T, D) and xs.is_contiguous() and xs.dtype == TD[dtype]
    inv_t = rope_inv_freq(D, 10000.0).numpy()
    inv_s = rope_inv_freq(D, 10000.0, {"rope_type": "linear", "factor": factor}).numpy()
    for b in range(B):
        _check(xt[b], R.rope_apply(x[b], inv_t, pos_np[b], dtype), x[b], dtype)
        _check(xs[b], R.rope_apply(x[b], inv_s, pos_np[b], dtype), x[b], dtype)


def test_rope_pair_takes_a_permuted_view_without_a_copy(gpu_available):
    """The captured q of an HF attention is a [B, T, H, D] tensor seen as
    [B, H, T, D]; the producer reads it through its strides."""
    from linearard_amd.rope import rope_pair

    g = torch.Generator(device="cuda").manual_seed(0)
    bthd = torch.randn((2, 100, 4, 128), device="cuda", generator=g).to(torch.bfloat16)
    view = bthd.permute(0, 2, 1, 3)
    assert not view.is_contiguous()
    a_s, a_t = rope_pair(view, 5e5, {"rope_type": "linear", "factor": 4.0})
    b_s, b_t = rope_pair(view.contiguous(), 5e5, {"rope_type": "linear", "factor": 4.0})
    assert torch.equal(a_s, b_s) and torch.equal(a_t, b_t)


def test_rope_pair_rejects_unsupported_head_dims(gpu_available):
    from linearard_amd.rope import rope_pair

    x = torch.zeros((1, 1, 8, 8), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        rope_pair(x, 1e4)


@pytest.mark.parametrize("dtype,scaling,student_base,max_pos", [
    ("bf16", None, 5e5 * 8, None),  # cfg3: teacher base 5e5, NTK student base x 8
    ("bf16", {"rope_type": "yarn", "factor": 8.0, "original_max_position_embeddings": 1024}, None, None),
    ("f16", {"rope_type": "dynamic", "factor": 4.0}, None, 256),
    ("bf16", {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
              "original_max_position_embeddings": 256}, None, None),
])
def test_rope_pair_other_rope_types_match_oracle(gpu_available, dtype, scaling, student_base, max_pos):
    """Every HF rope type the student of train.py:206-213 may use: the
    producer's student equals the oracle's rotation with rope_parameters'
    frequencies and attention scaling; the teacher keeps the native base."""
    from linearard_amd.rope import rope_pair, rope_parameters

    B, H, T, D = 1, 3, 700, 128
    base = 5e5
    rng = np.random.default_rng(17)
    x = round_to(rng.standard_normal((B, H, T, D)).astype(np.float32), dtype)
    xd = torch.tensor(x, device="cuda").to(TD[dtype])
    xs, xt = rope_pair(xd, base, scaling, student_base=student_base, max_position_embeddings=max_pos)
    inv_t, att_t = rope_parameters(D, base)
    inv_s, att_s = rope_parameters(D, student_base or base, scaling, max_position_embeddings=max_pos, seq_len=T)
    pos = np.arange(T)
    _check(xt[0], R.rope_apply(x[0], inv_t.numpy(), pos, dtype, att_t), x[0], dtype)
    ref_s = R.rope_apply(x[0], inv_s.numpy(), pos, dtype, att_s)
    _check(xs[0], ref_s, x[0], dtype)
    if student_base is not None or att_s != 1.0:  # the student really differs from the teacher
        assert not torch.equal(xs, xt)
