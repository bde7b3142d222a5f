"""Seeded sweep of ragged shapes through the autograd boundary
(integration.py:6-73) against the float64 oracle (oracle.attn_kl).

The cases put T at and around the kernels' tile sizes (64-key tiles,
256-row workgroups: 63, 65, 255, 256, 257, 511), at T = 1, past four query
tiles per column block at every padded head dim (333-700), and mix:
- GQA ratios, for the self relation and for the general q != k relation;
- padding masks, including one kept token and none;
- causal and non-causal;
- fp16 and bf16;
- D = 8, 16, 32, 64, 128 (the throughput kernels, head dims padded to 16,
  32, 64, 128) and D = 256 (the fused path);
- unequal student and teacher scales.
"""

import math

import numpy as np
import pytest
import torch

from linearard_amd import _lib
from linearard_amd.attention_KL.integration import kernel_path
from oracle import attn_kl as O
from tests._inputs import make_mask, mask_to_dev, randn, to_dev
from tests._tolerance import check_grad, check_loss

pytestmark = pytest.mark.gpu

# (dtype, B, Hq, Hkv, T, D, mask ratio or None, causal, scale ratio t/s, self relation)
CASES = [
    ("bf16", 1, 2, 2, 1, 128, None, True, 1.0, True),
    ("bf16", 1, 2, 2, 63, 128, None, True, 1.0, True),
    ("bf16", 1, 2, 2, 65, 128, 0.3, True, 1.0, True),
    ("f16", 2, 2, 2, 255, 64, None, True, 1.0, True),
    ("bf16", 1, 3, 3, 256, 128, None, False, 1.0, True),
    ("bf16", 1, 2, 2, 257, 128, 0.5, True, 1.3, True),
    ("f16", 1, 2, 2, 511, 128, None, True, 0.7, True),
    ("bf16", 2, 4, 1, 200, 128, 0.2, True, 1.0, False),
    ("bf16", 1, 8, 2, 130, 64, None, False, 1.0, False),
    ("f16", 2, 4, 4, 97, 128, 0.4, True, 1.0, False),
    ("bf16", 1, 2, 2, 300, 256, None, True, 1.0, True),
    ("bf16", 2, 2, 2, 129, 128, 1.0, True, 1.0, True),  # only token 0 of each sequence kept
    ("bf16", 2, 2, 2, 70, 128, "none", True, 1.0, True),  # no token kept
    # five or more 64-row query tiles per column block, so the column
    # kernel's ring is refilled inside its loop, at every padded head dim
    # (16, 32, 64): odd and even tile counts, a partial last tile
    ("f16", 1, 2, 2, 400, 8, None, True, 1.0, True),
    ("bf16", 1, 2, 1, 400, 16, 0.3, False, 1.0, False),
    ("bf16", 1, 2, 2, 450, 32, None, True, 1.2, True),
    ("f16", 2, 2, 2, 333, 64, 0.4, True, 1.0, True),
    ("bf16", 1, 4, 2, 700, 64, None, False, 1.0, False),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-B{c[1]}-H{c[2]}/{c[3]}-T{c[4]}-D{c[5]}-m{c[6]}-c{int(c[7])}-r{c[8]}-{'self' if c[9] else 'qk'}" for c in CASES])
def test_autograd_sweep(gpu_available, case):
    from linearard_amd.attention_KL import attn_kl_align

    cid = "sweep-" + "-".join(str(c) for c in case)
    dtype, B, Hq, Hkv, T, D, ratio, causal, sr, self_rel = case
    rng = np.random.default_rng(1000 + 7 * T + Hq + D)
    a_s = 1 / math.sqrt(D)
    a_t = a_s * sr
    if T > 256 and D <= 128:
        # the throughput kernels, with the column kernel's in-loop refills
        x = torch.empty((B, Hq, T, D), device="cuda", dtype=torch.bfloat16 if dtype == "bf16" else torch.float16)
        d = [_lib.tensor4(x)] * 4
        assert kernel_path(d, a_s, a_t)[0] == "throughput", kernel_path(d, a_s, a_t)
    if ratio == "none":
        mask = np.zeros((B, T), dtype=np.int32)
    else:
        mask = None if ratio is None else make_mask(rng, B, T, ratio)
    if self_rel:
        xt = randn(rng, (B, Hq, T, D), dtype)
        xs = O.round_to(xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32), dtype)
        x_s = to_dev(xs, dtype, requires_grad=True)
        x_t = to_dev(xt, dtype)
        loss = attn_kl_align(x_s, x_s, x_t, x_t, attn_mask=mask_to_dev(mask), causal=causal, sm_scale_s=a_s,
                             sm_scale_t=a_t)
        loss.backward()
        rl, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, mask, causal, a_s, a_t, self_relation=True)
        check_loss(loss.item(), rl, cid)
        check_grad(x_s.grad.float().cpu().numpy(), rdx, cid)
    else:
        qt = randn(rng, (B, Hq, T, D), dtype)
        kt = randn(rng, (B, Hkv, T, D), dtype)
        qs = O.round_to(qt + 0.3 * rng.standard_normal(qt.shape).astype(np.float32), dtype)
        ks = O.round_to(kt + 0.3 * rng.standard_normal(kt.shape).astype(np.float32), dtype)
        tqs, tks = to_dev(qs, dtype, True), to_dev(ks, dtype, True)
        loss = attn_kl_align(tqs, tks, to_dev(qt, dtype), to_dev(kt, dtype), attn_mask=mask_to_dev(mask),
                             causal=causal, sm_scale_s=a_s, sm_scale_t=a_t)
        loss.backward()
        rl, rdq, rdk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, causal, a_s, a_t)
        check_loss(loss.item(), rl, cid)
        check_grad(tqs.grad.float().cpu().numpy(), rdq, cid, "dq")
        check_grad(tks.grad.float().cpu().numpy(), rdk, cid, "dk")
    # No valid token (kernel_A.py:157-158, kernel_C.py:252-256), one kept token
    # or T = 1: every valid row has a single key, so P_s = P_t = 1 there and the
    # reference's lse == S makes its KL and D exactly 0 (kernel_A.py:147-157,
    # kernel_B.py:206-213, kernel_C.py:224-233): zero loss, zero gradient.
    if ratio in ("none", 1.0) or T == 1:
        assert loss.item() == 0.0
        grads = [x_s.grad] if self_rel else [tqs.grad, tks.grad]
        assert not any(bool(g.any()) for g in grads)
