"""GPU parity of the autograd boundary attn_kl_align (integration.py:6-73)."""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from tests._inputs import make_mask, mask_to_dev, randn, to_dev

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return abs(a - b) / max(abs(b), 1e-30)


@pytest.mark.parametrize("dtype,B,H,T,D,ratio,causal", [
    ("bf16", 1, 4, 300, 128, None, True),
    ("bf16", 2, 2, 129, 64, 0.2, True),
    ("f16", 1, 2, 77, 32, None, False),
    ("bf16", 1, 2, 1, 128, None, True),
])
def test_self_relation_fwd_bwd(gpu_available, dtype, B, H, T, D, ratio, causal):
    """train.py:380-402: attn_kl_align(x_s, x_s, x_t, x_t) with one shared gradient."""
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(100 + T)
    xt = randn(rng, (B, H, T, D), dtype)
    xs = O.round_to(xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32), dtype)
    mask = None if ratio is None else make_mask(rng, B, T, ratio)
    a = 1 / math.sqrt(D)
    x_s = to_dev(xs, dtype, requires_grad=True)
    x_t = to_dev(xt, dtype)
    loss = attn_kl_align(x_s, x_s, x_t, x_t, attn_mask=mask_to_dev(mask), causal=causal, sm_scale_s=a, sm_scale_t=a)
    assert loss.dim() == 0 and loss.dtype == torch.float32
    loss.backward()
    rl, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, mask, causal, a, a, self_relation=True)
    assert _rel(loss.item(), rl) <= 1e-3
    g = x_s.grad.float().cpu().numpy()
    assert x_s.grad.dtype == x_s.dtype
    denom = max(np.abs(rdx).max(), 1e-12)
    assert np.abs(g - rdx).max() / denom <= 2e-2


def test_general_gqa_masked_fwd_bwd_and_chain_rule(gpu_available):
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(9)
    B, Hq, Hks, Hkt, T, Ds, Dt = 2, 8, 4, 2, 70, 64, 32
    qs, ks = randn(rng, (B, Hq, T, Ds), "f16"), randn(rng, (B, Hks, T, Ds), "f16")
    qt, kt = randn(rng, (B, Hq, T, Dt), "f16"), randn(rng, (B, Hkt, T, Dt), "f16")
    mask = make_mask(rng, B, T, 0.3)
    tqs, tks = to_dev(qs, "f16", True), to_dev(ks, "f16", True)
    tqt, tkt = to_dev(qt, "f16"), to_dev(kt, "f16")
    loss = attn_kl_align(tqs, tks, tqt, tkt, attn_mask=mask_to_dev(mask), causal=True)
    (2.5 * loss).backward()
    rl, rdq, rdk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, True, dloss=2.5)
    assert _rel(loss.item(), rl) <= 1e-3
    for got, ref in ((tqs.grad, rdq), (tks.grad, rdk)):
        g = got.float().cpu().numpy()
        assert np.abs(g - ref).max() / np.abs(ref).max() <= 2e-2
    assert tqt.grad is None and tkt.grad is None


def test_identical_relations_give_exact_zero(gpu_available):
    """V/V with unrotated values: KL(P||P) == 0 exactly and the gradient vanishes."""
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(4)
    x = randn(rng, (1, 4, 513, 128), "bf16")
    x_s = to_dev(x, "bf16", True)
    x_t = to_dev(x, "bf16")
    loss = attn_kl_align(x_s, x_s, x_t, x_t)
    loss.backward()
    assert loss.item() == 0.0
    assert torch.count_nonzero(x_s.grad).item() == 0


def test_drop_in_import_path(gpu_available):
    from kernels.attention_KL.integration import attn_kl_align as via_reference_path
    from linearard_amd.attention_KL import attn_kl_align

    assert via_reference_path is attn_kl_align
