"""Pins of the float32 eager-PyTorch restatement (oracle/attn_kl_torch.py,
bench.py's CPU baseline) against the pinned numpy oracle (oracle/attn_kl.py)."""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from oracle import attn_kl_torch as OT


@pytest.mark.parametrize("causal", [True, False])
def test_materialized_kl_and_its_autograd_match_the_oracle(causal):
    rng = np.random.default_rng(11)
    B, H, n, d = 1, 3, 70, 32
    xt = rng.standard_normal((B, H, n, d)).astype(np.float32)
    xs = (xt + 0.3 * rng.standard_normal(xt.shape)).astype(np.float32)
    a = 1 / math.sqrt(d)
    x = torch.tensor(xs, requires_grad=True)
    loss = OT.materialized_kl(x, torch.tensor(xt), causal, a, a)
    loss.backward()
    ref_loss, ref_dx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, None, causal, a, a, self_relation=True)
    assert abs(loss.item() - ref_loss) <= 1e-5 * abs(ref_loss)
    assert np.abs(x.grad.numpy() - ref_dx).max() <= 1e-5 * np.abs(ref_dx).max()


@pytest.mark.parametrize("causal,chunk", [(True, 16), (True, 1000), (False, 24)])
def test_chunked_restatement_matches_the_oracle(causal, chunk):
    rng = np.random.default_rng(12)
    n, d = 90, 64
    xt = rng.standard_normal((n, d)).astype(np.float32)
    xs = (xt + 0.2 * rng.standard_normal(xt.shape)).astype(np.float32)
    a_s, a_t = 1 / math.sqrt(d), 1.3 / math.sqrt(d)
    loss, dx = OT.self_relation_chunked(torch.tensor(xs), torch.tensor(xt), causal, a_s, a_t, chunk=chunk)
    ref_loss, ref_dx, _, _, _ = O.attn_kl_align(xs[None, None], xs[None, None], xt[None, None], xt[None, None], None,
                                                causal, a_s, a_t, self_relation=True)
    assert abs(loss - ref_loss) <= 1e-5 * abs(ref_loss)
    assert np.abs(dx.numpy() - ref_dx[0, 0]).max() <= 1e-5 * np.abs(ref_dx).max()
    # identical relations: exactly zero loss and gradient
    z, dz = OT.self_relation_chunked(torch.tensor(xt), torch.tensor(xt), causal, a_s, a_s, chunk=chunk)
    assert z == 0.0 and not bool(dz.any())
