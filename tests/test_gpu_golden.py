"""The library against the committed golden fixtures (tests/golden/), through
every entry point: stage A/B/C and the autograd boundary."""

import math

import numpy as np
import pytest
import torch

from tests._inputs import mask_to_dev, to_dev
from tests._tolerance import check_grad, check_loss
from tests.golden import golden

pytestmark = pytest.mark.gpu

CASES = golden.load()


def _dev(c, key, requires_grad=False):
    return to_dev(c[key], c["dtype"], requires_grad)


@pytest.mark.parametrize("name", sorted(CASES))
def test_stages_match_golden(gpu_available, name):
    from linearard_amd.attention_KL import kl_backward, kl_forward, lse_stats

    c = CASES[name]
    print(f"golden stages: {name}", flush=True)
    qs, ks, qt, kt = (_dev(c, k) for k in ("qs", "ks", "qt", "kt"))
    m = mask_to_dev(c["mask"])
    lse_s = lse_stats(qs, ks, m, c["causal"])
    lse_t = lse_stats(qt, kt, m, c["causal"])
    for got, ref in ((lse_s, c["lse_s"]), (lse_t, c["lse_t"])):
        got = got.cpu().numpy().astype(np.float64)
        fin = np.isfinite(ref)
        assert np.array_equal(np.isfinite(got), fin)
        assert np.abs(got[fin] - ref[fin]).max() <= 1e-4 * max(1.0, np.abs(ref[fin]).max())
    loss = kl_forward(qs, ks, lse_s, qt, kt, lse_t, m, c["causal"])
    check_loss(loss.item(), c["loss"], f"golden-stages-{name}")
    dq, dk = kl_backward(qs, ks, lse_s, qt, kt, lse_t, m, c["causal"])
    check_grad(dq.cpu().numpy(), c["dq"], f"golden-stages-{name}", "dq")
    check_grad(dk.cpu().numpy(), c["dk"], f"golden-stages-{name}", "dk")


@pytest.mark.parametrize("name", sorted(CASES))
def test_autograd_matches_golden(gpu_available, name):
    from linearard_amd.attention_KL import attn_kl_align

    c = CASES[name]
    print(f"golden autograd: {name}", flush=True)
    m = mask_to_dev(c["mask"])
    cid = f"golden-autograd-{name}"
    if c["self_relation"]:
        x_s = _dev(c, "qs", requires_grad=True)
        x_t = _dev(c, "qt")
        loss = attn_kl_align(x_s, x_s, x_t, x_t, attn_mask=m, causal=c["causal"])
        loss.backward()
        check_loss(loss.item(), c["loss"], cid)
        check_grad(x_s.grad.float().cpu().numpy(), c["dq"] + c["dk"], cid)
    else:
        qs = _dev(c, "qs", requires_grad=True)
        ks = _dev(c, "ks", requires_grad=True)
        qt, kt = _dev(c, "qt"), _dev(c, "kt")
        loss = attn_kl_align(qs, ks, qt, kt, attn_mask=m, causal=c["causal"])
        (2.0 * loss).backward()
        check_loss(loss.item(), c["loss"], cid)
        check_grad(qs.grad.float().cpu().numpy(), 2.0 * c["dq"], cid, "dq")
        check_grad(ks.grad.float().cpu().numpy(), 2.0 * c["dk"], cid, "dk")
        assert qt.grad is None and kt.grad is None
