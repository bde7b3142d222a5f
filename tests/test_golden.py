"""The committed golden fixtures (tests/golden/) against the CPU oracle and an
independent formulation; no GPU needed."""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from tests.golden import golden

CASES = golden.load()


def test_fixture_set_is_complete():
    assert len(CASES) == 5
    assert any(c["self_relation"] for c in CASES.values())
    assert any(not c["causal"] for c in CASES.values())
    assert any(c["mask"] is not None for c in CASES.values())
    assert {c["dtype"] for c in CASES.values()} == {"bf16", "f16"}


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    c = CASES[name]
    loss, dq, dk, lse_s, lse_t = O.attn_kl_align(c["qs"], c["ks"], c["qt"], c["kt"], c["mask"], c["causal"],
                                                 None, None, d_cast=c["dtype"])
    assert loss == pytest.approx(c["loss"], rel=1e-12, abs=1e-12)
    np.testing.assert_allclose(lse_s, c["lse_s"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse_t, c["lse_t"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dq, c["dq"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(dk, c["dk"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_loss_matches_materialized_formula(name):
    """integration.py:102-127 restated as an explicit log-softmax, sharing no code with kl_rows."""
    c = CASES[name]
    ref = O.materialized_kl(c["qs"], c["ks"], c["qt"], c["kt"], c["mask"], c["causal"])
    assert c["loss"] == pytest.approx(ref, rel=1e-9, abs=1e-9)


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_grads_match_torch_autograd(name):
    """float64 autograd of the materialised loss; the fixtures cast D to the input
    dtype like kernel_C.py:233, so they agree to that dtype's precision."""
    c = CASES[name]
    qs = torch.tensor(c["qs"], dtype=torch.float64, requires_grad=True)
    ks = qs if c["self_relation"] else torch.tensor(c["ks"], dtype=torch.float64, requires_grad=True)
    qt = torch.tensor(c["qt"], dtype=torch.float64)
    kt = torch.tensor(c["kt"], dtype=torch.float64)
    B, Hq, T, Ds = qs.shape
    Dt = qt.shape[-1]
    g_s, g_t = Hq // ks.shape[1], Hq // kt.shape[1]
    ks_e = ks.repeat_interleave(g_s, dim=1)
    kt_e = kt.repeat_interleave(g_t, dim=1)
    valid = torch.ones(B, 1, T, T, dtype=torch.bool)
    if c["causal"]:
        valid &= torch.ones(T, T, dtype=torch.bool).tril()
    if c["mask"] is not None:
        m = torch.tensor(c["mask"] != 0)
        valid &= m[:, None, :, None] & m[:, None, None, :]
    ls = (qs @ ks_e.transpose(-1, -2)) / math.sqrt(Ds)
    lt = (qt @ kt_e.transpose(-1, -2)) / math.sqrt(Dt)
    neg = torch.finfo(torch.float64).min
    lps = torch.log_softmax(ls.masked_fill(~valid, neg), -1)
    lpt = torch.log_softmax(lt.masked_fill(~valid, neg), -1)
    rows = valid.any(-1, keepdim=True)
    loss = (lpt.exp() * (lpt - lps)).masked_fill(~(valid & rows), 0.0).sum()
    loss.backward()
    assert loss.item() == pytest.approx(c["loss"], rel=1e-9, abs=1e-9)
    if c["self_relation"]:
        got, ref = c["dq"] + c["dk"], qs.grad.numpy()
        assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()
    else:
        for got, ref in ((c["dq"], qs.grad.numpy()), (c["dk"], ks.grad.numpy())):
            assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()
