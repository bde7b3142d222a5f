"""Pins the logits-KL oracle (oracle/logits_kl.py) without a GPU.

Independent checks, each chosen so a plausible slip fails one of them:
scipy's log_softmax / rel_entr (a swapped t/s or a missing lse), closed
forms (a two-word vocabulary; identical and row-shifted logits give 0),
central finite differences of the loss for both gradients and both
reductions (a sign, a missing 1/T or 1/rows), and the reference's own lines
(train.py:412-419) evaluated by torch on the CPU (bf16 within the bound of
its roundings, float32 tightly).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.special import log_softmax, logsumexp, rel_entr

from oracle import logits_kl as O
from oracle.attn_kl import round_to


def _logits(rng, shape, dtype, scale=3.0):
    return round_to((scale * rng.standard_normal(shape)).astype(np.float32), dtype)


@pytest.mark.parametrize("T", [1.0, 2.0, 0.5])
def test_oracle_matches_scipy(T):
    rng = np.random.default_rng(1)
    t = _logits(rng, (2, 3, 50), "bf16")
    s = _logits(rng, (2, 3, 50), "bf16")
    loss, kl, lse_t, lse_s = O.logits_kl(t, s, T, "bf16")
    qt, qs = t.astype(np.float64) / T, s.astype(np.float64) / T  # 1/T exact: no rounding in x * (1/T)
    ref = rel_entr(np.exp(log_softmax(qt, axis=-1)), np.exp(log_softmax(qs, axis=-1))).sum(-1)
    np.testing.assert_allclose(kl, ref, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(lse_t, logsumexp(qt, axis=-1), rtol=1e-12)
    np.testing.assert_allclose(lse_s, logsumexp(qs, axis=-1), rtol=1e-12)
    assert loss == pytest.approx(ref.mean(), rel=1e-10)


def test_two_word_vocabulary_closed_form():
    rng = np.random.default_rng(2)
    t = rng.standard_normal((5, 2)).astype(np.float32)
    s = rng.standard_normal((5, 2)).astype(np.float32)
    _, kl, _, _ = O.logits_kl(t, s, 1.0, "f32")
    for r in range(5):
        p = 1.0 / (1.0 + math.exp(float(t[r, 0]) - float(t[r, 1])))  # P(word 1) under the teacher
        q = 1.0 / (1.0 + math.exp(float(s[r, 0]) - float(s[r, 1])))
        want = p * math.log(p / q) + (1 - p) * math.log((1 - p) / (1 - q))
        assert kl[r] == pytest.approx(want, rel=1e-12, abs=1e-15)


def test_identical_and_row_shifted_logits_give_zero():
    rng = np.random.default_rng(3)
    t = rng.standard_normal((3, 4, 64)).astype(np.float32)
    shift = np.arange(12, dtype=np.float32).reshape(3, 4, 1) * 0.25  # exact in float32
    loss, kl, _, _ = O.logits_kl(t, t + shift, 1.0, "f32")
    assert np.max(np.abs(kl)) < 1e-13 and abs(loss) < 1e-13
    loss0, _, _, _ = O.logits_kl(t, t, 1.0, "f32")
    assert loss0 == 0.0
    gt, gs = O.logits_kl_grads(t, t, 1.0, "f32")
    assert np.all(gt == 0.0) and np.all(gs == 0.0)


def test_kl_is_not_symmetric_and_positive():
    rng = np.random.default_rng(4)
    t = _logits(rng, (4, 40), "f32")
    s = _logits(rng, (4, 40), "f32")
    _, kts, _, _ = O.logits_kl(t, s, 1.0, "f32")
    _, kst, _, _ = O.logits_kl(s, t, 1.0, "f32")
    assert np.all(kts > 0) and np.all(kst > 0)
    assert np.max(np.abs(kts - kst)) > 1e-3  # the direction matters: KL(p_t || p_s)


def _fd_grads(t, s, T, reduction, w):
    """Central differences of sum_r w_r kl_r (or w * mean) over every logit,
    with the actual float32 step taken."""

    def f(tt, ss):
        loss, kl, _, _ = O.logits_kl(tt, ss, T, "f32")
        return float(np.sum(np.asarray(w) * kl)) if reduction == "none" else float(w) * loss

    h = 1e-3
    out = []
    for which in (0, 1):
        base = (t, s)[which]
        g = np.zeros(base.shape)
        for idx in np.ndindex(base.shape):
            xp, xm = base.copy(), base.copy()
            xp[idx] = np.float32(base[idx] + h)
            xm[idx] = np.float32(base[idx] - h)
            step = float(xp[idx]) - float(xm[idx])
            fp = f(xp, s) if which == 0 else f(t, xp)
            fm = f(xm, s) if which == 0 else f(t, xm)
            g[idx] = (fp - fm) / step
        out.append(g)
    return out


@pytest.mark.parametrize("T,reduction,tol", [
    (1.0, "mean", 2e-6),
    (2.0, "none", 2e-6),   # 1/T and x * (1/T) exact
    (1.7, "mean", 3e-4),   # x * (1/T) rounded to float32: the step is only approximately scaled
])
def test_gradients_match_finite_differences(T, reduction, tol):
    rng = np.random.default_rng(5)
    t = _logits(rng, (1, 2, 6), "f32", 1.5)
    s = _logits(rng, (1, 2, 6), "f32", 1.5)
    w = rng.uniform(0.5, 2.0, (1, 2)) if reduction == "none" else 1.3
    gt, gs = O.logits_kl_grads(t, s, T, "f32", dloss=w, reduction=reduction)
    ft, fs = _fd_grads(t, s, T, reduction, w)
    scale = max(np.max(np.abs(ft)), np.max(np.abs(fs)))
    assert np.max(np.abs(gt - ft)) <= tol * scale, (gt, ft)
    assert np.max(np.abs(gs - fs)) <= tol * scale, (gs, fs)


def _reference_lines(t_logits, s_logits, T):
    """train.py:412-419, verbatim operations, on CPU torch tensors."""
    t_logp = F.log_softmax(t_logits / T, dim=-1)
    s_logp = F.log_softmax(s_logits / T, dim=-1)
    t_p = t_logp.exp()
    kl_per_tok = (t_p * (t_logp - s_logp)).sum(dim=-1)
    return kl_per_tok.mean(), kl_per_tok


def bf16_pipeline_bound(t, s, T, dtype="bf16"):
    """Bound on |reference lines in `dtype` - exact| per row, from the exact
    values: every elementwise result rounded to the dtype (unit roundoff u),
    float32 accumulation of the vocabulary sum, one rounding of the sum."""
    u = 2.0 ** -8 if dtype == "bf16" else 2.0 ** -11
    qt = O.scale_logits(t, T, dtype).astype(np.float64)
    qs = O.scale_logits(s, T, dtype).astype(np.float64)
    lt = qt - logsumexp(qt, axis=-1, keepdims=True)
    ls = qs - logsumexp(qs, axis=-1, keepdims=True)
    pt = np.exp(lt)
    d = lt - ls
    dd = 1.01 * u * (np.abs(lt) + np.abs(ls) + np.abs(d))            # rounded log-probs and difference
    dp = pt * (np.exp(u * np.abs(lt)) * (1 + u) - 1)                 # rounded log-prob, exp, rounding
    prod = (pt + dp) * (np.abs(d) + dd)
    dprod = (pt + dp) * dd + np.abs(d) * dp + u * prod
    V = t.shape[-1]
    kl = np.sum(pt * d, axis=-1)
    row = np.sum(dprod, axis=-1) + (V * 2.0 ** -24) * np.sum(prod, axis=-1) + u * (np.abs(kl) + np.sum(dprod, -1))
    return row


@pytest.mark.parametrize("T", [1.0, 2.0])
def test_oracle_against_the_reference_lines_in_bf16(T):
    rng = np.random.default_rng(6)
    t = _logits(rng, (2, 4, 1000), "bf16", 4.0)
    s = round_to(0.5 * t + rng.standard_normal(t.shape).astype(np.float32), "bf16")
    loss, kl, _, _ = O.logits_kl(t, s, T, "bf16")
    ref_loss, ref_kl = _reference_lines(torch.from_numpy(t).to(torch.bfloat16),
                                        torch.from_numpy(s).to(torch.bfloat16), T)
    ref_kl = ref_kl.float().numpy().reshape(kl.shape)
    bound = 2.0 * bf16_pipeline_bound(t, s, T)
    err = np.abs(ref_kl - kl)
    assert np.all(err <= bound), (err.max(), bound.min())
    assert abs(float(ref_loss) - loss) <= bound.mean() + 2.0 ** -8 * abs(loss)
    # the bound still sees plausible slips: a wrong temperature, swapped roles
    _, kl_wrong_t, _, _ = O.logits_kl(t, s, 2.0 if T == 1.0 else 1.0, "bf16")
    assert np.any(np.abs(ref_kl - kl_wrong_t) > bound)
    if T == 1.0:
        _, kl_swapped, _, _ = O.logits_kl(s, t, T, "bf16")
        assert np.any(np.abs(ref_kl - kl_swapped) > bound)


def test_oracle_against_the_reference_lines_in_float32():
    rng = np.random.default_rng(7)
    t = _logits(rng, (3, 2, 777), "f32")
    s = _logits(rng, (3, 2, 777), "f32")
    loss, kl, _, _ = O.logits_kl(t, s, 0.8, "f32")
    ref_loss, ref_kl = _reference_lines(torch.from_numpy(t), torch.from_numpy(s), 0.8)
    np.testing.assert_allclose(ref_kl.numpy(), kl, rtol=2e-5, atol=2e-5)
    assert float(ref_loss) == pytest.approx(loss, rel=2e-5)


@pytest.mark.parametrize("T", [2.0, 0.5, 4.0])
def test_scale_logits_exact_reciprocals_match_tensor_division(T):
    rng = np.random.default_rng(8)
    x = _logits(rng, (4, 300), "bf16", 10.0)
    q = O.scale_logits(x, T, "bf16")
    want = (torch.from_numpy(x).to(torch.bfloat16) / T).float().numpy()
    assert np.array_equal(q, want)


def test_scale_logits_reciprocal_product_is_within_one_ulp_of_division():
    """For T with an inexact reciprocal the CUDA rule (x * (1/T), then the
    dtype rounding) and true division (torch's CPU kernel) differ at most
    by one bf16 ulp, and rarely."""
    rng = np.random.default_rng(9)
    x = _logits(rng, (64, 500), "bf16", 10.0)
    q = O.scale_logits(x, 0.7, "bf16")
    div = (torch.from_numpy(x).to(torch.bfloat16) / 0.7).float().numpy()
    ulp = np.abs(div) * 2.0 ** -7
    diff = np.abs(q - div)
    assert np.all(diff <= ulp)
    assert np.mean(diff > 0) < 0.01
    assert np.max(np.abs(q - x / 0.7)) <= np.max(np.abs(x / 0.7)) * 2.0 ** -8  # a division, not a product by T


def test_empty_inputs():
    loss, kl, lse_t, _ = O.logits_kl(np.zeros((0, 5), np.float32), np.zeros((0, 5), np.float32), 1.0, "f32")
    assert math.isnan(loss) and kl.shape == (0,)
    loss, kl, lse_t, _ = O.logits_kl(np.zeros((2, 0), np.float32), np.zeros((2, 0), np.float32), 1.0, "f32")
    # torch: log_softmax of an empty row is empty, its sum 0: KL 0
    assert loss == 0.0 and np.all(kl == 0.0)
