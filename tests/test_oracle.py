"""Pin the CPU oracle against formulations that do not share its code.

Every oracle function is checked here by something other than a retyped
copy of its own formula: pure-Python brute force (``math.fsum``), scipy's
``logsumexp`` / ``rel_entr``, closed forms, central finite differences and
torch float64 autograd.  ``test_planted_*`` confirm that plausible mistakes
(a dropped transpose, a sign flip, an off-by-one causal mask) are caught.
"""

import math

import numpy as np
import pytest
import scipy.special as sps
import torch

from oracle import attn_kl as O


def _rand(rng, *shape, scale=1.0):
    return rng.standard_normal(shape) * scale


def _mask(rng, B, T, ratio):
    m = (rng.random((B, T)) > ratio).astype(np.int32)
    m[:, 0] = 1  # the reference tests force column 0 valid (test_kernel_A.py:239)
    return m


# --------------------------------------------------------------------------
# brute-force restatements (tiny sizes only)
# --------------------------------------------------------------------------

def _brute_lse(q, k, mask, causal, scale):
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    out = np.zeros((B, Hq, T))
    for b in range(B):
        for h in range(Hq):
            for i in range(T):
                if mask is not None and mask[b, i] == 0:
                    out[b, h, i] = 0.0
                    continue
                vals = []
                for j in range(T):
                    if causal and j > i:
                        continue
                    if mask is not None and mask[b, j] == 0:
                        continue
                    s = math.fsum(float(q[b, h, i, d]) * float(k[b, h // g, j, d]) for d in range(D))
                    vals.append(s * scale)
                if not vals:
                    out[b, h, i] = -math.inf
                    continue
                m = max(vals)
                out[b, h, i] = m + math.log(math.fsum(math.exp(v - m) for v in vals))
    return out


def _brute_loss(qs, ks, qt, kt, mask, causal, ss, st):
    """sum_rows KL(P_t || P_s) from explicit softmax probabilities."""
    B, Hq, T, _ = qs.shape
    gs = Hq // ks.shape[1]
    gt = Hq // kt.shape[1]
    total = []
    for b in range(B):
        for h in range(Hq):
            for i in range(T):
                if mask is not None and mask[b, i] == 0:
                    continue
                js = [j for j in range(T) if (not causal or j <= i) and (mask is None or mask[b, j] != 0)]
                a = [ss * math.fsum(qs[b, h, i, d] * ks[b, h // gs, j, d] for d in range(qs.shape[3])) for j in js]
                c = [st * math.fsum(qt[b, h, i, d] * kt[b, h // gt, j, d] for d in range(qt.shape[3])) for j in js]
                za = math.fsum(math.exp(x - max(a)) for x in a)
                zc = math.fsum(math.exp(x - max(c)) for x in c)
                for x, y in zip(a, c):
                    ps = math.exp(x - max(a)) / za
                    pt = math.exp(y - max(c)) / zc
                    total.append(pt * (math.log(pt) - math.log(ps)))
    return math.fsum(total)


# --------------------------------------------------------------------------
# stage A
# --------------------------------------------------------------------------

@pytest.mark.parametrize("causal,ratio,hq,hkv", [(True, None, 2, 2), (False, 0.4, 4, 2), (True, 0.5, 4, 1)])
def test_lse_matches_bruteforce(causal, ratio, hq, hkv):
    rng = np.random.default_rng(11)
    B, T, D = 2, 6, 8
    q = _rand(rng, B, hq, T, D)
    k = _rand(rng, B, hkv, T, D)
    mask = None if ratio is None else _mask(rng, B, T, ratio)
    scale = 1.0 / math.sqrt(D)
    got = O.lse_stats(q, k, mask, causal, scale)
    ref = _brute_lse(q, k, mask, causal, scale)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_lse_matches_scipy_logsumexp():
    rng = np.random.default_rng(3)
    B, H, T, D = 1, 3, 17, 16
    q = _rand(rng, B, H, T, D)
    k = _rand(rng, B, H, T, D)
    mask = _mask(rng, B, T, 0.3)
    got = O.lse_stats(q, k, mask, True, 0.25)
    for h in range(H):
        for i in range(T):
            if mask[0, i] == 0:
                assert got[0, h, i] == 0.0
                continue
            cols = [j for j in range(i + 1) if mask[0, j]]
            s = 0.25 * (q[0, h, i] @ k[0, h, cols].T)
            assert abs(got[0, h, i] - sps.logsumexp(s)) < 1e-12


def test_lse_closed_forms_and_bounds():
    rng = np.random.default_rng(5)
    B, H, T, D = 2, 2, 40, 32
    x = _rand(rng, B, H, T, D, scale=2.0)
    a = 1.0 / math.sqrt(D)
    lse = O.lse_stats(x, x, None, True, a)
    # causal self relation, row 0 sees only itself: lse_0 = a * |x_0|^2
    np.testing.assert_allclose(lse[..., 0], a * (x[..., 0, :] ** 2).sum(-1), rtol=1e-13)
    # max S <= lse <= max S + log |V(i)|
    S = a * np.matmul(x, np.swapaxes(x, -1, -2))
    S = np.where(np.tril(np.ones((T, T), bool)), S, -np.inf)
    mx = S.max(-1)
    nvalid = np.arange(1, T + 1)
    assert np.all(lse >= mx - 1e-12)
    assert np.all(lse <= mx + np.log(nvalid) + 1e-12)


def test_lse_invalid_rows_zero_and_empty_rows_neg_inf():
    rng = np.random.default_rng(7)
    q = _rand(rng, 1, 2, 5, 8)
    mask = np.array([[1, 0, 1, 0, 1]])
    lse = O.lse_stats(q, q, mask, True, 0.3)
    assert np.all(lse[:, :, [1, 3]] == 0.0)
    assert np.all(np.isfinite(lse))
    # a q row whose k columns are all masked cannot occur with a shared mask;
    # exercise the -inf rule through a teacher/student lse pair instead
    lse_s = lse.copy()
    lse_s[0, 0, 2] = -np.inf
    rows = O.kl_rows(q, q, lse_s, q, q, lse, mask, True, 0.3, 0.3)
    assert rows[0, 0, 2] == 0.0


# --------------------------------------------------------------------------
# stage B
# --------------------------------------------------------------------------

def test_kl_matches_scipy_rel_entr():
    rng = np.random.default_rng(13)
    B, H, T, D = 1, 2, 20, 16
    xs = _rand(rng, B, H, T, D)
    xt = xs + 0.3 * _rand(rng, B, H, T, D)
    a = 1.0 / math.sqrt(D)
    lse_s = O.lse_stats(xs, xs, None, True, a)
    lse_t = O.lse_stats(xt, xt, None, True, a)
    rows = O.kl_rows(xs, xs, lse_s, xt, xt, lse_t, None, True, a, a)
    for h in range(H):
        for i in range(T):
            ps = sps.softmax(a * xs[0, h, i] @ xs[0, h, : i + 1].T)
            pt = sps.softmax(a * xt[0, h, i] @ xt[0, h, : i + 1].T)
            assert abs(rows[0, h, i] - sps.rel_entr(pt, ps).sum()) < 1e-12


@pytest.mark.parametrize("causal,ratio,hq,hks,hkt,ds,dt", [
    (True, None, 2, 2, 2, 8, 8),
    (False, 0.3, 4, 2, 1, 8, 16),
    (True, 0.5, 4, 1, 2, 16, 8),
])
def test_kl_matches_bruteforce(causal, ratio, hq, hks, hkt, ds, dt):
    rng = np.random.default_rng(17)
    B, T = 2, 5
    qs, ks = _rand(rng, B, hq, T, ds), _rand(rng, B, hks, T, ds)
    qt, kt = _rand(rng, B, hq, T, dt), _rand(rng, B, hkt, T, dt)
    mask = None if ratio is None else _mask(rng, B, T, ratio)
    ss, st = 1 / math.sqrt(ds), 1 / math.sqrt(dt)
    loss, *_ = O.attn_kl_align(qs, ks, qt, kt, mask, causal, ss, st)
    assert abs(loss - _brute_loss(qs, ks, qt, kt, mask, causal, ss, st)) < 1e-11


def test_kl_matches_materialized_formula():
    rng = np.random.default_rng(19)
    B, Hq, T = 2, 4, 23
    qs, ks = _rand(rng, B, Hq, T, 32), _rand(rng, B, 2, T, 32)
    qt, kt = _rand(rng, B, Hq, T, 16), _rand(rng, B, 1, T, 16)
    mask = _mask(rng, B, T, 0.3)
    for causal in (True, False):
        loss, *_ = O.attn_kl_align(qs, ks, qt, kt, mask, causal)
        ref = O.materialized_kl(qs, ks, qt, kt, mask, causal)
        assert abs(loss - ref) <= 1e-10 * max(1.0, abs(ref))


def test_kl_zero_for_identical_relations_and_nonnegative():
    rng = np.random.default_rng(23)
    x = _rand(rng, 1, 3, 30, 16)
    loss, dx, _, _, _ = O.attn_kl_align(x, x, x, x, None, True, 0.25, 0.25, self_relation=True)
    assert loss == 0.0
    assert np.all(dx == 0.0)
    y = x + 0.5 * _rand(rng, 1, 3, 30, 16)
    lse_s = O.lse_stats(x, x, None, True, 0.25)
    lse_t = O.lse_stats(y, y, None, True, 0.25)
    rows = O.kl_rows(x, x, lse_s, y, y, lse_t, None, True, 0.25, 0.25)
    assert np.all(rows >= -1e-14)
    assert np.all(rows[..., 0] == 0.0)  # causal row 0: both distributions are a point mass


# --------------------------------------------------------------------------
# stage C
# --------------------------------------------------------------------------

def _loss_of(qs, ks, qt, kt, mask, causal, ss, st):
    lse_s = O.lse_stats(qs, ks, mask, causal, ss)
    lse_t = O.lse_stats(qt, kt, mask, causal, st)
    return O.kl_forward(qs, ks, lse_s, qt, kt, lse_t, mask, causal, ss, st)


@pytest.mark.parametrize("causal,ratio", [(True, None), (False, 0.4), (True, 0.4)])
def test_grads_match_finite_differences(causal, ratio):
    rng = np.random.default_rng(29)
    B, Hq, Hks, Hkt, T, Ds, Dt = 1, 4, 2, 1, 6, 8, 16
    qs, ks = _rand(rng, B, Hq, T, Ds), _rand(rng, B, Hks, T, Ds)
    qt, kt = _rand(rng, B, Hq, T, Dt), _rand(rng, B, Hkt, T, Dt)
    mask = None if ratio is None else _mask(rng, B, T, ratio)
    ss, st = 0.4, 0.3
    _, dq, dk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, causal, ss, st)
    eps = 1e-6
    for arr, grad in ((qs, dq), (ks, dk)):
        idx = list(np.ndindex(arr.shape))
        for n in rng.choice(len(idx), size=40, replace=False):
            ix = idx[n]
            old = arr[ix]
            arr[ix] = old + eps
            lp = _loss_of(qs, ks, qt, kt, mask, causal, ss, st)
            arr[ix] = old - eps
            lm = _loss_of(qs, ks, qt, kt, mask, causal, ss, st)
            arr[ix] = old
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - grad[ix]) < 1e-6 * max(1.0, abs(fd)), (ix, fd, grad[ix])


def test_grads_match_torch_autograd_float64():
    rng = np.random.default_rng(31)
    B, Hq, Hks, Hkt, T, Ds, Dt = 2, 4, 2, 4, 19, 16, 32
    qs, ks = _rand(rng, B, Hq, T, Ds), _rand(rng, B, Hks, T, Ds)
    qt, kt = _rand(rng, B, Hq, T, Dt), _rand(rng, B, Hkt, T, Dt)
    mask = _mask(rng, B, T, 0.3)
    ss, st = 1 / math.sqrt(Ds), 1 / math.sqrt(Dt)
    _, dq, dk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, False, ss, st)

    tqs = torch.tensor(qs, requires_grad=True)
    tks = torch.tensor(ks, requires_grad=True)
    tqt, tkt = torch.tensor(qt), torch.tensor(kt)
    mb = torch.tensor(mask).bool()
    valid = mb[:, None, :, None] & mb[:, None, None, :]
    ls = torch.matmul(tqs, tks.repeat_interleave(Hq // Hks, 1).transpose(-1, -2)) * ss
    lt = torch.matmul(tqt, tkt.repeat_interleave(Hq // Hkt, 1).transpose(-1, -2)) * st
    ls = ls.masked_fill(~valid, float("-inf"))
    lt = lt.masked_fill(~valid, float("-inf"))
    rows = valid.any(-1, keepdim=True)
    lps = torch.log_softmax(ls.masked_fill(~rows, 0.0), -1)
    lpt = torch.log_softmax(lt.masked_fill(~rows, 0.0), -1)
    term = torch.where(valid, lpt.exp() * (lpt - lps), torch.zeros_like(lps))
    term.sum().backward()
    np.testing.assert_allclose(tqs.grad.numpy(), dq, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(tks.grad.numpy(), dk, rtol=1e-9, atol=1e-12)


def test_self_relation_gradient_is_dq_plus_dk():
    rng = np.random.default_rng(37)
    x = _rand(rng, 1, 2, 12, 8)
    y = x + 0.4 * _rand(rng, 1, 2, 12, 8)
    loss, dx, none, _, _ = O.attn_kl_align(x, x, y, y, None, True, 0.3, 0.3, self_relation=True)
    assert none is None
    # finite differences of the self relation loss w.r.t. the shared input
    eps = 1e-6
    for ix in [(0, 0, 0, 0), (0, 1, 5, 3), (0, 0, 11, 7), (0, 1, 2, 2)]:
        old = x[ix]
        x[ix] = old + eps
        lp = _loss_of(x, x, y, y, None, True, 0.3, 0.3)
        x[ix] = old - eps
        lm = _loss_of(x, x, y, y, None, True, 0.3, 0.3)
        x[ix] = old
        assert abs((lp - lm) / (2 * eps) - dx[ix]) < 1e-7


def test_chunked_self_relation_matches_full():
    rng = np.random.default_rng(41)
    T, D = 300, 16
    xs = rng.standard_normal((T, D))
    xt = xs + 0.3 * rng.standard_normal((T, D))
    mask = (rng.random(T) > 0.2).astype(np.int64)
    mask[0] = 1
    for causal in (True, False):
        loss, dx, lse_s, lse_t, _ = O.self_relation_chunked(xs, xt, causal, 0.25, 0.3, mask=mask,
                                                            chunk=64, dtype=np.float64)
        rl, rdx, _, rls, rlt = O.attn_kl_align(xs[None, None], xs[None, None], xt[None, None],
                                              xt[None, None], mask[None], causal, 0.25, 0.3,
                                              self_relation=True)
        assert abs(loss - rl) < 1e-10 * max(1, abs(rl))
        np.testing.assert_allclose(dx, rdx[0, 0], rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(lse_s, rls[0, 0], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(lse_t, rlt[0, 0], rtol=1e-12, atol=1e-12)


# --------------------------------------------------------------------------
# dtype emulation and planted mistakes
# --------------------------------------------------------------------------

def test_round_bf16_matches_torch():
    rng = np.random.default_rng(43)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-40, 3e38, -3e38, np.inf, -np.inf], np.float32)])
    ref = torch.tensor(x).to(torch.bfloat16).float().numpy()
    got = O.round_bf16(x)
    np.testing.assert_array_equal(got, ref)
    assert np.isnan(O.round_bf16(np.array([np.nan], np.float32)))[0]
    np.testing.assert_array_equal(O.round_f16(x[:10000]), torch.tensor(x[:10000]).half().float().numpy())


def test_d_cast_changes_result_only_at_dtype_precision():
    rng = np.random.default_rng(47)
    qs, qt = _rand(rng, 1, 2, 33, 64), _rand(rng, 1, 2, 33, 64)
    lse_s = O.lse_stats(qs, qs, None, True, 0.125)
    lse_t = O.lse_stats(qt, qt, None, True, 0.125)
    dq, dk = O.kl_backward(qs, qs, lse_s, qt, qt, lse_t, None, True, 0.125, 0.125)
    dqc, dkc = O.kl_backward(qs, qs, lse_s, qt, qt, lse_t, None, True, 0.125, 0.125, d_cast="bf16")
    rel = np.abs(dqc - dq).max() / np.abs(dq).max()
    assert 0 < rel < 1e-2


def test_planted_mistakes_are_caught_by_the_independent_checks():
    """A transposed dk, a flipped KL sign and an off-by-one causal mask must
    each disagree with the brute-force / autograd checks used above."""
    rng = np.random.default_rng(53)
    B, H, T, D = 1, 2, 6, 8
    qs, qt = _rand(rng, B, H, T, D), _rand(rng, B, H, T, D)
    a = 1 / math.sqrt(D)
    loss, dq, dk, lse_s, lse_t = O.attn_kl_align(qs, qs, qt, qt, None, True, a, a)
    brute = _brute_loss(qs, qs, qt, qt, None, True, a, a)
    assert abs(loss - brute) < 1e-11
    assert abs(-loss - brute) > 1e-3  # sign flip
    # off-by-one causal: strict lower triangle changes the LSE
    Sx = a * np.matmul(qs, np.swapaxes(qs, -1, -2))
    strict = np.where(np.tril(np.ones((T, T), bool), -1), Sx, -np.inf)[..., 1:, :]
    assert np.abs(sps.logsumexp(strict, axis=-1) - lse_s[..., 1:]).max() > 1e-3
    # dropping the transpose in the dk product breaks the self-relation FD check
    wrong_dx = dq + np.swapaxes(dk, -1, -2)[..., :D] if T == D else dq + dk[..., ::-1]
    eps = 1e-6
    ix = (0, 1, 4, 2)
    old = qs[ix]
    qs[ix] = old + eps
    lp = _loss_of(qs, qs, qt, qt, None, True, a, a)
    qs[ix] = old - eps
    lm = _loss_of(qs, qs, qt, qt, None, True, a, a)
    qs[ix] = old
    fd = (lp - lm) / (2 * eps)
    assert abs(fd - (dq + dk)[ix]) < 1e-7
    assert abs(fd - wrong_dx[ix]) > 1e-5
