"""float32 inputs: the stage entry points and the autograd pair against the
float64 oracle and against float32 eager PyTorch (materialised KL).

The reference's kernels take fp16/bf16 only (kernel_A.py:195-196); the
float32 path keeps the products and D = P_s - P_t in float32.  Tolerance
(written here, from the benchmark contract): loss relative error <= 1e-5
and gradient max-abs error <= 1e-5 of the gradient's max magnitude.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from tests._inputs import make_mask, mask_to_dev, randn, to_dev
from tests._tolerance import check_grad, check_loss

pytestmark = pytest.mark.gpu

F32_BAR = 1e-5  # the north star's float32 bar, for the loss and the gradients

CASES = [  # causal, ratio, B, hq, hks, hkt, T, ds, dt
    (True, None, 1, 4, 4, 4, 97, 128, 128),
    (False, 0.3, 2, 4, 2, 1, 65, 64, 64),
    (True, 0.2, 1, 8, 2, 4, 130, 32, 128),   # GQA on both sides, Ds != Dt
    (True, None, 1, 2, 2, 2, 40, 256, 8),
    (True, None, 1, 1, 1, 1, 1, 16, 16),     # one token
]


def _inputs(rng, B, hq, hks, hkt, T, ds, dt, ratio, scale=1.0):
    qs = randn(rng, (B, hq, T, ds), "f32", scale)
    ks = randn(rng, (B, hks, T, ds), "f32", scale)
    qt = randn(rng, (B, hq, T, dt), "f32", scale)
    kt = randn(rng, (B, hkt, T, dt), "f32", scale)
    mask = None if ratio is None else make_mask(rng, B, T, ratio)
    return qs, ks, qt, kt, mask


@pytest.mark.parametrize("causal,ratio,B,hq,hks,hkt,T,ds,dt", CASES)
def test_f32_stages_match_the_oracle(gpu_available, causal, ratio, B, hq, hks, hkt, T, ds, dt):
    from linearard_amd.attention_KL import kl_backward, kl_forward, lse_stats

    rng = np.random.default_rng(T * 31 + ds + dt)
    qs, ks, qt, kt, mask = _inputs(rng, B, hq, hks, hkt, T, ds, dt, ratio)
    a_s, a_t = 1 / math.sqrt(ds), 1 / math.sqrt(dt)
    d = [to_dev(x, "f32") for x in (qs, ks, qt, kt)]
    m = mask_to_dev(mask)
    lse_s = lse_stats(d[0], d[1], m, causal, a_s)
    lse_t = lse_stats(d[2], d[3], m, causal, a_t)
    rls = O.lse_stats(qs, ks, mask, causal, a_s)
    rlt = O.lse_stats(qt, kt, mask, causal, a_t)
    np.testing.assert_allclose(lse_s.cpu().numpy(), rls, rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(lse_t.cpu().numpy(), rlt, rtol=1e-6, atol=1e-5)
    loss = float(kl_forward(d[0], d[1], lse_s, d[2], d[3], lse_t, m, causal, a_s, a_t))
    ref = O.kl_forward(qs, ks, rls, qt, kt, rlt, mask, causal, a_s, a_t)
    case = f"f32-stages-c{int(causal)}-r{ratio}-T{T}-ds{ds}-dt{dt}"
    check_loss(loss, ref, case, bar=F32_BAR)
    dq, dk = kl_backward(d[0], d[1], lse_s, d[2], d[3], lse_t, m, causal, a_s, a_t)
    rq, rk = O.kl_backward(qs, ks, rls, qt, kt, rlt, mask, causal, a_s, a_t)  # D exact (no cast)
    for name, got, want in (("dq", dq, rq), ("dk", dk, rk)):
        check_grad(got.cpu().numpy(), want, case, name, bar=F32_BAR)


@pytest.mark.parametrize("ratio", [None, 0.25])
def test_f32_autograd_self_relation_matches_the_oracle(gpu_available, ratio):
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(17)
    B, H, T, D = 1, 4, 300, 128
    xt = randn(rng, (B, H, T, D), "f32")
    xs = (xt + 0.1 * rng.standard_normal(xt.shape)).astype(np.float32)
    mask = None if ratio is None else make_mask(rng, B, T, ratio)
    a = 1 / math.sqrt(D)
    x = to_dev(xs, "f32", requires_grad=True)
    y = to_dev(xt, "f32")
    loss = attn_kl_align(x, x, y, y, attn_mask=mask_to_dev(mask), causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    ref, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, mask, True, a, a, self_relation=True)
    check_loss(loss.item(), ref, f"f32-autograd-r{ratio}", bar=F32_BAR)
    assert x.grad.dtype == torch.float32
    check_grad(x.grad.cpu().numpy(), rdx, f"f32-autograd-r{ratio}", bar=F32_BAR)


def test_f32_cfg1_against_eager_pytorch(gpu_available):
    """BASELINE cfg1: B=1, H=32, n=1024, d=128, X_t ~ N(0,1) (seed 0),
    X_s = X_t + 0.1 N(0,1), scale 1/sqrt(d), causal; against float32 eager
    PyTorch with the n x n relation maps materialised (integration.py:102-127
    as a formula: sum over rows of KL(softmax(S_t) || softmax(S_s)))."""
    from linearard_amd.attention_KL import attn_kl_align

    g = torch.Generator().manual_seed(0)
    B, H, n, d = 1, 32, 1024, 128
    xt = torch.randn((B, H, n, d), generator=g)
    xs = xt + 0.1 * torch.randn((B, H, n, d), generator=g)
    a = 1 / math.sqrt(d)
    x = xs.cuda().requires_grad_(True)
    y = xt.cuda()
    loss = attn_kl_align(x, x, y, y, causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()

    xr = xs.cuda().requires_grad_(True)
    causal = torch.ones((n, n), dtype=torch.bool, device="cuda").tril()
    s_s = torch.matmul(xr, xr.transpose(-1, -2).contiguous()) * a
    s_t = torch.matmul(y, y.transpose(-1, -2).contiguous()) * a
    neg = torch.tensor(float("-inf"), device="cuda")
    ls = torch.log_softmax(torch.where(causal, s_s, neg), dim=-1)
    lt = torch.log_softmax(torch.where(causal, s_t, neg), dim=-1)
    pt = lt.exp()
    ref = torch.where(causal, pt * (lt - ls), torch.zeros((), device="cuda")).sum()
    ref.backward()
    # against the float64 oracle at the float32 bar
    rl, rdx, _, _, _ = O.attn_kl_align(xs.numpy(), xs.numpy(), xt.numpy(), xt.numpy(), None, True, a, a,
                                       self_relation=True)
    check_loss(loss.item(), rl, "f32-cfg1", bar=F32_BAR)
    check_grad(x.grad.cpu().numpy(), rdx, "f32-cfg1", bar=F32_BAR)
    # against float32 eager PyTorch, whose own float32 rounding is most of the
    # difference: the bar is F32_BAR or twice eager's deviation from float64
    eager_loss = abs(ref.item() - rl) / abs(rl)
    eager_grad = float(np.abs(xr.grad.cpu().numpy() - rdx).max() / np.abs(rdx).max())
    check_loss(loss.item(), ref.item(), "f32-cfg1-vs-eager-fp32", bar=max(F32_BAR, 2 * eager_loss))
    check_grad(x.grad.cpu().numpy(), xr.grad.cpu().numpy(), "f32-cfg1-vs-eager-fp32",
               bar=max(F32_BAR, 2 * eager_grad))


def test_f32_needs_f32_on_both_sides(gpu_available):
    from linearard_amd.attention_KL import attn_kl_align

    x = torch.zeros((1, 2, 8, 16), device="cuda")
    y = torch.zeros((1, 2, 8, 16), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="float32 on both sides"):
        attn_kl_align(x, x, y, y)
