"""GPU parity of distillation_loss with the reference's loss lines
(train.py:360-423) written out literally over attn_kl_align and torch ops."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tests._inputs import make_mask, mask_to_dev

pytestmark = pytest.mark.gpu


def _layers(g, L, B, T, D, Hq, Hkv):
    def pair(H):
        t = torch.randn((B, H, T, D), device="cuda", generator=g).to(torch.bfloat16)
        s = (t.float() + 0.3 * torch.randn(t.shape, device="cuda", generator=g)).to(torch.bfloat16)
        return s, t
    return [[pair(Hq), pair(Hkv), pair(Hkv)] for _ in range(L)]


def _leaves(layers):
    s = [[p[0].clone().requires_grad_(True) for p in layer] for layer in layers]
    t = [[p[1] for p in layer] for layer in layers]
    return s, t


def _reference(s, t, t_logits, s_logits, mask, lam_A, lam_L, T, scale):
    """train.py:360-423 with this package's attn_kl_align for the relation KL
    and torch float32 for the logits lines (on the bf16-rounded x * (1/T)
    the reference's `t_logits / T` produces)."""
    from linearard_amd.attention_KL import attn_kl_align

    Q = K = V = 0.0
    L = len(s)
    for l in range(L):
        (qs, ks, vs), (qt, kt, vt) = s[l], t[l]
        lq = attn_kl_align(qs, qs, qt, qt, attn_mask=mask, causal=True, sm_scale_s=scale, sm_scale_t=scale)
        lk = attn_kl_align(ks, ks, kt, kt, attn_mask=mask, causal=True, sm_scale_s=scale, sm_scale_t=scale)
        lv = attn_kl_align(vs, vs, vt, vt, attn_mask=mask, causal=True, sm_scale_s=scale, sm_scale_t=scale)
        if mask is None:
            denom = qs.shape[0] * qs.shape[1] * qs.shape[2]
        else:
            denom = mask.sum().clamp_min(1) * qs.shape[1]
        Q = Q + lq / denom
        K = K + lk / denom
        V = V + lv / denom
    attn = (Q + K + V) / max(1, L)
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(T, dtype=torch.float32)
    # s_logits may be a float32 copy (for a float32 gradient): the value is
    # rounded as the bf16 tensor op rounds it, the gradient passes in float32
    # (a .to(bfloat16) in the graph would round the gradient to bf16 as well)
    def scaled(x):
        y = x.float() * inv.item()
        return y + (y.to(torch.bfloat16).float() - y).detach()

    qt_ = scaled(t_logits)
    qs_ = scaled(s_logits)
    t_logp = F.log_softmax(qt_, dim=-1)
    s_logp = F.log_softmax(qs_, dim=-1)
    logits = (t_logp.exp() * (t_logp - s_logp)).sum(dim=-1).mean()
    # float32 rounding scales of the logits KL (KL = E[q_t - q_s] - lse_t + lse_s)
    # and of its gradient c (p_s - p_t) per element
    lscale = (1 + torch.logsumexp(qt_, -1).abs() + torch.logsumexp(qs_, -1).abs()
              + (t_logp.exp() * (qt_ - qs_).abs()).sum(-1)).mean().item()
    kl_rows = (t_logp.exp() * (t_logp - s_logp)).sum(-1, keepdim=True)
    c = lam_L / (t_logits.shape[0] * t_logits.shape[1]) * inv.item()
    gscale = (c * (t_logp.exp() + s_logp.exp()) * (1 + t_logp.abs() + s_logp.abs() + kl_rows.abs())).detach()
    return (lam_A * attn + lam_L * logits, attn, logits, Q, K, V), lscale, gscale


@pytest.mark.parametrize("ratio,lam_L,T", [(0.2, 0.3, 1.5), (None, 0.5, 1.0)])
def test_distillation_loss_is_the_train_py_loss(gpu_available, ratio, lam_L, T):
    from linearard_amd.distill import distillation_loss

    g = torch.Generator(device="cuda").manual_seed(7)
    L, B, Tn, D, Hq, Hkv = 3, 2, 96, 64, 4, 2
    layers = _layers(g, L, B, Tn, D, Hq, Hkv)
    mask = mask_to_dev(None if ratio is None else make_mask(np.random.default_rng(1), B, Tn, ratio))
    t_logits = (3 * torch.randn((B, 8, 1000), device="cuda", generator=g)).to(torch.bfloat16)
    s_logits0 = (t_logits.float() + torch.randn(t_logits.shape, device="cuda", generator=g)).to(torch.bfloat16)
    scale = 1 / math.sqrt(D)

    s1, t1 = _leaves(layers)
    sl1 = s_logits0.clone().requires_grad_(True)
    out = distillation_loss([x[0] for x in s1], [x[1] for x in s1], [x[2] for x in s1],
                            [x[0] for x in t1], [x[1] for x in t1], [x[2] for x in t1],
                            t_logits, sl1, attn_mask=mask, lam_A=0.7, lam_L=lam_L, temperature=T)
    out.loss.backward()

    s2, t2 = _leaves(layers)
    sl2 = s_logits0.float().clone().requires_grad_(True)
    ref, lscale, gscale = _reference(s2, t2, t_logits, sl2, mask, 0.7, lam_L, T, scale)
    ref[0].backward()

    # attention terms: the same kernels, summed in another order (relative 2e-5);
    # the logits term: float32 against float32 (2e-5 of its rounding scale)
    tol_attn = 2e-5 * abs(float(ref[1])) + 1e-8
    tol_logits = 2e-5 * lscale
    tols = [0.7 * tol_attn + lam_L * tol_logits, tol_attn, tol_logits] + [2e-5 * abs(float(x)) + 1e-8 for x in ref[3:]]
    for name, got, want, tol in zip(out._fields, out, ref, tols):
        assert abs(float(got) - float(want)) <= tol, (name, float(got), float(want), tol)
    for a, b in zip([x for layer in s1 for x in layer], [x for layer in s2 for x in layer]):
        err = (a.grad.float() - b.grad.float()).abs().max().item()
        assert err <= 4e-3 * b.grad.float().abs().max().item() + 1e-9  # same kernels; the bf16 cast may flip
    # the logits gradient: bf16 output against torch's float32 autograd
    want = sl2.grad
    err = (sl1.grad.float() - want).abs()
    # both sides carry float32 errors of that scale (torch's float32 log_softmax too): 2e-5
    bound = 2.0 ** -8 * want.abs() + 2e-5 * gscale + 1e-30
    assert bool((err <= bound).all()), float((err / bound).max())


def test_lam_L_zero_logs_the_logits_kl_without_a_gradient_pass(gpu_available):
    from linearard_amd.distill import distillation_loss
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(8)
    layers = _layers(g, 2, 1, 64, 32, 2, 1)
    s, t = _leaves(layers)
    t_logits = torch.randn((1, 4, 512), device="cuda", generator=g).to(torch.bfloat16)
    s_logits = torch.randn((1, 4, 512), device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    out = distillation_loss([x[0] for x in s], [x[1] for x in s], [x[2] for x in s],
                            [x[0] for x in t], [x[1] for x in t], [x[2] for x in t], t_logits, s_logits)
    out.loss.backward()
    assert s_logits.grad is None
    assert float(out.loss) == float(out.attn_loss)
    assert float(out.logits_loss) == float(logits_kl(t_logits, s_logits.detach()))
    assert all(x.grad is not None for layer in s for x in layer)
    none = distillation_loss([x[0] for x in s], [x[1] for x in s], [x[2] for x in s],
                             [x[0] for x in t], [x[1] for x in t], [x[2] for x in t])
    assert none.logits_loss is None and float(none.loss) == float(out.attn_loss)
