"""GPU parity of the batched relation loss (the caller's loop of train.py:369-410).

The batched launches must give what the per-relation calls give: the same
kernels run, so the gradients match bitwise and the loss to the rounding of
its summation order.  One case is also checked against the oracle directly.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from tests._inputs import make_mask, mask_to_dev, randn, to_dev
from tests._tolerance import check_grad, check_loss

pytestmark = pytest.mark.gpu


def _pairs(rng, B, heads, T, D, dtype):
    """Student/teacher pairs, one per head count (teacher + noise, like the bench)."""
    out = []
    for H in heads:
        xt = randn(rng, (B, H, T, D), dtype)
        xs = O.round_to(xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32), dtype)
        out.append((xs, xt))
    return out


def _per_relation(pairs, weights, mask, dtype, a_s, a_t):
    """sum_r w_r attn_kl_align(x_s, x_s, x_t, x_t) with the single-relation path."""
    from linearard_amd.attention_KL import attn_kl_align

    xs = [to_dev(p[0], dtype, requires_grad=True) for p in pairs]
    xt = [to_dev(p[1], dtype) for p in pairs]
    total = None
    for r in range(len(pairs)):
        l = attn_kl_align(xs[r], xs[r], xt[r], xt[r], attn_mask=mask, causal=True, sm_scale_s=a_s, sm_scale_t=a_t)
        term = l * weights[r]
        total = term if total is None else total + term
    total.backward()
    return total.item(), [x.grad.clone() for x in xs]


def _batched(pairs, weights, mask, dtype, a_s, a_t):
    from linearard_amd.attention_KL import attn_kl_align_batched

    xs = [to_dev(p[0], dtype, requires_grad=True) for p in pairs]
    xt = [to_dev(p[1], dtype) for p in pairs]
    w = torch.tensor(weights, device=xs[0].device, dtype=torch.float32)
    loss = attn_kl_align_batched(xs, xt, w, attn_mask=mask, sm_scale_s=a_s, sm_scale_t=a_t)
    assert loss.dim() == 0 and loss.dtype == torch.float32
    loss.backward()
    return loss.item(), [x.grad.clone() for x in xs]


@pytest.mark.parametrize("dtype,B,heads,T,D,ratio", [
    ("bf16", 2, (4, 2, 2), 200, 128, 0.2),  # Q/Q next to K/K and V/V with fewer heads
    ("f16", 1, (2, 1, 3), 77, 64, None),
    ("bf16", 1, (1, 1, 1, 1, 1, 2, 2, 2, 2, 1, 3), 65, 32, None),  # 11 relations: two launches of up to 8
])
def test_batched_matches_per_relation_calls(gpu_available, dtype, B, heads, T, D, ratio):
    rng = np.random.default_rng(len(heads) * 1000 + T)
    pairs = _pairs(rng, B, heads, T, D, dtype)
    weights = [float(w) for w in rng.uniform(0.1, 2.0, len(heads))]
    mask = mask_to_dev(None if ratio is None else make_mask(rng, B, T, ratio))
    a = 1 / math.sqrt(D)
    lb, gb = _batched(pairs, weights, mask, dtype, a, a)
    lr, gr = _per_relation(pairs, weights, mask, dtype, a, a)
    assert abs(lb - lr) <= 1e-5 * abs(lr) + 1e-6, (lb, lr)
    for g1, g2 in zip(gb, gr):
        assert g1.dtype == g2.dtype
        assert torch.equal(g1, g2)  # same kernels, same epilogue: bitwise


def test_batched_against_the_oracle(gpu_available):
    rng = np.random.default_rng(3)
    dtype, B, T, D = "bf16", 1, 150, 128
    pairs = _pairs(rng, B, (2, 1), T, D, dtype)
    weights = [0.7, 1.9]
    a = 1 / math.sqrt(D)
    lb, gb = _batched(pairs, weights, None, dtype, a, a)
    ref = 0.0
    for r, (xs, xt) in enumerate(pairs):
        rl, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, None, True, a, a, dloss=weights[r], self_relation=True)
        ref += weights[r] * rl
        check_grad(gb[r].float().cpu().numpy(), rdx, f"batched-rel{r}")
    check_loss(lb, ref, "batched")


@pytest.mark.parametrize("D,a", [(256, None), (64, 3e-7)])
def test_batched_outside_the_kernels_falls_back(gpu_available, D, a):
    """D = 256 and a scale below 1e-6 are not taken by the batched kernels; the
    Function then runs relation by relation and must give the same values."""
    rng = np.random.default_rng(D)
    pairs = _pairs(rng, 1, (2, 1), 40, D, "bf16")
    weights = [1.3, 0.4]
    lb, gb = _batched(pairs, weights, None, "bf16", a, a)
    lr, gr = _per_relation(pairs, weights, None, "bf16", a, a)
    assert abs(lb - lr) <= 1e-5 * abs(lr) + 1e-6, (lb, lr)
    for g1, g2 in zip(gb, gr):
        assert torch.equal(g1, g2)


def test_relation_kl_loss_is_the_train_py_formula(gpu_available):
    """train.py:369-410: per layer Q/Q + K/K + V/V over denom (query heads),
    summed, over the layer count; with a padding mask (denom = mask.sum()*Hq)."""
    from linearard_amd.attention_KL import attn_kl_align, relation_kl_loss

    rng = np.random.default_rng(11)
    dtype, B, T, D, Hq, Hkv, layers = "bf16", 2, 96, 64, 4, 2, 3
    mask = mask_to_dev(make_mask(rng, B, T, 0.25))
    a = 1 / math.sqrt(D)
    raw = [[_pairs(rng, B, (H,), T, D, dtype)[0] for H in (Hq, Hkv, Hkv)] for _ in range(layers)]

    def dev_tensors():
        s = [[to_dev(p[0], dtype, requires_grad=True) for p in layer] for layer in raw]
        t = [[to_dev(p[1], dtype) for p in layer] for layer in raw]
        return s, t

    s, t = dev_tensors()
    loss = relation_kl_loss([l[0] for l in s], [l[1] for l in s], [l[2] for l in s],
                            [l[0] for l in t], [l[1] for l in t], [l[2] for l in t],
                            attn_mask=mask, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    got = [x.grad.clone() for layer in s for x in layer]

    s2, t2 = dev_tensors()  # the reference loop, literally
    Q = K = V = 0.0
    for li in range(layers):
        lq = attn_kl_align(s2[li][0], s2[li][0], t2[li][0], t2[li][0], attn_mask=mask, causal=True,
                           sm_scale_s=a, sm_scale_t=a)
        lk = attn_kl_align(s2[li][1], s2[li][1], t2[li][1], t2[li][1], attn_mask=mask, causal=True,
                           sm_scale_s=a, sm_scale_t=a)
        lv = attn_kl_align(s2[li][2], s2[li][2], t2[li][2], t2[li][2], attn_mask=mask, causal=True,
                           sm_scale_s=a, sm_scale_t=a)
        denom = mask.sum().clamp_min(1) * s2[li][0].shape[1]
        Q = Q + lq / denom
        K = K + lk / denom
        V = V + lv / denom
    ref = (Q + K + V) / max(1, layers)
    ref.backward()
    want = [x.grad.clone() for layer in s2 for x in layer]
    assert abs(loss.item() - ref.item()) <= 1e-5 * abs(ref.item()), (loss.item(), ref.item())
    for g1, g2 in zip(got, want):
        assert (g1.float() - g2.float()).abs().max() <= 1e-2 * g2.float().abs().max() + 1e-6


def test_batched_is_deterministic(gpu_available):
    rng = np.random.default_rng(5)
    pairs = _pairs(rng, 1, (3, 1, 1), 130, 128, "bf16")
    a = 1 / math.sqrt(128)
    l1, g1 = _batched(pairs, [1.0, 0.5, 0.25], None, "bf16", a, a)
    l2, g2 = _batched(pairs, [1.0, 0.5, 0.25], None, "bf16", a, a)
    assert l1 == l2
    for x, y in zip(g1, g2):
        assert torch.equal(x, y)


def test_batched_takes_the_hooks_strided_views(gpu_available):
    """train.py:133-142 copies the captured [B, T, H, D] projections with
    .contiguous(); the batched API reads the permuted views directly, with
    the same results bit for bit."""
    from linearard_amd.attention_KL import attn_kl_align_batched

    g = torch.Generator(device="cuda").manual_seed(2)
    bthd = [torch.randn((1, 96, H, 64), device="cuda", generator=g).to(torch.bfloat16) for H in (4, 2)]
    bthd_t = [(x.float() + 0.3 * torch.randn(x.shape, device="cuda", generator=g)).to(torch.bfloat16) for x in bthd]
    views = [x.permute(0, 2, 1, 3).detach().requires_grad_(True) for x in bthd]
    copies = [x.permute(0, 2, 1, 3).contiguous().detach().requires_grad_(True) for x in bthd]
    t_views = [x.permute(0, 2, 1, 3) for x in bthd_t]
    assert not views[0].is_contiguous()
    w = torch.tensor([0.5, 2.0], device="cuda")
    l1 = attn_kl_align_batched(views, t_views, w)
    l1.backward()
    l2 = attn_kl_align_batched(copies, [x.contiguous() for x in t_views], w)
    l2.backward()
    assert l1.item() == l2.item()
    for a, b in zip(views, copies):
        assert torch.equal(a.grad, b.grad)
