"""Parity at the BASELINE configurations' full sizes (cfg2, cfg3, cfg4 shapes)
and at n = 131072.

At these sizes the oracle cannot check every head within seconds.  So each
test checks one full-length head against the chunked CPU oracle
(oracle.attn_kl.self_relation_chunked, which follows kernel_A.py:72-159,
kernel_B.py:105-218 and kernel_C.py:121-261). It also checks properties that
hold at any size:

* heads are independent: every head's gradient in the H = 32 launch equals,
  bitwise, a launch of that head alone (no cross-head reduction, no
  atomics), and the loss of the launch is the sum of the per-head losses (to
  float32 summation order);
* identical relations (x_s == x_t, equal scales) give a loss and a gradient
  of exactly zero (P_s == P_t element for element);
* a V/V relation of unrotated vectors is such a pair (cfg2's free exact check);
* the batched relation loss of train.py:369-410 at cfg3's shapes equals the
  per-call loop (loss to float32 summation order; gradients to the rounding
  of the 1/denom weights, which the batched kernels apply in their epilogue).
"""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from tests._tolerance import _grad_ok, _logit_bound, _loss_ok

pytestmark = pytest.mark.gpu


def _pair(B, H, n, d, seed, noise=0.1, outliers=4):
    """bf16 teacher x_t ~ N(0,1) with a few large channels, student x_t + noise
    (drawn on the device from one seeded generator, in a fixed order)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    xt = torch.randn((B, H, n, d), device="cuda", generator=g)
    if outliers:
        idx = torch.randperm(d, device="cuda", generator=g)[:outliers]
        xt[..., idx] *= 20.0 / math.sqrt(d)
    xs = xt + noise * torch.randn((B, H, n, d), device="cuda", generator=g)
    return xs.to(torch.bfloat16), xt.to(torch.bfloat16)


def _fwd_bwd(xs, xt, a):
    from linearard_amd.attention_KL import attn_kl_align

    x = xs.detach().clone().requires_grad_(True)
    loss = attn_kl_align(x, x, xt, xt, causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    return loss.detach(), x.grad


def test_cfg4_heads_independent_and_one_head_matches_the_oracle(gpu_available):
    """cfg4: B=1, H=32, n=32768, d=128, bf16, causal self relation."""
    B, H, n, d = 1, 32, 32768, 128
    a = 1 / math.sqrt(d)
    xs, xt = _pair(B, H, n, d, seed=4)
    loss, dx = _fwd_bwd(xs, xt, a)
    assert torch.isfinite(loss) and bool(torch.isfinite(dx).all())

    per_head = []
    for h in range(H):
        lh, dh = _fwd_bwd(xs[:, h:h + 1].contiguous(), xt[:, h:h + 1].contiguous(), a)
        assert lh.item() >= 0.0
        assert torch.equal(dh, dx[:, h:h + 1]), f"head {h}: gradient differs from the H=32 launch"
        per_head.append(lh.double().item())
    total = sum(per_head)
    assert abs(loss.double().item() - total) <= 1e-5 * total, (loss.item(), total)

    h = 0  # one full-length head against the oracle (float32, 1024-row chunks)
    x_s = xs[0, h].float().cpu().numpy()
    x_t = xt[0, h].float().cpu().numpy()
    ref_loss, ref_dx, _, _, kl_rows = O.self_relation_chunked(x_s, x_t, True, a, a, chunk=1024, dtype=np.float32)
    assert kl_rows.min() >= -1e-6  # KL >= 0 per row
    logit = _logit_bound((x_s, x_s, a), (x_t, x_t, a))
    assert _loss_ok(per_head[h], ref_loss, n, logit), (per_head[h], ref_loss)
    got = dx[0, h].float().cpu().numpy()
    assert _grad_ok(got, ref_dx, x_s, a, logit), np.abs(got - ref_dx).max() / np.abs(ref_dx).max()


def test_cfg4_identical_relations_are_exactly_zero(gpu_available):
    B, H, n, d = 1, 32, 32768, 128
    a = 1 / math.sqrt(d)
    _, xt = _pair(B, H, n, d, seed=5)
    loss, dx = _fwd_bwd(xt.clone(), xt, a)
    assert loss.item() == 0.0
    assert not bool(dx.any())


def test_cfg2_rope_pairs_and_unrotated_values(gpu_available):
    """cfg2: B=1, H=32, n=4096, d=128, bf16; teacher RoPE base 1e4 at p,
    student at p/8 (linear scaling 8), both from the RoPE pair producer; the
    V/V relation of the unrotated vectors is exactly zero."""
    from linearard_amd.rope import rope_pair

    B, H, n, d = 1, 32, 4096, 128
    a = 1 / math.sqrt(d)
    g = torch.Generator(device="cuda").manual_seed(2)
    v = torch.randn((B, H, n, d), device="cuda", generator=g)
    idx = torch.randperm(d, device="cuda", generator=g)[:4]
    v[..., idx] *= 20.0 / math.sqrt(d)
    v = v.to(torch.bfloat16)
    q_s, q_t = rope_pair(v, 10000.0, {"rope_type": "linear", "factor": 8.0})
    loss, dx = _fwd_bwd(q_s, q_t, a)
    assert loss.item() > 0.0
    for h in (0, H - 1):
        lh, dh = _fwd_bwd(q_s[:, h:h + 1].contiguous(), q_t[:, h:h + 1].contiguous(), a)
        assert torch.equal(dh, dx[:, h:h + 1])
        x_s = q_s[0, h].float().cpu().numpy()
        x_t = q_t[0, h].float().cpu().numpy()
        ref_loss, ref_dx, _, _, _ = O.self_relation_chunked(x_s, x_t, True, a, a, chunk=512, dtype=np.float32)
        logit = _logit_bound((x_s, x_s, a), (x_t, x_t, a))
        assert _loss_ok(lh.item(), ref_loss, n, logit), (h, lh.item(), ref_loss)
        got = dh[0, 0].float().cpu().numpy()
        assert _grad_ok(got, ref_dx, x_s, a, logit), (h, np.abs(got - ref_dx).max() / np.abs(ref_dx).max())
    lv, dv = _fwd_bwd(v, v, a)
    assert lv.item() == 0.0 and not bool(dv.any())


def test_cfg3_batched_relation_loss_equals_the_loop(gpu_available):
    """cfg3 shapes: Q/Q 32 heads, K/K and V/V 8 heads, n=8192, d=128, bf16,
    two layers; relation_kl_loss against train.py:369-410's loop of
    attn_kl_align calls."""
    from linearard_amd.attention_KL import attn_kl_align, relation_kl_loss

    B, n, d, layers = 1, 8192, 128, 2
    a = 1 / math.sqrt(d)
    raw = [[_pair(B, H, n, d, seed=30 + 3 * li + k, noise=0.3) for k, H in enumerate((32, 8, 8))]
           for li in range(layers)]

    def student():
        return [[p[0].clone().requires_grad_(True) for p in layer] for layer in raw]

    s = student()
    t = [[p[1] for p in layer] for layer in raw]
    loss = relation_kl_loss([l[0] for l in s], [l[1] for l in s], [l[2] for l in s],
                            [l[0] for l in t], [l[1] for l in t], [l[2] for l in t], sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    s2 = student()
    ref = 0.0
    for li in range(layers):
        denom = B * s2[li][0].shape[1] * n  # train.py:404, the layer's query heads for all three
        for k in range(3):
            ref = ref + attn_kl_align(s2[li][k], s2[li][k], t[li][k], t[li][k], causal=True,
                                      sm_scale_s=a, sm_scale_t=a) / denom
    ref = ref / layers
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-5 * abs(ref.item()), (loss.item(), ref.item())
    for l1, l2 in zip(s, s2):
        for x1, x2 in zip(l1, l2):
            g1, g2 = x1.grad.float(), x2.grad.float()
            assert (g1 - g2).abs().max() <= 1e-2 * g2.abs().max() + 1e-6


def test_long_context_128k_and_the_strided_view(gpu_available):
    """n = 131072 (4x cfg4), one head.  It checks:
    - loss and gradient are finite, and the loss is positive;
    - the student LSE of the first 2048 rows equals the chunked oracle's, and
      the last row's equals scipy's logsumexp;
    - the same head read by the batched API through the permuted view of a
      [B, T, H, D] tensor (row stride H*d) gives the same loss and gradient;
    - identical relations give exactly 0."""
    from scipy.special import logsumexp

    from linearard_amd.attention_KL import attn_kl_align, attn_kl_align_batched, lse_stats

    B, H, n, d = 1, 4, 131072, 128
    a = 1 / math.sqrt(d)
    g = torch.Generator(device="cuda").manual_seed(7)
    raw_t = torch.randn((B, n, H, d), device="cuda", generator=g)
    raw_s = raw_t + 0.1 * torch.randn((B, n, H, d), device="cuda", generator=g)
    bt, bs = raw_t.to(torch.bfloat16), raw_s.to(torch.bfloat16)
    del raw_t, raw_s
    xt = bt.permute(0, 2, 1, 3)[:, 1:2].contiguous()  # head 1: [1, 1, n, d]
    xs = bs.permute(0, 2, 1, 3)[:, 1:2].contiguous().requires_grad_(True)
    loss = attn_kl_align(xs, xs, xt, xt, causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    assert math.isfinite(loss.item()) and loss.item() > 0.0
    assert bool(torch.isfinite(xs.grad).all())

    base = bs.detach().clone().requires_grad_(True)  # the hook's [B, T, H, D] layout, read in place
    w = torch.ones(1, device="cuda", dtype=torch.float32)
    lb = attn_kl_align_batched([base.permute(0, 2, 1, 3)[:, 1:2]], [bt.permute(0, 2, 1, 3)[:, 1:2]], w,
                               causal=True, sm_scale_s=a, sm_scale_t=a)
    lb.backward()
    assert abs(lb.item() - loss.item()) <= 1e-6 * loss.item(), (lb.item(), loss.item())
    gb = base.grad.permute(0, 2, 1, 3)[:, 1:2].float()
    assert (gb - xs.grad.float()).abs().max() <= 1e-2 * xs.grad.float().abs().max()
    assert not bool(base.grad[:, :, 0].any())  # the other heads get no gradient

    lse = lse_stats(xs.detach(), xs.detach(), causal=True, sm_scale=a)[0, 0].double().cpu().numpy()
    x_s = xs.detach()[0, 0].float().cpu().numpy()
    x_t = xt[0, 0].float().cpu().numpy()
    _, _, ref_lse, _, ref_kl = O.self_relation_chunked(x_s, x_t, True, a, a, chunk=512, dtype=np.float64,
                                                       want_grad=False, rows_subset=2048)
    assert np.abs(lse[:2048] - ref_lse[:2048]).max() <= 1e-4
    assert ref_kl[:2048].min() >= -1e-9
    last = logsumexp(a * (x_s.astype(np.float64) @ x_s[-1].astype(np.float64)))
    assert abs(lse[-1] - last) <= 1e-4 * max(1.0, abs(last)), (lse[-1], last)

    same = xt.clone().requires_grad_(True)
    z = attn_kl_align(same, same, xt, xt, causal=True, sm_scale_s=a, sm_scale_t=a)
    z.backward()
    assert z.item() == 0.0 and not bool(same.grad.any())
