"""Size-independent properties at cfg4's size and at n = 131072.

(The BASELINE configurations' own inputs are checked against the oracle in
tests/test_gpu_configs.py.)  Here:

* identical relations (x_s == x_t, equal scales) give a loss and a gradient
  of exactly zero at cfg4's size (P_s == P_t element for element);
* at n = 131072 (4x cfg4) one head's LSEs match the chunked oracle on the
  first rows and scipy on the last, the batched API reads the head in place
  from a [B, T, H, D] tensor with the same result as the contiguous copy,
  and identical relations give exactly zero;
* a real padding mask at n = 16384 (a padded tail and random holes) against
  the oracle, with exactly zero gradient on the masked tokens.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O


pytestmark = pytest.mark.gpu


def _pair(B, H, n, d, seed, noise=0.1):
    """bf16 teacher x_t ~ N(0,1), student x_t + noise (drawn on the device from
    one seeded generator, in a fixed order)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    xt = torch.randn((B, H, n, d), device="cuda", generator=g)
    xs = xt + noise * torch.randn((B, H, n, d), device="cuda", generator=g)
    return xs.to(torch.bfloat16), xt.to(torch.bfloat16)


def _fwd_bwd(xs, xt, a):
    from linearard_amd.attention_KL import attn_kl_align

    x = xs.detach().clone().requires_grad_(True)
    loss = attn_kl_align(x, x, xt, xt, causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    return loss.detach(), x.grad


def test_cfg4_identical_relations_are_exactly_zero(gpu_available):
    B, H, n, d = 1, 32, 32768, 128
    a = 1 / math.sqrt(d)
    _, xt = _pair(B, H, n, d, seed=5)
    loss, dx = _fwd_bwd(xt.clone(), xt, a)
    assert loss.item() == 0.0
    assert not bool(dx.any())


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


def test_padding_mask_at_16k_against_the_oracle(gpu_available):
    """A real padding mask at cfg5's sequence length (B=2, H=4, n=16384,
    d=128, bf16, causal): sequence 0 ends in 2500 padded tokens, sequence 1
    has 10 % random holes (token 0 kept).  Masked rows and columns take the
    kernels' token-validity paths on every tile; heads (0, 1) and (1, 3)
    against the chunked float32 oracle (kernel_A.py:91-120 masking,
    kernel_C.py:252-256 zero rows and columns), the rest by head
    independence, and masked tokens get exactly zero gradient."""
    from tests.test_gpu_configs import _relation

    B, H, n, d = 2, 4, 16384, 128
    a = 1 / math.sqrt(d)
    xs, xt = _pair(B, H, n, d, seed=16, noise=0.3)
    rng = np.random.default_rng(16)
    mask = np.ones((B, n), dtype=np.int32)
    mask[0, n - 2500:] = 0
    mask[1] = rng.random(n) > 0.1
    mask[1, 0] = 1
    m = torch.tensor(mask, device="cuda")
    _relation("pad16k", xs, xt, a, heads={(0, 1), (1, 3)}, mask=m)
    _, dx = _fwd_bwd_masked(xs, xt, a, m)
    assert not bool(dx[0, :, n - 2500:].any())
    assert not bool(dx[1][:, torch.tensor(mask[1] == 0, device="cuda")].any())


def _fwd_bwd_masked(xs, xt, a, mask):
    from linearard_amd.attention_KL import attn_kl_align

    x = xs.detach().clone().requires_grad_(True)
    loss = attn_kl_align(x, x, xt, xt, attn_mask=mask, causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    return loss.detach(), x.grad
