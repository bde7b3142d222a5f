"""Parity at the BASELINE configurations' own shapes and inputs (cfg2, cfg3,
cfg4, cfg5), drawn by bench.config_relations -- the same inputs the
benchmark times.

Each relation launch covers every head of the configuration; one or two
full-length heads per relation kind are checked against the chunked CPU
oracle (oracle.attn_kl.self_relation_chunked, following kernel_A.py:72-159,
kernel_B.py:105-218 and kernel_C.py:121-261; float64 where the logits are
large), with the parity bar stated once here:

    loss:     |got - ref| <= 1e-3 |ref|                 (BASELINE, bf16)
    gradient: max |got - ref| <= 2e-2 max |ref|         (BASELINE, bf16)

and the other heads by properties that hold at any size: a head's gradient
in the full launch equals, bitwise, a launch of that head alone; the
launch's loss is the sum of the per-head losses; identical relations (the
unrotated V/V of cfg2 and cfg3) give exactly zero.
"""

import math

import numpy as np
import pytest
import torch

import bench
from oracle import attn_kl as O
from tests._tolerance import check_grad, check_loss

pytestmark = pytest.mark.gpu

LOSS_RTOL = 1e-3
GRAD_RTOL = 2e-2


def _fwd_bwd(xs, xt, a, mask=None):
    from linearard_amd.attention_KL import attn_kl_align

    x = xs.detach().clone().requires_grad_(True)
    loss = attn_kl_align(x, x, xt, xt, attn_mask=mask, causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    return loss.detach(), x.grad


def _check_head(name, xs, xt, b, h, a, loss_h, grad_h, dtype, chunk=1024, mask_b=None):
    x_s = xs[b, h].float().cpu().numpy()
    x_t = xt[b, h].float().cpu().numpy()
    ref_loss, ref_dx, _, _, kl_rows = O.self_relation_chunked(x_s, x_t, True, a, a, mask=mask_b, chunk=chunk,
                                                              dtype=dtype)
    assert kl_rows.min() >= -1e-6, kl_rows.min()  # KL >= 0 per row
    case = f"{name}-b{b}h{h}"
    check_loss(loss_h, ref_loss, case, bar=LOSS_RTOL)
    check_grad(grad_h.float().cpu().numpy(), ref_dx, case, bar=GRAD_RTOL)


def _relation(name, xs, xt, a, heads, mask=None, dtype=np.float32):
    """The whole relation in one launch; `heads` = [(b, h)] checked against
    the oracle through single-head launches whose gradients must equal the
    full launch's bitwise."""
    loss, dx = _fwd_bwd(xs, xt, a, mask)
    assert torch.isfinite(loss) and bool(torch.isfinite(dx).all())
    total = 0.0
    B, H = xs.shape[:2]
    for b in range(B):
        for h in range(H):
            m = None if mask is None else mask[b:b + 1]
            lh, dh = _fwd_bwd(xs[b:b + 1, h:h + 1].contiguous(), xt[b:b + 1, h:h + 1].contiguous(), a, m)
            assert torch.equal(dh, dx[b:b + 1, h:h + 1]), f"head ({b}, {h}): gradient differs from the full launch"
            total += lh.double().item()
            if (b, h) in heads:
                mb = None if mask is None else mask[b].cpu().numpy()
                _check_head(name, xs, xt, b, h, a, lh.double().item(), dh[0, 0], dtype, mask_b=mb)
    assert abs(loss.double().item() - total) <= 1e-5 * abs(total), (loss.item(), total)
    return loss


def test_cfg2_true_outliers_against_the_oracle(gpu_available):
    """cfg2: B=1, H=32, n=4096, d=128, bf16; pre-RoPE N(0,1) with 4 channels
    x20 (diagonal logits ~150: the large-logit regime), teacher RoPE base 1e4
    at p, student p/8.  Q/Q heads 0 and 31 and K/K head 7 against the
    float64 oracle; V/V of the unrotated vectors exactly zero."""
    rel = bench.config_relations("cfg2", seed=2)
    a = 1 / math.sqrt(128)
    xs, xt = rel["q"]
    x0 = xt[0, 0].float()
    assert float((a * (x0 * x0).sum(-1)).max()) > 100.0  # really the large-logit regime
    _relation("cfg2-q", xs, xt, a, heads={(0, 0), (0, 31)}, dtype=np.float64)
    xs, xt = rel["k"]
    _relation("cfg2-k", xs, xt, a, heads={(0, 7)}, dtype=np.float64)
    v, _ = rel["v"]
    lv, dv = _fwd_bwd(v, v, a)
    assert lv.item() == 0.0 and not bool(dv.any())


def test_cfg3_own_inputs_against_the_oracle(gpu_available):
    """cfg3: n=8192, d=128, bf16; Q/Q 32 heads, K/K 8; per-head std U(0.5, 2);
    teacher RoPE base 5e5, NTK student base x8 (the producer's student_base).
    Q/Q head 5 and K/K head 3 against the oracle; the batched relation loss
    (train.py:369-410) on these inputs equals the per-call loop."""
    from linearard_amd.attention_KL import attn_kl_align, relation_kl_loss

    rel = bench.config_relations("cfg3", seed=3)
    a = 1 / math.sqrt(128)
    _relation("cfg3-q", *rel["q"], a, heads={(0, 5)})
    _relation("cfg3-k", *rel["k"], a, heads={(0, 3)})
    v, _ = rel["v"]
    lv, dv = _fwd_bwd(v, v, a)
    assert lv.item() == 0.0 and not bool(dv.any())

    s1 = [rel[k][0].detach().clone().requires_grad_(True) for k in "qkv"]
    t = [rel[k][1] for k in "qkv"]
    loss = relation_kl_loss([s1[0]], [s1[1]], [s1[2]], [t[0]], [t[1]], [t[2]], sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    s2 = [rel[k][0].detach().clone().requires_grad_(True) for k in "qkv"]
    denom = 1 * 32 * 8192  # train.py:404, the layer's query heads for all three
    ref = sum(attn_kl_align(s2[j], s2[j], t[j], t[j], causal=True, sm_scale_s=a, sm_scale_t=a) / denom
              for j in range(3))
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-5 * abs(ref.item()), (loss.item(), ref.item())
    for x1, x2 in zip(s1, s2):
        g1, g2 = x1.grad.float(), x2.grad.float()
        assert (g1 - g2).abs().max() <= 1e-2 * g2.abs().max() + 1e-9


def test_cfg4_bench_inputs_against_the_oracle(gpu_available):
    """cfg4 as the benchmark times it: B=1, H=32, n=32768, d=128, bf16,
    pre-RoPE N(0,1), teacher RoPE at p, student at p/8; head 0 against the
    chunked float32 oracle, every head by head independence."""
    rel = bench.config_relations("cfg4")
    _relation("cfg4-q", *rel["q"], 1 / math.sqrt(128), heads={(0, 0)})


def test_cfg5_layer_against_the_oracle(gpu_available):
    """cfg5, one layer: B=2, n=16384, d=128, bf16, all-ones int64 mask (the
    HAS_MASK path of train.py's PG19 blocks); Q/Q 32 heads, K/K and V/V 8;
    8 Student-t(3) channels; RoPE base 1e4, student p/4.  One head of each
    kind against the oracle (both sequences of the batch covered), the rest
    by head independence; the batched relation loss equals the per-call
    loop."""
    from linearard_amd.attention_KL import attn_kl_align, relation_kl_loss

    rel = bench.config_relations("cfg5", seed=5)
    a = 1 / math.sqrt(128)
    mask = rel["mask"]
    assert mask.dtype == torch.int64 and bool((mask == 1).all())
    # float64 oracle: the Student-t channels give large logits, where a float32
    # oracle's own per-row KL already goes negative by ~1e-6
    _relation("cfg5-q", *rel["q"], a, heads={(0, 11)}, mask=mask, dtype=np.float64)
    _relation("cfg5-k", *rel["k"], a, heads={(1, 2)}, mask=mask, dtype=np.float64)
    _relation("cfg5-v", *rel["v"], a, heads={(0, 6)}, mask=mask, dtype=np.float64)

    s1 = [rel[k][0].detach().clone().requires_grad_(True) for k in "qkv"]
    t = [rel[k][1] for k in "qkv"]
    loss = relation_kl_loss([s1[0]], [s1[1]], [s1[2]], [t[0]], [t[1]], [t[2]], attn_mask=mask, sm_scale_s=a,
                            sm_scale_t=a)
    loss.backward()
    s2 = [rel[k][0].detach().clone().requires_grad_(True) for k in "qkv"]
    denom = float(mask.sum()) * 32  # train.py:405-406: mask.sum() * the layer's query heads
    ref = sum(attn_kl_align(s2[j], s2[j], t[j], t[j], attn_mask=mask, causal=True, sm_scale_s=a, sm_scale_t=a) /
              denom for j in range(3))
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-5 * abs(ref.item()), (loss.item(), ref.item())
    for x1, x2 in zip(s1, s2):
        g1, g2 = x1.grad.float(), x2.grad.float()
        assert (g1 - g2).abs().max() <= 1e-2 * g2.abs().max() + 1e-9
