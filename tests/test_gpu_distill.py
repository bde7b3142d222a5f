"""GPU parity of distillation_loss (train.py:360-423) against the CPU oracles.

The relation terms come from oracle.attn_kl (float64: attn_kl_align for the
small case, the chunked self-relation restatement at cfg5's length), the
logits term from oracle.logits_kl; the bars are the north star's
(tests/_tolerance.py).  At cfg5's launch shape (8 relations of each kind per
batched launch, B=2, n=16384) one head per relation is checked against the
oracle and the others through properties that hold at any size: a head's
gradient in the full step equals a launch of that head alone, and the
losses are sums over relations and heads.
"""

import math

import numpy as np
import pytest
import torch

import bench
from oracle import attn_kl as O
from oracle import logits_kl as OL
from tests._inputs import make_mask, mask_to_dev
from tests._oracle_pool import oracle_heads
from tests._tolerance import _rel, check_grad, check_loss

pytestmark = pytest.mark.gpu


def _layers(g, L, B, T, D, Hq, Hkv):
    def pair(H):
        t = torch.randn((B, H, T, D), device="cuda", generator=g).to(torch.bfloat16)
        s = (t.float() + 0.3 * torch.randn(t.shape, device="cuda", generator=g)).to(torch.bfloat16)
        return s, t
    return [[pair(Hq), pair(Hkv), pair(Hkv)] for _ in range(L)]


def _np(x):
    return x.detach().float().cpu().numpy()


def _oracle_step(layers, t_logits, s_logits, mask, lam_A, lam_L, T, scale):
    """train.py:360-423 on the CPU: the relation KLs and their gradients from
    oracle.attn_kl (float64), the logits KL from oracle.logits_kl.
    Returns (loss, attn, logits, Q, K, V) and the gradients of the student
    projections ([layer][q, k, v]) and of s_logits."""
    L = len(layers)
    sums = [0.0, 0.0, 0.0]
    grads = []
    for layer in layers:
        B, Hq, Tn, _ = layer[0][0].shape
        denom = B * Hq * Tn if mask is None else max(int(mask.sum()), 1) * Hq  # train.py:403-406
        g_layer = []
        for j, (xs, xt) in enumerate(layer):
            loss, dx, _, _, _ = O.attn_kl_align(_np(xs), _np(xs), _np(xt), _np(xt), mask, True, scale, scale,
                                                self_relation=True)
            sums[j] += loss / denom
            g_layer.append(dx * (lam_A / max(1, L) / denom))
        grads.append(g_layer)
    attn = sum(sums) / max(1, L)
    logits, _, _, _ = OL.logits_kl(_np(t_logits), _np(s_logits), T, "bf16")
    _, g_logits = OL.logits_kl_grads(_np(t_logits), _np(s_logits), T, "bf16", dloss=lam_L)
    return (lam_A * attn + lam_L * logits, attn, logits, *sums), grads, g_logits


@pytest.mark.parametrize("ratio,lam_L,T", [(0.2, 0.3, 1.5), (None, 0.5, 1.0)])
def test_distillation_loss_against_the_oracle(gpu_available, ratio, lam_L, T):
    """Three layers (Q/Q 4 heads, K/K and V/V 2, n=96, d=64) and a [2, 8, 1000]
    logits pair: every returned loss and every student gradient against the
    float64 oracles."""
    from linearard_amd.distill import distillation_loss

    g = torch.Generator(device="cuda").manual_seed(7)
    L, B, Tn, D, Hq, Hkv = 3, 2, 96, 64, 4, 2
    layers = _layers(g, L, B, Tn, D, Hq, Hkv)
    mask_np = None if ratio is None else make_mask(np.random.default_rng(1), B, Tn, ratio)
    mask = mask_to_dev(mask_np)
    t_logits = (3 * torch.randn((B, 8, 1000), device="cuda", generator=g)).to(torch.bfloat16)
    s_logits = (t_logits.float() + torch.randn(t_logits.shape, device="cuda", generator=g)).to(torch.bfloat16)
    scale = 1 / math.sqrt(D)

    s = [[p[0].clone().requires_grad_(True) for p in layer] for layer in layers]
    t = [[p[1] for p in layer] for layer in layers]
    sl = s_logits.clone().requires_grad_(True)
    out = distillation_loss([x[0] for x in s], [x[1] for x in s], [x[2] for x in s],
                            [x[0] for x in t], [x[1] for x in t], [x[2] for x in t],
                            t_logits, sl, attn_mask=mask, lam_A=0.7, lam_L=lam_L, temperature=T)
    out.loss.backward()

    ref, ref_grads, ref_gl = _oracle_step(layers, t_logits, s_logits, mask_np, 0.7, lam_L, T, scale)
    case = f"distill-L3-r{ratio}-T{T}"
    for name, got, want in zip(out._fields, out, ref):
        check_loss(float(got), want, f"{case}-{name}")
    for l in range(L):
        for j, kind in enumerate("qkv"):
            check_grad(_np(s[l][j].grad), ref_grads[l][j], f"{case}-layer{l}", f"d{kind}")
    check_grad(_np(sl.grad), ref_gl, case, "dlogit")


def test_lam_L_zero_logs_the_logits_kl_without_a_gradient_pass(gpu_available):
    from linearard_amd.distill import distillation_loss
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(8)
    layers = _layers(g, 2, 1, 64, 32, 2, 1)
    s = [[p[0].clone().requires_grad_(True) for p in layer] for layer in layers]
    t = [[p[1] for p in layer] for layer in layers]
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


# ---------------------------------------------------------------------------
# cfg5's launch shape
# ---------------------------------------------------------------------------

def test_distillation_step_at_the_cfg5_launch_shape(gpu_available):
    """Eight cfg5 layers (B=2, n=16384, d=128, bf16; Q/Q 32 heads, K/K and V/V
    8; all-ones int64 mask; Student-t(3) channels; RoPE base 1e4, student
    p/4): each kind is one batched launch of 8 relations, the launch shape of
    the 32-layer cfg5 step (4 launches of 8 per kind).

    * one head of every Q/Q relation (both sequences), one K/K and one V/V
      head against the float64 chunked oracle: the head's loss (a launch of
      that head alone) and its gradient inside the full step;
    * every Q/Q head: its gradient in the full step equals, bitwise, a
      fwd+bwd launch of that head alone with the step's upstream gradient,
      and its single-head losses sum to the relation's loss;
    * Q_loss, K_loss, V_loss are the per-relation launches' losses over the
      denominator (train.py:403-410), attn their mean.
    """
    from linearard_amd.attention_KL import attn_kl_align
    from linearard_amd.distill import distillation_loss

    L, B, n, Hq = 8, 2, 16384, 32
    a = 1 / math.sqrt(128)
    rels = [bench.config_relations("cfg5", seed=500 + l, device_rng=True) for l in range(L)]
    mask = rels[0]["mask"]
    s = {k: [r[k][0].detach().clone().requires_grad_(True) for r in rels] for k in "qkv"}
    t = {k: [r[k][1] for r in rels] for k in "qkv"}
    del rels
    # bf16 values below 2^15 are float16 values: the kernels' float16 keys
    # then need no scaling, per relation or per head alike
    assert max(float(x.detach().abs().max()) for k in "qkv" for x in s[k] + t[k]) < 2.0 ** 15

    print("cfg5 launch shape: distillation_loss over 8 layers", flush=True)
    out = distillation_loss(s["q"], s["k"], s["v"], t["q"], t["k"], t["v"], attn_mask=mask)
    out.loss.backward()
    torch.cuda.synchronize()
    denom = float(mask.sum()) * Hq                     # train.py:405-406
    c = 1.0 / L / denom                                # lam_A = 1: d loss / d relation loss
    assert c == 2.0 ** -23

    picks = [("q", l, l % 2, (7 * l + 3) % Hq) for l in range(L)] + [("k", 3, 1, 5), ("v", 6, 0, 2)]
    jobs = [(_np(s[k][l][b, h]).astype(np.float64), _np(t[k][l][b, h]).astype(np.float64), a,
             mask[b].cpu().numpy()) for k, l, b, h in picks]
    print(f"cfg5 launch shape: {len(jobs)} oracle heads on the CPU", flush=True)
    refs = oracle_heads(jobs)
    for (k, l, b, h), (ref_loss, ref_dx, kl_min) in zip(picks, refs):
        assert kl_min >= -1e-9, kl_min  # the oracle's per-row KL >= 0
        with torch.no_grad():
            lh = attn_kl_align(s[k][l][b:b + 1, h:h + 1].detach(), s[k][l][b:b + 1, h:h + 1].detach(),
                               t[k][l][b:b + 1, h:h + 1], t[k][l][b:b + 1, h:h + 1], attn_mask=mask[b:b + 1],
                               causal=True, sm_scale_s=a, sm_scale_t=a)
        case = f"cfg5-step-{k}{l}-b{b}h{h}"
        check_loss(lh.item(), ref_loss, case)
        check_grad(_np(s[k][l].grad[b, h]), c * ref_dx, case, f"d{k}")

    print("cfg5 launch shape: single-head launches of every Q/Q head", flush=True)
    for l in range(L):
        total = 0.0
        for b in range(B):
            for h in range(Hq):
                x = s["q"][l][b:b + 1, h:h + 1].detach().clone().requires_grad_(True)
                xt = t["q"][l][b:b + 1, h:h + 1]
                lh = attn_kl_align(x, x, xt, xt, attn_mask=mask[b:b + 1], causal=True, sm_scale_s=a, sm_scale_t=a)
                lh.backward(torch.tensor(c, device="cuda"))
                assert torch.equal(x.grad[0, 0], s["q"][l].grad[b, h]), f"Q/Q relation {l} head ({b}, {h})"
                total += lh.double().item()
        with torch.no_grad():
            lr = attn_kl_align(s["q"][l].detach(), s["q"][l].detach(), t["q"][l], t["q"][l], attn_mask=mask,
                               causal=True, sm_scale_s=a, sm_scale_t=a).double().item()
        assert _rel(lr, total) <= 1e-5, (l, lr, total)

    sums = {}
    for k in "qkv":
        with torch.no_grad():
            sums[k] = sum(attn_kl_align(x.detach(), x.detach(), y, y, attn_mask=mask, causal=True, sm_scale_s=a,
                                        sm_scale_t=a).double().item() for x, y in zip(s[k], t[k])) / denom
    for k, got in (("q", out.Q_loss), ("k", out.K_loss), ("v", out.V_loss)):
        assert _rel(got.item(), sums[k]) <= 1e-5, (k, got.item(), sums[k])
    attn = (sums["q"] + sums["k"] + sums["v"]) / L
    assert _rel(out.attn_loss.item(), attn) <= 1e-5 and out.loss.item() == out.attn_loss.item()
