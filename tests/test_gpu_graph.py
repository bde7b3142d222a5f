"""Forward + backward captured in a HIP graph and replayed: attn_kl_align,
the batched relation loss (relation_kl_loss), the logits KL, and the RoPE
pair producer feeding distillation_loss.

The library only launches kernels on the caller's stream: no allocation, no
memset node, no host synchronisation (the drop-in boundary's graph-capture
contract). Its outputs and workspaces come from torch's graph pool.  A
replay on new input values must therefore equal the eager computation on
those values, bitwise: the loss is summed in a fixed order, and no gradient
uses atomics.  The replays are separated by eager work and a
synchronisation, and every replay is checked.
"""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _draw(g, shape, noise):
    xt = torch.randn(shape, device="cuda", generator=g)
    xs = xt + noise * torch.randn(shape, device="cuda", generator=g)
    return xs.to(torch.bfloat16), xt.to(torch.bfloat16)


@pytest.mark.parametrize("masked", [False, True])
def test_fwd_bwd_graph_replays_match_eager(gpu_available, masked):
    from linearard_amd.attention_KL import attn_kl_align

    B, H, T, D = 2, 4, 1024, 128
    a = 1 / math.sqrt(D)
    g = torch.Generator(device="cuda").manual_seed(17)
    mask = None
    if masked:
        mask = (torch.rand((B, T), device="cuda", generator=g) > 0.2).to(torch.int32)
    s0, t0 = _draw(g, (B, H, T, D), 0.2)
    xs = s0.clone().requires_grad_(True)  # static graph inputs
    xt = t0.clone()

    def run(x, y):
        loss = attn_kl_align(x, x, y, y, attn_mask=mask, causal=True, sm_scale_s=a, sm_scale_t=a)
        (grad,) = torch.autograd.grad(loss, x)
        return loss, grad

    side = torch.cuda.Stream()  # warm up off the capture stream, as torch requires
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run(xs, xt)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss_g, grad_g = run(xs, xt)

    for rep in range(3):
        s_new, t_new = _draw(g, (B, H, T, D), 0.1 + 0.1 * rep)
        with torch.no_grad():
            xs.copy_(s_new)
            xt.copy_(t_new)
        graph.replay()
        torch.cuda.synchronize()
        got_loss, got_grad = loss_g.clone(), grad_g.clone()
        x = s_new.clone().requires_grad_(True)  # eager on the same values, between replays
        want_loss, want_grad = run(x, t_new)
        torch.cuda.synchronize()
        assert torch.equal(got_loss, want_loss), (rep, got_loss.item(), want_loss.item())
        assert torch.equal(got_grad, want_grad), rep
        assert got_loss.item() > 0.0


def _capture_and_check(run, inputs, redraw, reps=3):
    """Warm up, capture run(*inputs) -> (loss, *grads) once, then for each
    replay: redraw the inputs in place, replay, and compare with run() on
    fresh copies of the same values."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run(*inputs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run(*inputs)
    for rep in range(reps):
        values = redraw(rep)
        with torch.no_grad():
            for dst, v in zip(inputs, values):
                dst.copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        fresh = [v.clone().requires_grad_(src.requires_grad) for src, v in zip(inputs, values)]
        want = run(*fresh)
        torch.cuda.synchronize()
        for i, (x, y) in enumerate(zip(got, want)):
            assert torch.equal(x, y), (rep, i)


def test_batched_relation_loss_graph_replays_match_eager(gpu_available):
    """relation_kl_loss (train.py:369-410 in batched launches): descriptors in
    the kernel arguments, per-relation weights as device scalars."""
    from linearard_amd.attention_KL import relation_kl_loss

    B, T, D, layers = 1, 512, 128, 2
    a = 1 / math.sqrt(D)
    g = torch.Generator(device="cuda").manual_seed(23)
    heads = [h for _ in range(layers) for h in (8, 2, 2)]

    def redraw(rep):
        pairs = [_draw(g, (B, h, T, D), 0.2 + 0.05 * rep) for h in heads]
        return [p[0] for p in pairs] + [p[1] for p in pairs]

    first = redraw(0)
    n = len(heads)
    inputs = [v.clone().requires_grad_(i < n) for i, v in enumerate(first)]

    def run(*xs):
        s, t = xs[:n], xs[n:]
        loss = relation_kl_loss(s[0::3], s[1::3], s[2::3], t[0::3], t[1::3], t[2::3], sm_scale_s=a, sm_scale_t=a)
        grads = torch.autograd.grad(loss, list(s))
        return (loss, *grads)

    _capture_and_check(run, inputs, redraw)


def test_logits_kl_graph_replays_match_eager(gpu_available):
    """logits_kl (train.py:412-420): forward, finish and gradient kernels."""
    from linearard_amd.logits_kl import logits_kl

    B, K, V = 2, 64, 32000
    g = torch.Generator(device="cuda").manual_seed(29)

    def redraw(rep):
        t = torch.randn((B, K, V), device="cuda", generator=g)
        s = t + (0.5 + 0.1 * rep) * torch.randn((B, K, V), device="cuda", generator=g)
        return [s.to(torch.bfloat16), t.to(torch.bfloat16)]

    first = redraw(0)
    inputs = [first[0].clone().requires_grad_(True), first[1].clone()]

    def run(s, t):
        loss = logits_kl(t, s, temperature=2.0)
        (gs,) = torch.autograd.grad(loss, s)
        return loss, gs

    _capture_and_check(run, inputs, redraw)


def test_rope_pair_and_distillation_loss_graph_replays_match_eager(gpu_available):
    """The RoPE pair producer feeding distillation_loss (train.py:360-423,
    lam_L != 0, masked), forward + backward, in one graph."""
    from linearard_amd.distill import distillation_loss
    from linearard_amd.rope import rope_pair

    B, T, D, H, Hkv, L, K, V = 2, 256, 128, 4, 2, 2, 16, 1024
    g = torch.Generator(device="cuda").manual_seed(31)
    mask = torch.ones((B, T), device="cuda", dtype=torch.int64)
    mask[1, T - 40:] = 0
    shapes = [(B, T, h, D) for _ in range(L) for h in (H, Hkv, Hkv)]  # per layer: q, k, v as the hook sees them

    def redraw(rep):
        pre = [torch.randn(sh, device="cuda", generator=g).to(torch.bfloat16) for sh in shapes]
        t_log = torch.randn((B, K, V), device="cuda", generator=g)
        s_log = t_log + (0.3 + 0.1 * rep) * torch.randn((B, K, V), device="cuda", generator=g)
        return pre + [s_log.to(torch.bfloat16), t_log.to(torch.bfloat16)]

    first = redraw(0)
    n = len(shapes)
    inputs = [v.clone().requires_grad_(i == n) for i, v in enumerate(first)]  # the student logits take a gradient

    def run(*xs):
        pre, s_log, t_log = xs[:n], xs[n], xs[n + 1]
        qs, qt, ks, kt, vs, vt = [], [], [], [], [], []
        for li in range(L):
            q, k, v = (pre[3 * li + j].permute(0, 2, 1, 3) for j in range(3))
            q_s, q_t = rope_pair(q, 10000.0, {"rope_type": "linear", "factor": 4.0})
            k_s, k_t = rope_pair(k, 10000.0, {"rope_type": "linear", "factor": 4.0})
            qs.append(q_s.detach().requires_grad_(True)); qt.append(q_t)
            ks.append(k_s.detach().requires_grad_(True)); kt.append(k_t)
            vs.append((v + 0.01).detach().requires_grad_(True)); vt.append(v)
        out = distillation_loss(qs, ks, vs, qt, kt, vt, t_logits=t_log, s_logits=s_log, attn_mask=mask,
                                lam_A=1.0, lam_L=0.5, temperature=2.0)
        grads = torch.autograd.grad(out.loss, qs + ks + vs + [s_log])
        return (out.loss, out.attn_loss, out.logits_loss, *grads)

    _capture_and_check(run, inputs, redraw)
