"""attn_kl_align forward + backward captured in a HIP graph and replayed.

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
