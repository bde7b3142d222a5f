"""lard_attn_kl_forward_noalloc (the forward without a workspace argument,
no counterpart in the reference) against lard_attn_kl_forward, through the C
ABI: two calls in a row, the second with a smaller input, each equal bitwise
to the workspace entry point (the same kernels run on the same inputs)."""

import ctypes
import math

import numpy as np
import pytest
import torch

from linearard_amd import _lib
from tests._inputs import make_mask, mask_to_dev, randn, to_dev

pytestmark = pytest.mark.gpu


def _forward(L, xs, xt, mask, causal, a, noalloc):
    B, H, T, _ = xs.shape
    lse_s = torch.full((B, H, T), float("nan"), device="cuda")
    lse_t = torch.full((B, H, T), float("nan"), device="cuda")
    loss = torch.full((), float("nan"), device="cuda")
    d = [_lib.tensor4(x) for x in (xs, xs, xt, xt)]
    md = _lib.mask_desc(mask)
    args = [ctypes.byref(x) for x in d] + [ctypes.byref(md), int(causal), a, a, lse_s.data_ptr(), lse_t.data_ptr(),
                                           loss.data_ptr()]
    if noalloc:
        rc = L.lard_attn_kl_forward_noalloc(*args, _lib.stream_of(xs))
    else:
        nb = L.lard_attn_kl_forward_workspace_bytes(B, H, T)
        ws = torch.empty((nb,), device="cuda", dtype=torch.uint8)
        rc = L.lard_attn_kl_forward(*args, ws.data_ptr(), nb, _lib.stream_of(xs))
    assert rc == 0, L.lard_last_error()
    torch.cuda.synchronize()
    return loss, lse_s, lse_t


def test_noalloc_first_call_captured_in_a_graph(gpu_available):
    """The process's first noalloc call -- with its one-time lookup of this
    device's scratch array -- made under HIP graph capture (this test runs
    before the file's other noalloc calls); every replay on new input values
    equals the workspace forward bitwise, and a warm eager call leaves the
    device's free memory unchanged."""
    L = _lib.lib()
    B, H, T, D = 2, 4, 700, 128
    a = 1 / math.sqrt(D)
    g = torch.Generator(device="cuda").manual_seed(5)

    def draw():
        xt = torch.randn((B, H, T, D), device="cuda", generator=g)
        return (xt + 0.3 * torch.randn(xt.shape, device="cuda", generator=g)).to(torch.bfloat16), \
            xt.to(torch.bfloat16)

    x_s, x_t = draw()  # static graph inputs and outputs
    lse_s, lse_t = torch.empty((B, H, T), device="cuda"), torch.empty((B, H, T), device="cuda")
    loss = torch.empty((), device="cuda")
    d = [_lib.tensor4(x) for x in (x_s, x_s, x_t, x_t)]
    md = _lib.mask_desc(None)

    def call():
        rc = L.lard_attn_kl_forward_noalloc(*[ctypes.byref(x) for x in d], ctypes.byref(md), 1, a, a,
                                            lse_s.data_ptr(), lse_t.data_ptr(), loss.data_ptr(),
                                            _lib.stream_of(x_s))
        assert rc == 0, L.lard_last_error()

    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(3):
        s_new, t_new = draw()
        x_s.copy_(s_new)
        x_t.copy_(t_new)
        graph.replay()
        torch.cuda.synchronize()
        got = (loss.clone(), lse_s.clone(), lse_t.clone())
        want = _forward(L, s_new, t_new, None, True, a, noalloc=False)  # eager, between replays
        for x, y in zip(got, want):
            assert torch.equal(x, y), rep
        assert got[0].item() > 0.0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    call()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0


def test_noalloc_forward_equals_the_workspace_forward(gpu_available):
    L = _lib.lib()
    cases = [  # (dtype, B, H, T, D, mask ratio, causal): the second call is smaller
        ("bf16", 2, 8, 1500, 128, 0.2, True),
        ("f16", 1, 3, 300, 64, None, False),
        ("bf16", 1, 2, 257, 256, None, True),  # the fused D = 256 forward
    ]
    rng = np.random.default_rng(77)
    for dtype, B, H, T, D, ratio, causal in cases:
        xt = randn(rng, (B, H, T, D), dtype)
        xs = xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32)
        x_s, x_t = to_dev(xs, dtype), to_dev(xt, dtype)
        mask = mask_to_dev(None if ratio is None else make_mask(rng, B, T, ratio))
        a = 1 / math.sqrt(D)
        got = _forward(L, x_s, x_t, mask, causal, a, noalloc=True)
        ref = _forward(L, x_s, x_t, mask, causal, a, noalloc=False)
        for g, r in zip(got, ref):
            assert torch.equal(g, r), (dtype, B, H, T, D)
        assert got[0].item() > 0.0
