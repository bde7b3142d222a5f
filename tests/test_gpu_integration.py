"""GPU parity of the autograd boundary attn_kl_align (integration.py:6-73)."""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from tests._inputs import make_mask, mask_to_dev, randn, to_dev
from tests._tolerance import _grad_ok, _logit_bound, _loss_ok, _rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,B,H,T,D,ratio,causal", [
    ("bf16", 1, 4, 300, 128, None, True),
    ("bf16", 2, 2, 129, 64, 0.2, True),
    ("f16", 1, 2, 77, 32, None, False),
    ("bf16", 1, 2, 1, 128, None, True),
])
def test_self_relation_fwd_bwd(gpu_available, dtype, B, H, T, D, ratio, causal):
    """train.py:380-402: attn_kl_align(x_s, x_s, x_t, x_t) with one shared gradient."""
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(100 + T)
    xt = randn(rng, (B, H, T, D), dtype)
    xs = O.round_to(xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32), dtype)
    mask = None if ratio is None else make_mask(rng, B, T, ratio)
    a = 1 / math.sqrt(D)
    x_s = to_dev(xs, dtype, requires_grad=True)
    x_t = to_dev(xt, dtype)
    loss = attn_kl_align(x_s, x_s, x_t, x_t, attn_mask=mask_to_dev(mask), causal=causal, sm_scale_s=a, sm_scale_t=a)
    assert loss.dim() == 0 and loss.dtype == torch.float32
    loss.backward()
    rl, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, mask, causal, a, a, self_relation=True)
    lb = _logit_bound((xs, xs, a), (xt, xt, a))
    assert _loss_ok(loss.item(), rl, B * H * T, lb), (loss.item(), rl)
    g = x_s.grad.float().cpu().numpy()
    assert x_s.grad.dtype == x_s.dtype
    assert _grad_ok(g, rdx, xs, a, lb)


def test_general_gqa_masked_fwd_bwd_and_chain_rule(gpu_available):
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(9)
    B, Hq, Hks, Hkt, T, Ds, Dt = 2, 8, 4, 2, 70, 64, 32
    qs, ks = randn(rng, (B, Hq, T, Ds), "f16"), randn(rng, (B, Hks, T, Ds), "f16")
    qt, kt = randn(rng, (B, Hq, T, Dt), "f16"), randn(rng, (B, Hkt, T, Dt), "f16")
    mask = make_mask(rng, B, T, 0.3)
    tqs, tks = to_dev(qs, "f16", True), to_dev(ks, "f16", True)
    tqt, tkt = to_dev(qt, "f16"), to_dev(kt, "f16")
    loss = attn_kl_align(tqs, tks, tqt, tkt, attn_mask=mask_to_dev(mask), causal=True)
    (2.5 * loss).backward()
    rl, rdq, rdk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, True, dloss=2.5)
    assert _loss_ok(loss.item(), rl, B * Hq * T), (loss.item(), rl)
    for got, ref in ((tqs.grad, rdq), (tks.grad, rdk)):
        g = got.float().cpu().numpy()
        assert np.abs(g - ref).max() / np.abs(ref).max() <= 2e-2
    assert tqt.grad is None and tkt.grad is None


def test_identical_relations_give_exact_zero(gpu_available):
    """V/V with unrotated values: KL(P||P) == 0 exactly and the gradient vanishes."""
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(4)
    x = randn(rng, (1, 4, 513, 128), "bf16")
    x_s = to_dev(x, "bf16", True)
    x_t = to_dev(x, "bf16")
    loss = attn_kl_align(x_s, x_s, x_t, x_t)
    loss.backward()
    assert loss.item() == 0.0
    assert torch.count_nonzero(x_s.grad).item() == 0


def test_drop_in_import_path(gpu_available):
    from kernels.attention_KL.integration import attn_kl_align as via_reference_path
    from linearard_amd.attention_KL import attn_kl_align

    assert via_reference_path is attn_kl_align


@pytest.mark.parametrize("dtype,D,T,H", [("f16", 8, 45, 2), ("bf16", 16, 200, 2), ("bf16", 256, 97, 2), ("f16", 128, 1000, 2)])
def test_self_relation_fused_and_fallback_dims(gpu_available, dtype, D, T, H):
    """D <= 128 runs the throughput kernels; D = 256 the generic fused forward
    and the stage C kernels."""
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(7 + D)
    xt = randn(rng, (1, H, T, D), dtype)
    xs = O.round_to(xt + 0.2 * rng.standard_normal(xt.shape).astype(np.float32), dtype)
    x_s = to_dev(xs, dtype, requires_grad=True)
    loss = attn_kl_align(x_s, x_s, to_dev(xt, dtype), to_dev(xt, dtype))
    loss.backward()
    rl, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, None, True, self_relation=True)
    a = D ** -0.5
    assert _loss_ok(loss.item(), rl, H * T, _logit_bound((xs, xs, a), (xt, xt, a))), (loss.item(), rl)
    g = x_s.grad.float().cpu().numpy()
    assert np.abs(g - rdx).max() / np.abs(rdx).max() <= 2e-2


def test_slower_paths_warn_once_per_condition(gpu_available):
    """Inputs off the throughput kernels (here D = 256, and Ds != Dt) raise one
    RuntimeWarning per condition naming it; the throughput path warns nothing."""
    import warnings

    from linearard_amd.attention_KL import attn_kl_align, integration

    integration._WARNED.clear()
    x = torch.randn((1, 2, 40, 256), device="cuda", dtype=torch.bfloat16)
    with pytest.warns(RuntimeWarning, match="head dim 256 > 128.*fused-forward"):
        attn_kl_align(x, x, x, x)
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # the same condition again: no second warning
        attn_kl_align(x, x, x, x)
        y = torch.randn((1, 2, 40, 128), device="cuda", dtype=torch.bfloat16)
        attn_kl_align(y, y, y, y)  # throughput kernels: silent
    z = torch.randn((1, 2, 40, 64), device="cuda", dtype=torch.bfloat16)
    with pytest.warns(RuntimeWarning, match="student head dim 64 != teacher head dim 128.*stage"):
        attn_kl_align(z, z, y, y)


def test_fused_forward_and_backward_match_stage_kernels(gpu_available):
    """lard_attn_kl_forward / _backward (throughput kernels) against the
    reference-semantics stage kernels: stage A x2, stage B, stage C."""
    import ctypes

    from linearard_amd import _lib
    from linearard_amd.attention_KL import kl_backward, kl_forward, lse_stats

    rng = np.random.default_rng(21)
    B, H, T, D = 2, 4, 333, 128
    xs, xt = randn(rng, (B, H, T, D), "bf16"), randn(rng, (B, H, T, D), "bf16")
    ks_, kt_ = randn(rng, (B, H, T, D), "bf16"), randn(rng, (B, H, T, D), "bf16")
    mask = make_mask(rng, B, T, 0.25)
    s, t, m = to_dev(xs, "bf16"), to_dev(xt, "bf16"), mask_to_dev(mask)
    sk, tk = to_dev(ks_, "bf16"), to_dev(kt_, "bf16")
    a = D ** -0.5
    L = _lib.lib()
    for (qs, ks, qt, kt, self_rel) in ((s, s, t, t, 1), (s, sk, t, tk, 0)):
        lse_s, lse_t = torch.empty((B, H, T), device="cuda"), torch.empty((B, H, T), device="cuda")
        loss = torch.empty((), device="cuda")
        nb = L.lard_attn_kl_forward_workspace_bytes(B, H, T)
        ws = torch.empty((nb,), device="cuda", dtype=torch.uint8)
        d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
        md = _lib.mask_desc(m)
        rc = L.lard_attn_kl_forward(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), ctypes.byref(d[3]),
                                    ctypes.byref(md), 1, a, a, lse_s.data_ptr(), lse_t.data_ptr(), loss.data_ptr(),
                                    ws.data_ptr(), nb, _lib.stream_of(s))
        _lib.check(rc, "forward")
        ref_ls, ref_lt = lse_stats(qs, ks, m, True, a), lse_stats(qt, kt, m, True, a)
        torch.testing.assert_close(lse_s, ref_ls, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(lse_t, ref_lt, rtol=1e-5, atol=1e-5)
        ref_loss = kl_forward(qs, ks, ref_ls, qt, kt, ref_lt, m, True, a, a).item()
        assert _rel(loss.item(), ref_loss) <= 1e-4

        dq = torch.empty((B, H, T, D), device="cuda")
        dk = torch.empty((B, H, T, D), device="cuda")
        nb = L.lard_attn_kl_backward_workspace_bytes(B, H, H, T, D, self_rel)
        ws = torch.empty((nb,), device="cuda", dtype=torch.uint8)
        rc = L.lard_attn_kl_backward(ctypes.byref(d[0]), ctypes.byref(d[1]), lse_s.data_ptr(), ctypes.byref(d[2]),
                                     ctypes.byref(d[3]), lse_t.data_ptr(), ctypes.byref(md), 1, a, a, None, self_rel,
                                     dq.data_ptr(), dk.data_ptr(), ws.data_ptr(), nb, _lib.stream_of(s))
        _lib.check(rc, "backward")
        ref_dq, ref_dk = kl_backward(qs, ks, lse_s, qt, kt, lse_t, m, True, a, a)
        pairs = ((dk, ref_dq + ref_dk),) if self_rel else ((dq, ref_dq), (dk, ref_dk))
        for got, ref in pairs:
            err = (got - ref).abs().max().item() / ref.abs().max().item()
            assert err <= 5e-3, err  # same formula, same D cast: agreement to summation order


def test_forward_without_grad_and_determinism(gpu_available):
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(8)
    xs, xt = randn(rng, (1, 8, 700, 128), "bf16"), randn(rng, (1, 8, 700, 128), "bf16")
    s, t = to_dev(xs, "bf16", True), to_dev(xt, "bf16")
    with torch.no_grad():
        l0 = attn_kl_align(s, s, t, t).item()
    l1 = attn_kl_align(s, s, t, t)
    l1.backward()
    g1 = s.grad.clone()
    s.grad = None
    l2 = attn_kl_align(s, s, t, t)
    l2.backward()
    assert _rel(l0, l1.item()) <= 1e-6  # no-grad instance vs grad instance of the fused kernel
    assert l1.item() == l2.item()       # bitwise deterministic: no atomics anywhere
    assert torch.equal(g1, s.grad)


@pytest.mark.parametrize("causal", [True, False])
def test_hot_path_gqa_masked(gpu_available, causal):
    """Ds == Dt (the throughput kernels) with GQA on both sides and padding."""
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(31)
    B, Hq, Hks, Hkt, T, D = 2, 8, 2, 4, 150, 64
    qs, ks = randn(rng, (B, Hq, T, D), "bf16"), randn(rng, (B, Hks, T, D), "bf16")
    qt, kt = randn(rng, (B, Hq, T, D), "bf16"), randn(rng, (B, Hkt, T, D), "bf16")
    mask = make_mask(rng, B, T, 0.3, "bool")
    tqs, tks = to_dev(qs, "bf16", True), to_dev(ks, "bf16", True)
    loss = attn_kl_align(tqs, tks, to_dev(qt, "bf16"), to_dev(kt, "bf16"), attn_mask=mask_to_dev(mask),
                         causal=causal)
    loss.backward()
    rl, rdq, rdk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, causal)
    assert _loss_ok(loss.item(), rl, B * Hq * T), (loss.item(), rl)
    for got, ref in ((tqs.grad, rdq), (tks.grad, rdk)):
        g = got.float().cpu().numpy()
        assert np.abs(g - ref).max() / np.abs(ref).max() <= 2e-2


@pytest.mark.parametrize("a_s,a_t", [(-0.09, -0.09), (0.05, -0.12), (0.3, 0.02), (3e-7, 0.1), (1e-4, 150.0)])
def test_hot_path_signed_and_unequal_scales(gpu_available, a_s, a_t):
    """Scales of either sign and ratio (the reference accepts any finite scale).
    The last two cases (a scale below 1e-6, a ratio above 1e6) take the stage
    kernels instead of the throughput kernels."""
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(7)
    B, H, T, D = 1, 2, 333, 128
    xt = randn(rng, (B, H, T, D), "bf16")
    xs = O.round_to(xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32), "bf16")
    x_s = to_dev(xs, "bf16", requires_grad=True)
    x_t = to_dev(xt, "bf16")
    loss = attn_kl_align(x_s, x_s, x_t, x_t, causal=True, sm_scale_s=a_s, sm_scale_t=a_t)
    loss.backward()
    rl, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, None, True, a_s, a_t, self_relation=True)
    lb = _logit_bound((xs, xs, abs(a_s)), (xt, xt, abs(a_t)))
    assert _loss_ok(loss.item(), rl, B * H * T, lb), (loss.item(), rl)
    assert _grad_ok(x_s.grad.float().cpu().numpy(), rdx, xs, abs(a_s), lb)
