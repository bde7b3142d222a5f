"""GPU parity of the autograd boundary attn_kl_align (integration.py:6-73)."""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from oracle import attn_kl_torch as OT
from tests._inputs import make_mask, mask_to_dev, randn, to_dev
from tests._tolerance import _rel, check_grad, check_loss

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
    cid = f"self-{dtype}-B{B}-H{H}-T{T}-D{D}-m{ratio}-c{int(causal)}"
    check_loss(loss.item(), rl, cid)
    g = x_s.grad.float().cpu().numpy()
    assert x_s.grad.dtype == x_s.dtype
    check_grad(g, rdx, cid)


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
    check_loss(loss.item(), rl, "gqa-masked-ds64-dt32")
    for name, got, ref in (("dq", tqs.grad, rdq), ("dk", tks.grad, rdk)):
        check_grad(got.float().cpu().numpy(), ref, "gqa-masked-ds64-dt32", name)
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
    # D = 256 here: a loss of 1.1e-3 summed from rows whose terms are ~16, so
    # float32 itself misses the 1e-3 bar (the fp32 eager oracle by 1.4e-3)
    l32 = OT.materialized_kl(torch.tensor(xs), torch.tensor(xt)).item()
    check_loss(loss.item(), rl, f"self-{dtype}-D{D}-T{T}", fp32=l32)
    check_grad(x_s.grad.float().cpu().numpy(), rdx, f"self-{dtype}-D{D}-T{T}")


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
    cid = f"gqa-both-masked-c{int(causal)}"
    check_loss(loss.item(), rl, cid)
    for name, got, ref in (("dq", tqs.grad, rdq), ("dk", tks.grad, rdk)):
        check_grad(got.float().cpu().numpy(), ref, cid, name)


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
    check_loss(loss.item(), rl, f"scales-{a_s}-{a_t}")
    check_grad(x_s.grad.float().cpu().numpy(), rdx, f"scales-{a_s}-{a_t}")


@pytest.mark.parametrize("self_rel", [1, 0])
def test_rowgrad_entry_points_through_the_c_abi(gpu_available, self_rel):
    """lard_attn_kl_forward_rowgrad + lard_attn_kl_backward_colgrad (the
    autograd pair of the throughput shapes) against the float64 oracle, with
    GQA and padding for q != k; the loss and LSEs equal lard_attn_kl_forward's."""
    from linearard_amd import _lib

    rng = np.random.default_rng(41 + self_rel)
    B, Hq, T, D = 2, 4, 290, 128
    Hkv = Hq if self_rel else 2
    qt = randn(rng, (B, Hq, T, D), "bf16")
    qs = O.round_to(qt + 0.3 * rng.standard_normal(qt.shape).astype(np.float32), "bf16")
    if self_rel:
        ks, kt = qs, qt
    else:
        kt = randn(rng, (B, Hkv, T, D), "bf16")
        ks = O.round_to(kt + 0.3 * rng.standard_normal(kt.shape).astype(np.float32), "bf16")
    mask = make_mask(rng, B, T, 0.2)
    tqs, tqt = to_dev(qs, "bf16"), to_dev(qt, "bf16")
    tks, tkt = (tqs, tqt) if self_rel else (to_dev(ks, "bf16"), to_dev(kt, "bf16"))
    m = mask_to_dev(mask)
    a = D ** -0.5
    L = _lib.lib()
    d = [_lib.tensor4(x) for x in (tqs, tks, tqt, tkt)]
    md = _lib.mask_desc(m)
    st = _lib.stream_of(tqs)
    lse_s, lse_t = torch.empty((B, Hq, T), device="cuda"), torch.empty((B, Hq, T), device="cuda")
    loss = torch.empty((), device="cuda")
    dq_row = torch.empty((B, Hq, T, D), device="cuda")
    nb = L.lard_attn_kl_forward_rowgrad_workspace_bytes(B, Hq, Hkv, Hkv, T, D)
    ws = torch.empty((nb,), device="cuda", dtype=torch.uint8)
    rc = L.lard_attn_kl_forward_rowgrad(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), ctypes.byref(d[3]),
                                        ctypes.byref(md), 1, a, a, lse_s.data_ptr(), lse_t.data_ptr(), loss.data_ptr(),
                                        dq_row.data_ptr(), ws.data_ptr(), nb, st)
    _lib.check(rc, "forward_rowgrad")
    # the plain forward gives the same loss and LSEs
    lse_s2, lse_t2, loss2 = torch.empty_like(lse_s), torch.empty_like(lse_t), torch.empty_like(loss)
    nb2 = L.lard_attn_kl_forward_workspace_bytes(B, Hq, T)
    ws2 = torch.empty((nb2,), device="cuda", dtype=torch.uint8)
    rc = L.lard_attn_kl_forward(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), ctypes.byref(d[3]),
                                ctypes.byref(md), 1, a, a, lse_s2.data_ptr(), lse_t2.data_ptr(), loss2.data_ptr(),
                                ws2.data_ptr(), nb2, st)
    _lib.check(rc, "forward")
    torch.testing.assert_close(lse_s, lse_s2, rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(lse_t, lse_t2, rtol=2e-6, atol=2e-6)
    assert _rel(loss.item(), loss2.item()) <= 1e-5
    # backward: column side, dloss = 1.5
    dloss = torch.full((), 1.5, device="cuda")
    dk = dq_row if self_rel else torch.empty((B, Hkv, T, D), device="cuda")
    nb3 = L.lard_attn_kl_backward_workspace_bytes(B, Hq, Hkv, T, D, self_rel)
    ws3 = torch.empty((nb3,), device="cuda", dtype=torch.uint8)
    rc = L.lard_attn_kl_backward_colgrad(ctypes.byref(d[0]), ctypes.byref(d[1]), lse_s.data_ptr(), ctypes.byref(d[2]),
                                         ctypes.byref(d[3]), lse_t.data_ptr(), ctypes.byref(md), 1, a, a,
                                         dloss.data_ptr(), self_rel, dq_row.data_ptr(), dk.data_ptr(), ws3.data_ptr(),
                                         nb3, st)
    _lib.check(rc, "backward_colgrad")
    rl, rdq, rdk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, True, a, a, dloss=1.5)
    cid = f"c-abi-rowgrad-self{self_rel}"
    check_loss(loss.item(), rl, cid)
    if self_rel:
        check_grad(dk.cpu().numpy(), rdq + rdk, cid)
    else:
        check_grad(dq_row.cpu().numpy(), rdq, cid, "dq")
        check_grad(dk.cpu().numpy(), rdk, cid, "dk")


def _abi_forward(qs, ks, qt, kt, m, causal):
    """lard_attn_kl_forward through the C-ABI: (lse_s, lse_t, loss)."""
    from linearard_amd import _lib

    L = _lib.lib()
    B, Hq, T, _ = qs.shape
    d = [_lib.tensor4(x) for x in (qs, ks, qt, kt)]
    md = _lib.mask_desc(m)
    lse_s, lse_t = torch.empty((B, Hq, T), device="cuda"), torch.empty((B, Hq, T), device="cuda")
    loss = torch.empty((), device="cuda")
    nb = L.lard_attn_kl_forward_workspace_bytes(B, Hq, T)
    ws = torch.empty((nb,), device="cuda", dtype=torch.uint8)
    rc = L.lard_attn_kl_forward(ctypes.byref(d[0]), ctypes.byref(d[1]), ctypes.byref(d[2]), ctypes.byref(d[3]),
                                ctypes.byref(md), int(causal), qs.shape[3] ** -0.5, qt.shape[3] ** -0.5,
                                lse_s.data_ptr(), lse_t.data_ptr(), loss.data_ptr(), ws.data_ptr(), nb,
                                _lib.stream_of(qs))
    _lib.check(rc, "attn_kl_forward")
    return lse_s.cpu().numpy(), lse_t.cpu().numpy(), loss.item()


def _check_lse(got, ref, case):
    """Float32 LSEs of the throughput kernels against the float64 oracle: masked
    rows are exactly 0, the rest within 1e-5 relative (+1e-5 absolute)."""
    got = np.asarray(got, np.float64)
    zero = ref == 0.0
    assert not np.any(got[zero]), f"{case}: masked rows must have LSE 0"
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5, err_msg=case)


def _left_padded(T, firsts, rng, holes=0.1):
    m = rng.random((len(firsts), T)) > holes
    for b, f in enumerate(firsts):
        m[b, :f] = False
        m[b, f] = True
    return m.astype(np.int32)


@pytest.mark.parametrize("api", ["attn_kl_align", "batched"])
def test_left_padding_first_valid_token_past_zero(gpu_available, api):
    """Causal rows whose first valid key is not token 0: the first valid token
    of each sequence (1, 300, 5000: another thread, wave and 64-key tile of
    the token scan) is a one-key row (KL 0, LSE = its logit, no gradient),
    every later row a normal one, against the float64 oracle."""
    from linearard_amd.attention_KL import attn_kl_align, attn_kl_align_batched

    rng = np.random.default_rng(55)
    B, H, T, D = 3, 2, 5200, 64
    mask = _left_padded(T, (1, 300, 5000), rng)
    xt = randn(rng, (B, H, T, D), "bf16")
    xs = O.round_to(xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32), "bf16")
    x_s = to_dev(xs, "bf16", requires_grad=True)
    x_t = to_dev(xt, "bf16")
    m = mask_to_dev(mask)
    if api == "attn_kl_align":
        loss = attn_kl_align(x_s, x_s, x_t, x_t, attn_mask=m, causal=True)
    else:
        loss = attn_kl_align_batched([x_s], [x_t], attn_mask=m, causal=True)
    loss.backward()
    rl, rdx, _, rls, rlt = O.attn_kl_align(xs, xs, xt, xt, mask, True, self_relation=True)
    check_loss(loss.item(), rl, f"left-padded-{api}")
    g = x_s.grad.float().cpu().numpy()
    check_grad(g, rdx, f"left-padded-{api}")
    for b, f in enumerate((1, 300, 5000)):
        # padding gets no gradient; the first valid token only its key side
        assert not np.any(g[b, :, :f]), "padding tokens get no gradient"
        diag = np.einsum("hd,hd->h", xs[b, :, f].astype(np.float64), xs[b, :, f].astype(np.float64)) / 8
        np.testing.assert_allclose(rls[b, :, f], diag, rtol=1e-12)  # a one-key row: LSE = its logit
    lse_s, lse_t, _ = _abi_forward(x_s.detach(), x_s.detach(), x_t, x_t, m, True)
    _check_lse(lse_s, rls, f"left-padded-{api} lse_s")
    _check_lse(lse_t, rlt, f"left-padded-{api} lse_t")


def test_single_valid_token_above_zero_non_causal(gpu_available):
    """Non-causal, one valid token per sequence at an index above 0: that row
    has one key (KL 0, LSE its logit), every other row is masked (LSE 0)."""
    from linearard_amd.attention_KL import attn_kl_align, lse_stats

    rng = np.random.default_rng(56)
    B, H, T, D = 2, 2, 400, 128
    mask = np.zeros((B, T), np.int32)
    mask[0, 77] = 1
    mask[1, 333] = 1
    xt = randn(rng, (B, H, T, D), "bf16")
    xs = O.round_to(xt + 0.3 * rng.standard_normal(xt.shape).astype(np.float32), "bf16")
    x_s = to_dev(xs, "bf16", requires_grad=True)
    x_t = to_dev(xt, "bf16")
    m = mask_to_dev(mask)
    loss = attn_kl_align(x_s, x_s, x_t, x_t, attn_mask=m, causal=False)
    loss.backward()
    assert loss.item() == 0.0
    assert not torch.any(x_s.grad)
    ref_s, ref_t = O.lse_stats(xs, xs, mask, False), O.lse_stats(xt, xt, mask, False)
    lse_s, lse_t, loss2 = _abi_forward(x_s.detach(), x_s.detach(), x_t, x_t, m, False)
    assert loss2 == 0.0
    _check_lse(lse_s, ref_s, "single-token lse_s")
    _check_lse(lse_t, ref_t, "single-token lse_t")
    got = lse_stats(x_s.detach(), x_s.detach(), m, False).cpu().numpy()  # stage A agrees
    _check_lse(got, ref_s, "single-token stage A")


@pytest.mark.parametrize("self_rel", [1, 0])
def test_keys_beyond_the_float16_range_take_a_scale(gpu_available, self_rel):
    """bf16 inputs with a few entries of magnitude 2^15 to 2^17 (the rest
    N(0, 256^2); scale 2^-19, inside the throughput kernels' range): the
    float16 copies of the keys then take a power-of-two scale (the fix-up
    pass after the conversion), for the student and the teacher, with the
    large entries in k or, for q != k, only in q; against the float64 oracle."""
    from linearard_amd import _lib
    from linearard_amd.attention_KL import attn_kl_align

    rng = np.random.default_rng(90 + self_rel)
    B, Hq, T, D = 1, 2, 300, 64
    Hkv = Hq if self_rel else 1
    a = 2.0 ** -19

    def draw(H, big):
        x = rng.standard_normal((B, H, T, D)).astype(np.float32) * 256
        if big:
            idx = tuple(rng.integers(0, s, 6) for s in x.shape)
            x[idx] = rng.choice([-1.0, 1.0], 6) * rng.uniform(2.0 ** 15, 2.0 ** 17, 6)
        return O.round_to(x, "bf16")

    if self_rel:
        qs = ks = draw(Hq, True)
        qt = kt = draw(Hq, True)
    else:
        qs, ks = draw(Hq, True), draw(Hkv, False)   # the student's large entries only in q
        qt, kt = draw(Hq, False), draw(Hkv, True)   # the teacher's only in k
    tqs = to_dev(qs, "bf16", requires_grad=True)
    tks = tqs if self_rel else to_dev(ks, "bf16", requires_grad=True)
    tqt = to_dev(qt, "bf16")
    tkt = tqt if self_rel else to_dev(kt, "bf16")
    L = _lib.lib()
    d = [_lib.tensor4(x.detach()) for x in (tqs, tks, tqt, tkt)]
    assert L.lard_attn_kl_path(*[ctypes.byref(x) for x in d], a, a) == 0  # the throughput kernels
    loss = attn_kl_align(tqs, tks, tqt, tkt, causal=True, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    rl, rdq, rdk, _, _ = O.attn_kl_align(qs, ks, qt, kt, None, True, a, a, self_relation=bool(self_rel))
    cid = f"f16-key-scale-self{self_rel}"
    check_loss(loss.item(), rl, cid)
    check_grad(tqs.grad.float().cpu().numpy(), rdq, cid, "dX" if self_rel else "dq")
    if not self_rel:
        check_grad(tks.grad.float().cpu().numpy(), rdk, cid, "dk")


@pytest.mark.parametrize("case", ["self", "gqa", "batched"])
def test_second_backward_through_the_same_graph(gpu_available, case):
    """retain_graph: the first backward adds the column side to the row side
    the forward formed; the second finds that buffer consumed and runs the
    full backward.  Both gradients against the float64 oracle."""
    from linearard_amd.attention_KL import attn_kl_align, attn_kl_align_batched

    rng = np.random.default_rng(61)
    B, Hq, T, D = 2, 4, 300, 128
    Hkv = 2 if case == "gqa" else Hq
    qt = randn(rng, (B, Hq, T, D), "bf16")
    qs = O.round_to(qt + 0.3 * rng.standard_normal(qt.shape).astype(np.float32), "bf16")
    mask = make_mask(rng, B, T, 0.2)
    m = mask_to_dev(mask)
    if case == "gqa":
        kt = randn(rng, (B, Hkv, T, D), "bf16")
        ks = O.round_to(kt + 0.3 * rng.standard_normal(kt.shape).astype(np.float32), "bf16")
        x_q, x_k = to_dev(qs, "bf16", True), to_dev(ks, "bf16", True)
        y_q, y_k = to_dev(qt, "bf16"), to_dev(kt, "bf16")
        loss = attn_kl_align(x_q, x_k, y_q, y_k, attn_mask=m, causal=True)
        inputs = [x_q, x_k]
        rl, rdq, rdk, _, _ = O.attn_kl_align(qs, ks, qt, kt, mask, True)
        refs = [("dq", rdq), ("dk", rdk)]
    else:
        x, y = to_dev(qs, "bf16", True), to_dev(qt, "bf16")
        if case == "self":
            loss = attn_kl_align(x, x, y, y, attn_mask=m, causal=True)
        else:
            loss = attn_kl_align_batched([x], [y], attn_mask=m, causal=True)
        inputs = [x]
        rl, rdx, _, _, _ = O.attn_kl_align(qs, qs, qt, qt, mask, True, self_relation=True)
        refs = [("dX", rdx)]
    check_loss(loss.item(), rl, f"second-backward-{case}")
    for rep in ("first", "second"):
        grads = torch.autograd.grad(loss, inputs, retain_graph=True)
        for (name, ref), g in zip(refs, grads):
            check_grad(g.float().cpu().numpy(), ref, f"second-backward-{case}-{rep}", name)
