"""GPU parity of the logits KL (train.py:412-420) against the float64 oracle,
torch's float32 evaluation of the same formula, and the reference's own
lines run in bf16 on the GPU.

Tolerances (float32 arithmetic against float64):
* per-row KL: 1e-5 * (1 + |lse_t| + |lse_s| + E_pt|q_t - q_s|): the float32
  roundings of the exponents (|q| log2 e relative 2^-24), of v_exp_f32 and
  of the sums, carried through KL = E_pt[q_t - q_s] - lse_t + lse_s;
* lse: 1e-5 * (1 + |lse|);
* gradients: one rounding to the output dtype (2^-8 bf16, 2^-11 fp16
  relative, half the fp16 subnormal spacing absolute) plus
  1e-5 * c * (p_t + p_s) * (1 + |l_t| + |l_s| + |KL|).
"""

import ctypes
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import logits_kl as O
from oracle.attn_kl import round_to

pytestmark = pytest.mark.gpu

_TORCH = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
_REL = {"bf16": 2.0 ** -8, "f16": 2.0 ** -11, "f32": 0.0}
_ABS = {"bf16": 0.0, "f16": 2.0 ** -25, "f32": 0.0}


def _pair(rng, shape, dtype, scale=3.0, noise=1.5):
    t = round_to((scale * rng.standard_normal(shape)).astype(np.float32), dtype)
    s = round_to(t + (noise * rng.standard_normal(shape)).astype(np.float32), dtype)
    return t, s


def _dev(x, dtype, requires_grad=False):
    return torch.from_numpy(x).to(_TORCH[dtype]).cuda().requires_grad_(requires_grad)


def _abi_forward(t, s, T):
    """lard_logits_kl_forward through the C ABI: (loss, kl, lse_t, lse_s) on the host."""
    from linearard_amd import _lib

    L = _lib.lib()
    B, K, V = t.shape
    rows = B * K
    lse_t, lse_s, kl = (torch.empty(rows, device="cuda") for _ in range(3))
    loss = torch.empty((), device="cuda")
    nbytes = L.lard_logits_kl_workspace_bytes(rows, V)
    ws = torch.empty(max(nbytes, 16), device="cuda", dtype=torch.uint8)
    dt, ds = _lib.logits_desc(t), _lib.logits_desc(s)
    rc = L.lard_logits_kl_forward(ctypes.byref(dt), ctypes.byref(ds), T, lse_t.data_ptr(), lse_s.data_ptr(),
                                  kl.data_ptr(), loss.data_ptr(), ws.data_ptr(), nbytes, _lib.stream_of(t))
    _lib.check(rc, "lard_logits_kl_forward")
    torch.cuda.synchronize()
    return loss.item(), kl.cpu().numpy(), lse_t.cpu().numpy(), lse_s.cpu().numpy()


def _row_scale(t, s, T, dtype):
    qt = O.scale_logits(t, T, dtype).astype(np.float64)
    qs = O.scale_logits(s, T, dtype).astype(np.float64)
    _, _, lse_t, lse_s = O.logits_kl(t, s, T, dtype)
    pt = np.exp(qt - lse_t[..., None])
    return 1.0 + np.abs(lse_t) + np.abs(lse_s) + np.sum(pt * np.abs(qt - qs), axis=-1)


def _grad_tol(t, s, T, dtype, c):
    qt = O.scale_logits(t, T, dtype).astype(np.float64)
    qs = O.scale_logits(s, T, dtype).astype(np.float64)
    _, kl, lse_t, lse_s = O.logits_kl(t, s, T, dtype)
    lt, ls = qt - lse_t[..., None], qs - lse_s[..., None]
    pt, ps = np.exp(lt), np.exp(ls)
    return 1e-5 * np.abs(c) * (pt + ps) * (1 + np.abs(lt) + np.abs(ls) + np.abs(kl[..., None]))


def _check_grad(got, want, tol, dtype):
    got = got.float().cpu().numpy().astype(np.float64)
    bound = _REL[dtype] * np.abs(want) + _ABS[dtype] + tol * (1 + _REL[dtype]) + 1e-30
    err = np.abs(got - want)
    assert np.all(err <= bound), (float(err.max()), float((err / bound).max()))


CASES = [
    ("bf16", 1, 7, 1000, 1.0),
    ("bf16", 2, 5, 32000, 1.0),      # Llama-2 / Mistral-7B-v0.1 vocabulary
    ("bf16", 1, 3, 4099, 0.7),       # odd V (rows copied to 16-byte boundaries), inexact 1/T
    ("f16", 1, 4, 2051, 1.0),
    ("f32", 2, 3, 777, 2.0),
    ("bf16", 1, 16, 128256, 1.0),    # Llama-3 vocabulary
]


@pytest.mark.parametrize("dtype,B,K,V,T", CASES)
def test_forward_and_gradients_match_the_oracle(gpu_available, dtype, B, K, V, T):
    from linearard_amd.logits_kl import logits_kl

    rng = np.random.default_rng(B * 1000 + V)
    t, s = _pair(rng, (B, K, V), dtype)
    xt, xs = _dev(t, dtype, True), _dev(s, dtype, True)
    loss = logits_kl(xt, xs, temperature=T)
    assert loss.dtype == torch.float32 and loss.dim() == 0
    loss.backward()
    rl, kl, _, _ = O.logits_kl(t, s, T, dtype)
    scale = _row_scale(t, s, T, dtype)
    assert abs(loss.item() - rl) <= 1e-5 * scale.mean(), (loss.item(), rl)
    gt, gs = O.logits_kl_grads(t, s, T, dtype, dloss=1.0, reduction="mean")
    c = 1.0 / (B * K) * float(np.float32(1) / np.float32(T))
    _check_grad(xs.grad, gs, _grad_tol(t, s, T, dtype, c), dtype)
    _check_grad(xt.grad, gt, _grad_tol(t, s, T, dtype, c), dtype)
    assert xs.grad.dtype == xs.dtype and xs.grad.shape == xs.shape


@pytest.mark.parametrize("dtype,B,K,V,T", [("bf16", 2, 6, 3000, 1.0), ("f32", 1, 5, 1024, 1.3)])
def test_abi_outputs_match_the_oracle(gpu_available, dtype, B, K, V, T):
    rng = np.random.default_rng(V)
    t, s = _pair(rng, (B, K, V), dtype)
    loss, kl, lse_t, lse_s = _abi_forward(_dev(t, dtype), _dev(s, dtype), T)
    rl, rkl, rlt, rls = O.logits_kl(t, s, T, dtype)
    scale = _row_scale(t, s, T, dtype).ravel()
    assert np.all(np.abs(kl - rkl.ravel()) <= 1e-5 * scale)
    assert np.all(np.abs(lse_t - rlt.ravel()) <= 1e-5 * (1 + np.abs(rlt.ravel())))
    assert np.all(np.abs(lse_s - rls.ravel()) <= 1e-5 * (1 + np.abs(rls.ravel())))
    assert abs(loss - rl) <= 1e-5 * scale.mean()


def test_per_position_reduction_with_upstream_weights(gpu_available):
    from linearard_amd.logits_kl import logits_kl

    rng = np.random.default_rng(12)
    dtype, B, K, V = "bf16", 2, 3, 5000
    t, s = _pair(rng, (B, K, V), dtype)
    w = rng.uniform(-1.0, 2.0, (B, K)).astype(np.float32)
    xs = _dev(s, dtype, True)
    kl = logits_kl(_dev(t, dtype), xs, reduction="none")
    assert kl.shape == (B, K) and kl.dtype == torch.float32
    (kl * torch.from_numpy(w).cuda()).sum().backward()
    _, rkl, _, _ = O.logits_kl(t, s, 1.0, dtype)
    assert np.all(np.abs(kl.detach().cpu().numpy() - rkl) <= 1e-5 * _row_scale(t, s, 1.0, dtype))
    _, gs = O.logits_kl_grads(t, s, 1.0, dtype, dloss=w, reduction="none")
    _check_grad(xs.grad, gs, _grad_tol(t, s, 1.0, dtype, w[..., None]), dtype)


def test_large_and_rising_logits_take_the_rescale_path(gpu_available):
    """Logits rising along the vocabulary (the running maximum is raised
    again and again) and spanning +-60, in fp32."""
    from linearard_amd.logits_kl import logits_kl

    rng = np.random.default_rng(13)
    V = 20000
    ramp = np.linspace(-60.0, 60.0, V, dtype=np.float32)
    t = (ramp + rng.standard_normal((2, 3, V)).astype(np.float32)).astype(np.float32)
    s = (ramp[::-1] * 0.5 + 3.0 * rng.standard_normal((2, 3, V)).astype(np.float32)).astype(np.float32)
    xs = _dev(s, "f32", True)
    loss = logits_kl(_dev(t, "f32"), xs)
    loss.backward()
    rl, _, _, _ = O.logits_kl(t, s, 1.0, "f32")
    assert abs(loss.item() - rl) <= 1e-5 * _row_scale(t, s, 1.0, "f32").mean()
    _, gs = O.logits_kl_grads(t, s, 1.0, "f32")
    _check_grad(xs.grad, gs, _grad_tol(t, s, 1.0, "f32", 1.0 / 6), "f32")


def test_matches_torch_float32_formula_at_the_llama3_shape(gpu_available):
    """B=1, K=512 (--logits-keep-k), V=128256 (Llama-3-8B) bf16 logits: the
    kernels against torch's float32 evaluation of train.py:413-419 on the
    same device, and against the reference's own lines in bf16 within the
    bound of their roundings."""
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(0)
    B, K, V = 1, 512, 128256
    t = (3.0 * torch.randn((B, K, V), device="cuda", generator=g)).to(torch.bfloat16)
    s = (t.float() + 1.5 * torch.randn((B, K, V), device="cuda", generator=g)).to(torch.bfloat16)
    xs = s.clone().requires_grad_(True)
    loss = logits_kl(t, xs)
    loss.backward()

    t32, s32 = t.float(), s.float()
    lt = F.log_softmax(t32, dim=-1)
    ls = F.log_softmax(s32, dim=-1)
    pt = lt.exp()
    kl_rows = (pt * (lt - ls)).sum(-1)
    ref = kl_rows.mean().item()
    scale = (1 + torch.logsumexp(t32, -1).abs() + torch.logsumexp(s32, -1).abs()
             + (pt * (t32 - s32).abs()).sum(-1)).mean().item()
    # float32 torch is itself off by ~V * 2^-24 relative in its sums: allow both
    assert abs(loss.item() - ref) <= 2e-5 * scale, (loss.item(), ref)
    want = (ls.exp() - pt) / (B * K)
    err = (xs.grad.float() - want).abs()
    tol = 2.0 ** -8 * want.abs() + 1e-5 / (B * K) * (pt + ls.exp()) * (1 + lt.abs() + ls.abs() + kl_rows.abs()[..., None])
    assert bool((err <= tol * 1.01 + 1e-30).all()), float((err / (tol + 1e-30)).max())

    # the reference's lines, verbatim, in bf16 on the GPU
    t_logp = F.log_softmax(t / 1.0, dim=-1)
    s_logp = F.log_softmax(s / 1.0, dim=-1)
    kl_per_tok = (t_logp.exp() * (t_logp - s_logp)).sum(dim=-1)
    ref_bf16 = kl_per_tok.mean().float().item()
    u = 2.0 ** -8
    d = lt - ls
    dd = 1.01 * u * (lt.abs() + ls.abs() + d.abs())
    dp = pt * (torch.exp(u * lt.abs()) * (1 + u) - 1)
    prod = (pt + dp) * (d.abs() + dd)
    row = ((pt + dp) * dd + d.abs() * dp + u * prod).sum(-1) + V * 2.0 ** -24 * prod.sum(-1) + u * kl_rows.abs()
    assert abs(ref_bf16 - loss.item()) <= 2 * row.mean().item() + u * abs(loss.item())


def test_identical_logits_give_exact_zeros_at_full_size(gpu_available):
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(1)
    t = (4.0 * torch.randn((2, 512, 32000), device="cuda", generator=g)).to(torch.bfloat16)
    xs = t.clone().requires_grad_(True)
    xt = t.clone().requires_grad_(True)
    kl = logits_kl(xt, xs, reduction="none")
    kl.sum().backward()
    assert bool((kl == 0).all())
    assert bool((xs.grad == 0).all()) and bool((xt.grad == 0).all())


def test_student_gradient_rows_sum_to_zero_and_kl_is_nonnegative(gpu_available):
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(2)
    t = (3.0 * torch.randn((1, 512, 128256), device="cuda", generator=g)).to(torch.bfloat16)
    s = (0.7 * t.float() + torch.randn(t.shape, device="cuda", generator=g)).to(torch.bfloat16)
    xs = s.clone().requires_grad_(True)
    kl = logits_kl(t, xs, temperature=2.0, reduction="none")
    kl.sum().backward()
    assert bool((kl >= -1e-5).all())
    # sum_v (p_s - p_t) / T = 0: each row's gradient sums to 0 up to its rounding
    rows = xs.grad.float().sum(-1)
    assert float(rows.abs().max()) <= 2.0 ** -8 * float(xs.grad.float().abs().sum(-1).max()) + 1e-6


def test_deterministic(gpu_available):
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(3)
    t = torch.randn((2, 64, 50000), device="cuda", generator=g).to(torch.bfloat16)
    s = torch.randn((2, 64, 50000), device="cuda", generator=g).to(torch.bfloat16)
    out = []
    for _ in range(2):
        xs = s.clone().requires_grad_(True)
        loss = logits_kl(t, xs)
        loss.backward()
        out.append((loss.item(), xs.grad.clone()))
    assert out[0][0] == out[1][0] and torch.equal(out[0][1], out[1][1])


def test_kept_positions_as_a_strided_view(gpu_available):
    """logits[:, -K:, :] of a [B, T, V] tensor (rows of the view are strided)
    gives the same results bit for bit as a contiguous copy; [K, V] input works."""
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(4)
    full_t = torch.randn((2, 40, 4096), device="cuda", generator=g).to(torch.bfloat16)
    full_s = torch.randn((2, 40, 4096), device="cuda", generator=g).to(torch.bfloat16)
    vt, vs = full_t[:, -16:, :], full_s[:, -16:, :].detach().requires_grad_(True)
    assert not vt.is_contiguous()
    l1 = logits_kl(vt, vs)
    l1.backward()
    cs = vs.detach().contiguous().requires_grad_(True)
    l2 = logits_kl(vt.contiguous(), cs)
    l2.backward()
    assert l1.item() == l2.item() and torch.equal(vs.grad, cs.grad)
    l3 = logits_kl(vt[0], vs.detach()[0])
    l4 = logits_kl(vt[:1], vs.detach()[:1])
    assert l3.item() == l4.item()


def test_edge_cases(gpu_available):
    from linearard_amd.logits_kl import logits_kl

    g = torch.Generator(device="cuda").manual_seed(5)
    one = (4.0 * torch.randn((2, 3, 1), device="cuda", generator=g)).to(torch.bfloat16)
    xs = (4.0 * torch.randn((2, 3, 1), device="cuda", generator=g)).to(torch.bfloat16).requires_grad_(True)
    loss = logits_kl(one, xs)
    loss.backward()
    # one word: both distributions are 1 and the KL 0, up to the float32
    # roundings of KL = E[q_t - q_s] - lse_t + lse_s (|q| <= 16 here)
    assert abs(loss.item()) <= 1e-5 and float(xs.grad.float().abs().max()) <= 1e-6
    empty = torch.empty((1, 0, 100), device="cuda", dtype=torch.bfloat16)
    assert math.isnan(logits_kl(empty, empty).item())  # the mean of no positions, as torch gives
    novocab = torch.empty((1, 4, 0), device="cuda", dtype=torch.bfloat16)
    assert logits_kl(novocab, novocab).item() == 0.0
    with pytest.raises(AssertionError):
        logits_kl(one, one.float())
    with pytest.raises(RuntimeError):
        logits_kl(one, one, temperature=0.0)
