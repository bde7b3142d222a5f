"""GPU parity of the three reference stages against the CPU oracle.

The case matrices replay the reference tests' shapes (test_kernel_A.py:208-229,
test_kernel_B.py:245-266, test_kernel_C.py:255-310) with CPU-seeded inputs.
Tolerances: the reference's own (fp16 rtol 1e-2 / atol 2e-2, bf16 2e-2 / 3e-2)
are the outer bar; the kernels are held to much tighter ones below because
they consume exactly the oracle's rounded inputs.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attn_kl as O
from tests._inputs import make_mask, mask_to_dev, randn, to_dev

pytestmark = pytest.mark.gpu

DIMS = O.SUPPORTED_HEAD_DIMS


def _a_cases():
    cases = []
    for D in DIMS:
        for hq, hkv in ((8, 8), (8, 4)):
            cases.append(("f16", True, None, 2, hq, hkv, 33, D))
            cases.append(("f16", False, 0.3, 2, hq, hkv, 33, D))
    cases += [
        ("f16", True, 0.7, 2, 8, 2, 33, 8),
        ("f16", False, 0.3, 2, 16, 4, 33, 16),
        ("bf16", True, None, 2, 8, 8, 33, 8),
        ("bf16", False, 0.3, 2, 8, 4, 33, 256),
        ("f16", True, None, 1, 8, 4, 127, 64),
        ("f16", False, 0.3, 1, 8, 2, 127, 64),
        ("bf16", True, 0.2, 1, 4, 4, 300, 128),
        ("bf16", True, None, 1, 2, 2, 1, 128),
    ]
    return cases


@pytest.mark.parametrize("dtype,causal,ratio,B,hq,hkv,T,D", _a_cases())
def test_stage_a_lse(gpu_available, dtype, causal, ratio, B, hq, hkv, T, D):
    from linearard_amd.attention_KL import lse_stats

    rng = np.random.default_rng(1000 + D + T + hq)
    q = randn(rng, (B, hq, T, D), dtype)
    k = randn(rng, (B, hkv, T, D), dtype)
    mask = None if ratio is None else make_mask(rng, B, T, ratio)
    scale = 1.0 / math.sqrt(D)
    out = lse_stats(to_dev(q, dtype), to_dev(k, dtype), mask_to_dev(mask), causal, scale)
    ref = O.lse_stats(q, k, mask, causal, scale)
    got = out.cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)


def _bc_cases():
    cases = [("f16", True, None, 1, 8, 8, 8, 16, ds, dt) for ds in DIMS for dt in DIMS]
    cases += [
        ("f16", False, 0.3, 2, 8, 4, 2, 33, 8, 128),
        ("f16", True, 0.7, 2, 8, 2, 4, 33, 128, 8),
        ("f16", False, 0.3, 2, 16, 4, 4, 33, 16, 32),
        ("bf16", True, None, 2, 8, 8, 8, 33, 64, 64),
        ("f16", False, 0.3, 1, 8, 4, 2, 127, 64, 128),
        ("bf16", True, 0.1, 1, 4, 2, 4, 257, 128, 128),
    ]
    return cases


def _two_sided_inputs(rng, dtype, B, hq, hks, hkt, T, ds, dt, ratio):
    qs = randn(rng, (B, hq, T, ds), dtype)
    ks = randn(rng, (B, hks, T, ds), dtype)
    qt = randn(rng, (B, hq, T, dt), dtype)
    kt = randn(rng, (B, hkt, T, dt), dtype)
    mask = None if ratio is None else make_mask(rng, B, T, ratio)
    return qs, ks, qt, kt, mask


@pytest.mark.parametrize("dtype,causal,ratio,B,hq,hks,hkt,T,ds,dt", _bc_cases())
def test_stage_b_kl_forward(gpu_available, dtype, causal, ratio, B, hq, hks, hkt, T, ds, dt):
    from linearard_amd.attention_KL import kl_forward, lse_stats

    rng = np.random.default_rng(2000 + ds * 7 + dt + T)
    qs, ks, qt, kt, mask = _two_sided_inputs(rng, dtype, B, hq, hks, hkt, T, ds, dt, ratio)
    ss, st = 1 / math.sqrt(ds), 1 / math.sqrt(dt)
    d = [to_dev(x, dtype) for x in (qs, ks, qt, kt)]
    m = mask_to_dev(mask)
    lse_s = lse_stats(d[0], d[1], m, causal, ss)
    lse_t = lse_stats(d[2], d[3], m, causal, st)
    out = float(kl_forward(d[0], d[1], lse_s, d[2], d[3], lse_t, m, causal, ss, st).item())
    # stage B in isolation: the oracle consumes the kernel's lse (test_kernel_B.py:281-285)
    ref_b = O.kl_forward(qs, ks, lse_s.cpu().numpy(), qt, kt, lse_t.cpu().numpy(), mask, causal, ss, st)
    # end to end against the oracle's own lse
    ref = O.attn_kl_align(qs, ks, qt, kt, mask, causal, ss, st)[0]
    scale = max(1.0, abs(ref))
    assert abs(out - ref_b) <= 1e-4 * scale, (out, ref_b)
    assert abs(out - ref) <= 1e-4 * scale, (out, ref)


@pytest.mark.parametrize("dtype,causal,ratio,B,hq,hks,hkt,T,ds,dt", _bc_cases() + [
    ("f16", True, 0.3, 2, 16, 4, 8, 33, 32, 64),  # test_kernel_C.py:255-286 dk aggregation stress
])
def test_stage_c_kl_backward(gpu_available, dtype, causal, ratio, B, hq, hks, hkt, T, ds, dt):
    from linearard_amd.attention_KL import kl_backward, lse_stats

    rng = np.random.default_rng(3000 + ds * 7 + dt + T)
    qs, ks, qt, kt, mask = _two_sided_inputs(rng, dtype, B, hq, hks, hkt, T, ds, dt, ratio)
    ss, st = 1 / math.sqrt(ds), 1 / math.sqrt(dt)
    d = [to_dev(x, dtype) for x in (qs, ks, qt, kt)]
    m = mask_to_dev(mask)
    lse_s = lse_stats(d[0], d[1], m, causal, ss)
    lse_t = lse_stats(d[2], d[3], m, causal, st)
    dq, dk = kl_backward(d[0], d[1], lse_s, d[2], d[3], lse_t, m, causal, ss, st)
    assert dq.dtype == torch.float32 and dk.dtype == torch.float32
    assert tuple(dq.shape) == (B, hq, T, ds) and tuple(dk.shape) == (B, hks, T, ds)
    ls, lt = lse_s.cpu().numpy(), lse_t.cpu().numpy()
    # emulate the D cast of kernel_C.py:233: agreement to float32 rounding noise
    rq, rk = O.kl_backward(qs, ks, ls, qt, kt, lt, mask, causal, ss, st, d_cast=dtype)
    gq, gk = dq.cpu().numpy(), dk.cpu().numpy()
    for got, ref in ((gq, rq), (gk, rk)):
        denom = max(np.abs(ref).max(), 1e-6)
        assert np.abs(got - ref).max() <= 5e-3 * denom
    # the reference test's own tolerance against the exact (uncast) gradient
    eq, ek = O.kl_backward(qs, ks, ls, qt, kt, lt, mask, causal, ss, st)
    rtol, atol = (1e-2, 2e-2) if dtype == "f16" else (2e-2, 3e-2)
    np.testing.assert_allclose(gq, eq, rtol=rtol, atol=atol)
    np.testing.assert_allclose(gk, ek, rtol=rtol, atol=atol)


@pytest.mark.parametrize("causal", [True, False])
def test_stages_on_long_padded_sequences(gpu_available, causal):
    """Stages A, B, C at T = 700 (ragged against the 32- and 128-row tiles)
    with GQA on both sides, Ds != Dt, and a mask that leaves most tiles whole
    (the kernels' full-tile form) and some partial (a padded tail in one
    sequence; left padding and scattered holes in the other)."""
    from linearard_amd.attention_KL import kl_backward, kl_forward, lse_stats

    dtype, B, hq, hks, hkt, T, ds, dt = "bf16", 2, 4, 2, 4, 700, 64, 128
    rng = np.random.default_rng(4100 + int(causal))
    qs, ks, qt, kt, _ = _two_sided_inputs(rng, dtype, B, hq, hks, hkt, T, ds, dt, None)
    mask = np.ones((B, T), np.int32)
    mask[0, T - 150:] = 0
    mask[1, :40] = 0
    mask[1, rng.choice(np.arange(40, T), size=T // 10, replace=False)] = 0
    ss, st = 1 / math.sqrt(ds), 1 / math.sqrt(dt)
    d = [to_dev(x, dtype) for x in (qs, ks, qt, kt)]
    m = mask_to_dev(mask)
    lse_s = lse_stats(d[0], d[1], m, causal, ss)
    lse_t = lse_stats(d[2], d[3], m, causal, st)
    np.testing.assert_allclose(lse_s.cpu().numpy(), O.lse_stats(qs, ks, mask, causal, ss), rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(lse_t.cpu().numpy(), O.lse_stats(qt, kt, mask, causal, st), rtol=2e-5, atol=2e-5)
    out = float(kl_forward(d[0], d[1], lse_s, d[2], d[3], lse_t, m, causal, ss, st).item())
    ls, lt = lse_s.cpu().numpy(), lse_t.cpu().numpy()
    ref_b = O.kl_forward(qs, ks, ls, qt, kt, lt, mask, causal, ss, st)
    assert abs(out - ref_b) <= 1e-4 * max(1.0, abs(ref_b)), (out, ref_b)
    dq, dk = kl_backward(d[0], d[1], lse_s, d[2], d[3], lse_t, m, causal, ss, st)
    rq, rk = O.kl_backward(qs, ks, ls, qt, kt, lt, mask, causal, ss, st, d_cast=dtype)
    for got, ref in ((dq.cpu().numpy(), rq), (dk.cpu().numpy(), rk)):
        assert np.abs(got - ref).max() <= 5e-3 * max(np.abs(ref).max(), 1e-6)
    # padded tokens: no gradient in either output
    dead = mask == 0
    assert not dq.cpu().numpy()[np.broadcast_to(dead[:, None, :, None], dq.shape)].any()
    assert not dk.cpu().numpy()[np.broadcast_to(dead[:, None, :, None], dk.shape)].any()


@pytest.mark.parametrize("kind", ["bool", "u8", "i32", "i64"])
def test_mask_dtypes_and_cpu_mask(gpu_available, kind):
    from linearard_amd.attention_KL import lse_stats

    rng = np.random.default_rng(77)
    q = randn(rng, (2, 4, 65, 32), "bf16")
    mask = make_mask(rng, 2, 65, 0.4, kind)
    ref = O.lse_stats(q, q, mask, True, 0.2)
    dev = lse_stats(to_dev(q, "bf16"), to_dev(q, "bf16"), mask_to_dev(mask), True, 0.2)
    cpu_mask = lse_stats(to_dev(q, "bf16"), to_dev(q, "bf16"), torch.from_numpy(np.ascontiguousarray(mask)), True, 0.2)
    np.testing.assert_allclose(dev.cpu().numpy(), ref, rtol=2e-5, atol=2e-5)
    assert torch.equal(dev, cpu_mask)


def test_stage_b_is_deterministic(gpu_available):
    from linearard_amd.attention_KL import kl_forward, lse_stats

    rng = np.random.default_rng(5)
    x = to_dev(randn(rng, (1, 8, 1000, 128), "bf16"), "bf16")
    y = to_dev(randn(rng, (1, 8, 1000, 128), "bf16"), "bf16")
    ls, lt = lse_stats(x, x), lse_stats(y, y)
    outs = [kl_forward(x, x, ls, y, y, lt).item() for _ in range(3)]
    assert outs[0] == outs[1] == outs[2]


def test_wrapper_validation_messages(gpu_available):
    from linearard_amd.attention_KL import kl_forward, lse_stats

    q = torch.zeros((1, 2, 8, 16), dtype=torch.float64, device="cuda")
    with pytest.raises(AssertionError, match="q dtype supports only fp16/bf16/fp32"):
        lse_stats(q, q)
    h = torch.zeros((1, 3, 8, 16), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((1, 2, 8, 16), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(AssertionError, match="Hq must be divisible by Hkv"):
        lse_stats(h, k)
    d = torch.zeros((1, 2, 8, 24), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(AssertionError, match="D is not in the supported set"):
        lse_stats(d, d)
    g = torch.zeros((1, 2, 8, 16), dtype=torch.bfloat16, device="cuda")
    lse = torch.zeros((1, 2, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(AssertionError, match="attn_mask shape must be"):
        kl_forward(g, g, lse, g, g, lse, attn_mask=torch.ones((1, 7), dtype=torch.int32, device="cuda"))
    with pytest.raises(AssertionError, match="sm_scale_s must be a scalar"):
        kl_forward(g, g, lse, g, g, lse, sm_scale_s=torch.tensor(0.1))
