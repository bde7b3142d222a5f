"""Rows whose logits keep rising in the kernels' key order, so the online
softmax raises its running maxima again and again (the
rare branch of the lazy maxima: a sub-block whose sums pass 2^20 is rescaled
and recomputed), checked through the autograd boundary against the float64
oracle (kernel_A.py:72-159, kernel_B.py:105-218, kernel_C.py:121-261).

Channel 0 of every token carries a ramp g(j) that dominates the logits,
S_ij = a (g(i) g(j) + small noise): non-causal launches read key tiles in
ascending order, so the ramp rises with j; causal launches read the diagonal
tile first and go down, so the ramp falls with j.  With T = 256 and logits
up to 400 nats, a row i gains about 72 (i+1)/T (non-causal) or 72 (T-i)/T
(causal) log2 units per sub-block: more than 20 on most rows, which take
the rescale branch on every sub-block (non-causal) or every 64-key tile
(causal: the two sub-blocks of a tile are still read in ascending order,
so the second one rises no further).  The teacher's ramp is steeper than
the student's, so the two softmaxes differ and the KL is far above the fp32
floor of the gate.
"""

import math

import numpy as np
import pytest

from oracle import attn_kl as O
from tests._inputs import to_dev
from tests._tolerance import check_grad, check_loss

pytestmark = pytest.mark.gpu

T = 256


def _ramp_pair(D, causal, dtype, seed):
    rng = np.random.default_rng(seed)
    j = np.arange(T, dtype=np.float64)
    ramp = (j + 1) / T if not causal else (T - j) / T
    noise = 0.3 * rng.standard_normal((1, 2, T, D))
    xt = noise.copy()
    xs = noise + 0.05 * rng.standard_normal(noise.shape)
    # a * c^2 = 400 nats at the top of the teacher's ramp
    c = math.sqrt(400.0 * math.sqrt(D))
    xt[..., 0] = c * ramp
    xs[..., 0] = 0.85 * c * ramp
    return O.round_to(xs.astype(np.float32), dtype), O.round_to(xt.astype(np.float32), dtype)


@pytest.mark.parametrize("D,causal", [(128, False), (128, True), (64, True), (256, False), (256, True)])
def test_rising_logits_take_the_rescale_path(gpu_available, D, causal):
    from linearard_amd.attention_KL import attn_kl_align

    dtype = "bf16"
    xs, xt = _ramp_pair(D, causal, dtype, seed=D + causal)
    a = 1 / math.sqrt(D)
    # the premise: per 32 keys the top rows' logits rise by more than 20 log2 units
    g = xt[0, 0, :, 0].astype(np.float64)
    top = 128 if causal else T - 1  # causal: row 128's keys run from its diagonal down to j = 0
    step_bits = a * abs(g[top]) * abs(g[0] - g[32]) / math.log(2)
    assert step_bits > 20, step_bits
    x_s = to_dev(xs, dtype, requires_grad=True)
    loss = attn_kl_align(x_s, x_s, to_dev(xt, dtype), to_dev(xt, dtype), causal=causal, sm_scale_s=a, sm_scale_t=a)
    loss.backward()
    rl, rdx, _, _, _ = O.attn_kl_align(xs, xs, xt, xt, None, causal, a, a, self_relation=True)
    assert rl > 1e-2 * 2 * T, rl  # a real KL, not the fp32 floor of the gate
    assert np.isfinite(loss.item())
    check_loss(loss.item(), rl, f"rescale-D{D}-c{int(causal)}")
    g_dx = x_s.grad.float().cpu().numpy()
    assert np.isfinite(g_dx).all()
    check_grad(g_dx, rdx, f"rescale-D{D}-c{int(causal)}")
