"""Parity gates shared by the GPU tests (tolerances are stated here, once)."""

import numpy as np


def _rel(a, b):
    return abs(a - b) / max(abs(b), 1e-30)


def _logit_bound(*pairs):
    """max |logit| over the given (x, scale) relations: a * max_i |x_i|^2 bounds
    |a x_i . x_j| by Cauchy-Schwarz (for q != k, a * max|q| * max|k|)."""
    out = 1.0
    for q, k, a in pairs:
        nq = np.sqrt((np.asarray(q, np.float64) ** 2).sum(-1)).max()
        nk = np.sqrt((np.asarray(k, np.float64) ** 2).sum(-1)).max()
        out = max(out, a * nq * nk)
    return out


def _loss_ok(got, ref, rows, logit=16.0):
    """Loss gate: relative error <= 1e-3 (BASELINE parity bar) plus, per row,
    a few fp32 ulps of the largest logit -- the resolution of any fp32
    log-domain softmax (logits are rounded to fp32 before they are
    exponentiated).  It only matters when the whole loss is ~1e-6 per row,
    e.g. a single-key row whose two distributions are both point masses."""
    return abs(got - ref) <= 1e-3 * abs(ref) + rows * logit * 2.0 ** -21


def _grad_ok(got, ref, x, a, logit):
    """Gradient gate: max|diff| <= 2e-2 * max|ref| (BASELINE bar) plus the fp32
    resolution of P (relative error |logit| 2^-23 per entry) propagated
    through a * sum_j D_ij x_j <= a max|x| |logit| 2^-22 (2^-20 with margin);
    that floor only matters for references that are exactly zero."""
    floor = a * np.abs(x).max() * logit * 2.0 ** -20
    return np.abs(got - ref).max() <= 2e-2 * np.abs(ref).max() + floor
