"""Parity gates shared by the GPU tests (the bars are stated here, once).

The bars are the north star's for 16-bit inputs:
  loss:      |got - ref| <= 1e-3 |ref|
  gradients: max|got - ref| <= 2e-2 max|ref|      (the L2-relative error
             ||got - ref|| / ||ref|| is reported next to it)
against the float64 oracle (oracle/attn_kl.py) on the same inputs.  A
reference that is exactly zero (identical relations, one-key rows) needs an
exactly zero result.

Where float32 arithmetic itself cannot meet a bar (a loss that is a small
difference of large per-row terms), a test passes the float32 eager oracle's
value on the same inputs (oracle/attn_kl_torch.py) and the bar becomes
FP32_MULTIPLE times that oracle's own deviation from the float64 one, never
less than the plain bar.  Such checks are marked "fp32x2" in the table.

Every check records what it achieved; conftest.py prints the table at the
end of the session, so the errors are visible in every run, not only when a
check fails.
"""

import numpy as np

LOSS_REL = 1e-3
GRAD_MAX_REL = 2e-2
FP32_MULTIPLE = 2.0

# (test case, quantity, max-relative or relative error, L2-relative error or None, bar)
RESULTS = []


def _rel(a, b):
    return abs(a - b) / max(abs(b), 1e-30)


def check_loss(got, ref, case, bar=LOSS_REL, fp32=None):
    """Loss gate: relative error <= bar (1e-3 unless stated by the caller).

    ``fp32``: the float32 eager oracle's loss on the same inputs; the bar is
    then max(bar, FP32_MULTIPLE * its relative deviation)."""
    got, ref = float(got), float(ref)
    if ref == 0.0:
        RESULTS.append((case, "loss", abs(got), None, 0.0))
        assert got == 0.0, (case, got, ref)
        return 0.0
    name = "loss"
    if fp32 is not None:
        fp32_bar = FP32_MULTIPLE * _rel(float(fp32), ref)
        if fp32_bar > bar:
            bar, name = fp32_bar, "loss fp32x2"
    err = _rel(got, ref)
    RESULTS.append((case, name, err, None, bar))
    assert err <= bar, f"{case}: loss {got!r} vs {ref!r}: relative error {err:.3e} > {bar:.1e}"
    return err


def check_grad(got, ref, case, name="dX", bar=GRAD_MAX_REL):
    """Gradient gate: max|diff| <= bar max|ref|; the L2-relative error is recorded too."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (case, got.shape, ref.shape)
    diff = got - ref
    scale = np.abs(ref).max()
    if scale == 0.0:
        RESULTS.append((case, name, float(np.abs(got).max()), None, 0.0))
        assert not np.any(got), f"{case}: {name} must be exactly 0"
        return 0.0, 0.0
    maxrel = float(np.abs(diff).max() / scale)
    l2 = float(np.linalg.norm(diff) / np.linalg.norm(ref))
    RESULTS.append((case, name, maxrel, l2, bar))
    assert maxrel <= bar, f"{case}: {name} max|diff|/max|ref| = {maxrel:.3e} > {bar:.1e} (L2-relative {l2:.3e})"
    return maxrel, l2


def summary_lines():
    if not RESULTS:
        return []
    out = ["achieved errors against the float64 oracle (max-rel: max|diff|/max|ref| for gradients, "
           "relative error for losses; bar in the last column)"]
    width = max(len(r[0]) for r in RESULTS)
    for case, name, err, l2, bar in RESULTS:
        l2s = "" if l2 is None else f"  l2 {l2:.2e}"
        out.append(f"  {case:<{width}}  {name:<11} {err:.2e}{l2s:<14}  bar {bar:.1e}")
    worst = {}
    for case, name, err, l2, bar in RESULTS:
        key = "loss" if name.startswith("loss") else "grad"
        if bar > 0:
            worst[key] = max(worst.get(key, 0.0), err / bar)
    out.append("  worst fraction of the bar: " + ", ".join(f"{k} {v:.3f}" for k, v in sorted(worst.items())))
    return out
