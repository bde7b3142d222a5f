"""Writes tests/golden/attn_kl_golden.npz: fixed inputs and expected outputs
of the attention-relation KL path, computed by the CPU oracle (oracle/attn_kl.py).

The reference ships no golden vectors (its tests compare against in-file
fp32 references), so these fixtures come from the oracle, which is pinned
by independent checks (tests/test_oracle.py).  Each case stores its inputs
as 16-bit bit patterns (exactly the values the kernels read) plus

    loss            float64  the 0-d SUM of per-row KL (integration.py:70-73)
    lse_s, lse_t    float64  stage A of both relations (kernel_A.py:157-158)
    dq, dk          float32  stage C with D cast to the input dtype (kernel_C.py:232-233)

Self-relation cases (q is k, the train.py call) store ks / kt implicitly:
they are qs / qt.

Regenerate with  `python tests/golden/make_golden.py`  (deterministic).
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attn_kl as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attn_kl_golden.npz")

# name: (B, Hq, Hkv_s, Hkv_t, T, Ds, Dt, dtype, causal, mask ratio or None, self relation, seed)
CASES = {
    "self_causal_bf16_d16": (1, 2, 2, 2, 37, 16, 16, "bf16", True, None, True, 11),
    "self_causal_f16_d8": (1, 2, 2, 2, 40, 8, 8, "f16", True, None, True, 12),
    "self_masked_bf16_d128": (2, 1, 1, 1, 48, 128, 128, "bf16", True, 0.3, True, 13),
    "gqa_masked_f16_ds32_dt16": (2, 4, 2, 1, 29, 32, 16, "f16", True, 0.25, False, 14),
    "noncausal_bf16_d64": (1, 2, 2, 2, 48, 64, 64, "bf16", False, 0.2, False, 15),
}


def bits(x, dtype):
    """16-bit patterns of float32 values already rounded to `dtype`."""
    x = np.ascontiguousarray(x, np.float32)
    if dtype == "bf16":
        return (x.view(np.uint32) >> 16).astype(np.uint16)
    return x.astype(np.float16).view(np.uint16)


def make_case(B, Hq, Hkv_s, Hkv_t, T, Ds, Dt, dtype, causal, ratio, self_rel, seed):
    rng = np.random.default_rng(seed)

    def randn(shape, scale=1.0):
        return O.round_to(rng.standard_normal(shape).astype(np.float32) * scale, dtype)

    qs = randn((B, Hq, T, Ds))
    qt = randn((B, Hq, T, Dt), 1.5)
    if self_rel:
        ks, kt = qs, qt
    else:
        ks = randn((B, Hkv_s, T, Ds))
        kt = randn((B, Hkv_t, T, Dt), 1.5)
    mask = None
    if ratio is not None:
        mask = (rng.random((B, T)) > ratio).astype(np.uint8)
        mask[:, 0] = 1
    loss, dq, dk, lse_s, lse_t = O.attn_kl_align(qs, ks, qt, kt, mask, causal, None, None,
                                                 self_relation=False, d_cast=dtype)
    case = {"qs": bits(qs, dtype), "qt": bits(qt, dtype),
            "loss": np.float64(loss), "lse_s": np.asarray(lse_s, np.float64), "lse_t": np.asarray(lse_t, np.float64),
            "dq": np.asarray(dq, np.float32), "dk": np.asarray(dk, np.float32),
            "meta": np.array([B, Hq, Hkv_s, Hkv_t, T, Ds, Dt, int(causal), int(self_rel)], np.int64),
            "dtype": np.array(dtype)}
    if not self_rel:
        case["ks"] = bits(ks, dtype)
        case["kt"] = bits(kt, dtype)
    if mask is not None:
        case["mask"] = mask
    return case


def main():
    arrays = {}
    for name, spec in CASES.items():
        for key, val in make_case(*spec).items():
            arrays[f"{name}/{key}"] = val
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {len(CASES)} cases, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
