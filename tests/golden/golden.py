"""Loader of the golden fixtures written by make_golden.py."""

from __future__ import annotations

import os

import numpy as np

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attn_kl_golden.npz")


def _floats(bits, dtype):
    bits = np.asarray(bits, np.uint16)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def load():
    """{case name: dict of inputs (float32 values), flags and expected outputs}."""
    z = np.load(PATH, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    cases = {}
    for n in names:
        g = {k.split("/")[1]: z[k] for k in z.files if k.startswith(n + "/")}
        dtype = str(g["dtype"])
        B, Hq, Hkv_s, Hkv_t, T, Ds, Dt, causal, self_rel = (int(v) for v in g["meta"])
        qs = _floats(g["qs"], dtype)
        qt = _floats(g["qt"], dtype)
        ks = qs if self_rel else _floats(g["ks"], dtype)
        kt = qt if self_rel else _floats(g["kt"], dtype)
        cases[n] = {"qs": qs, "ks": ks, "qt": qt, "kt": kt, "mask": g.get("mask"), "dtype": dtype,
                    "causal": bool(causal), "self_relation": bool(self_rel), "loss": float(g["loss"]),
                    "lse_s": g["lse_s"], "lse_t": g["lse_t"], "dq": g["dq"], "dk": g["dk"]}
    return cases
