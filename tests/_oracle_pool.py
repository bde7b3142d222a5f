"""The chunked float64 oracle over several heads at once, in worker
processes started fresh (spawn) that import numpy and oracle.attn_kl only:
no torch and no GPU in the workers.  Test infrastructure."""

from __future__ import annotations

import multiprocessing as mp
import os

import numpy as np

from oracle import attn_kl as O

_THREAD_VARS = ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")


def _head(args):
    xs, xt, a, mask_b = args
    loss, dx, _, _, kl_rows = O.self_relation_chunked(xs, xt, True, a, a, mask=mask_b, chunk=1024,
                                                      dtype=np.float64)
    return loss, dx, float(kl_rows.min())


def oracle_heads(jobs, workers=8, threads=2):
    """[(xs [n, d], xt [n, d], scale, mask row or None)] -> [(loss, dX, min row KL)]
    of each causal self relation, float64."""
    saved = {k: os.environ.get(k) for k in _THREAD_VARS}
    for k in _THREAD_VARS:
        os.environ[k] = str(threads)
    try:
        with mp.get_context("spawn").Pool(max(1, min(len(jobs), workers))) as pool:
            return pool.map(_head, jobs)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
