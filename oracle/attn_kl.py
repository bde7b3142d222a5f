"""CPU oracle for the attention-relation KL path (numpy).

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / CPU baseline, never as the
code path being measured or shipped.

It restates the reference algorithm of ``kernels/attention_KL`` in plain
numpy, in float64 unless a caller asks for float32:

* ``lse_stats``      -- stage A, ``kernel_A.py:72-159`` (masking, online
                        log-sum-exp, 0 for invalid rows, -inf for empty rows);
                        the reference's own fp32 oracle is
                        ``test_kernel_A.py:62-98``.
* ``kl_forward``     -- stage B, ``kernel_B.py:105-218`` (row_has_lse gate
                        ``:140-143``, zeroed log-probs ``:206-210``, sum of
                        ``p_t (l_t - l_s)`` ``:213-217``); reference oracle
                        ``test_kernel_B.py:63-106``.
* ``kl_backward``    -- stage C, ``kernel_C.py:121-261`` (D = p_s - p_t on the
                        valid set ``:224-232``, optional cast of D to the input
                        dtype ``:233``, dq = a_s D K_s ``:236-239``, dk summed
                        over the GQA group ``:242-253``); reference oracle
                        ``test_kernel_C.py:64-117``.
* ``attn_kl_align``  -- ``integration.py:6-73``: stage A twice, stage B, and
                        the stage C gradients scaled by ``dloss``; for a
                        self relation (q is k) the two gradients are summed.
* ``materialized_kl``-- the independent log_softmax formulation of
                        ``integration.py:102-127``.
* ``self_relation_chunked`` -- a linear-memory (row-chunked) float32/64
                        restatement of the self relation fwd+bwd used for
                        large n (CPU baseline and size-independent checks).

Pinning (see tests/test_oracle.py): every function is checked against an
independent formulation -- pure-Python ``math.fsum`` brute force at tiny
sizes, ``scipy.special.logsumexp`` / ``scipy.special.rel_entr``, closed forms
(causal row 0, KL == 0 for identical inputs), central finite differences of
the loss, and torch float64 autograd of the materialised loss.
"""

from __future__ import annotations

import math

import numpy as np

SUPPORTED_HEAD_DIMS = (8, 16, 32, 64, 128, 256)  # kernel_A.py:18

_NEG_INF = -np.inf


# ---------------------------------------------------------------------------
# dtype emulation
# ---------------------------------------------------------------------------

def round_bf16(x):
    """Round float32 values to bfloat16 (round-to-nearest-even), as float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def round_f16(x):
    """Round float32 values to float16 (round-to-nearest-even), as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype):
    """Cast-and-back emulation of ``tensor.to(dtype)`` for dtype names."""
    if dtype in ("bf16", "bfloat16"):
        return round_bf16(x)
    if dtype in ("f16", "fp16", "float16"):
        return round_f16(x)
    if dtype in ("f32", "fp32", "float32", None):
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


# ---------------------------------------------------------------------------
# validity sets (Appendix of the reference semantics)
# ---------------------------------------------------------------------------

def _mask_bool(mask, B, T):
    if mask is None:
        return np.ones((B, T), dtype=bool)
    m = np.asarray(mask)
    return m != 0


def validity(B, T, mask, causal):
    """Return (row_valid [B,T], valid [B,1,T,T]).

    ``row(b,i) = i<T and mask[b,i] != 0``; ``col`` likewise;
    ``V = row & col & (j <= i if causal)``  (kernel_A.py:91-97, :115-120,
    :139-141).
    """
    mb = _mask_bool(mask, B, T)
    valid = mb[:, None, :, None] & mb[:, None, None, :]
    if causal:
        valid = valid & np.tril(np.ones((T, T), dtype=bool))[None, None]
    return mb, valid


def _expand_kv(k, Hq):
    """GQA head map kv(h) = h // (Hq / Hkv)  (kernel_A.py:77)."""
    Hkv = k.shape[1]
    if Hq % Hkv != 0:
        raise ValueError("Hq must be divisible by Hkv")
    g = Hq // Hkv
    return k[:, np.arange(Hq) // g]


def relation_logits(q, k, scale, dtype=np.float64):
    """S[b,h,i,j] = scale * q[b,h,i] . k[b,kv(h),j] (exact products, wide sum)."""
    q = np.asarray(q, dtype=dtype)
    k = _expand_kv(np.asarray(k, dtype=dtype), q.shape[1])
    return np.matmul(q, np.swapaxes(k, -1, -2)) * dtype(scale)


# ---------------------------------------------------------------------------
# stage A: row log-sum-exp
# ---------------------------------------------------------------------------

def lse_stats(q, k, mask=None, causal=True, sm_scale=None):
    """Stage A (kernel_A.py:72-159): per-row LSE over the valid set.

    Invalid query rows get 0 (``:157-158``); a valid row with no valid
    column gets -inf.
    """
    q = np.asarray(q, dtype=np.float64)
    B, Hq, T, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)  # kernel_A.py:224-225
    S = relation_logits(q, k, sm_scale)
    rows, valid = validity(B, T, mask, causal)
    Sm = np.where(valid, S, _NEG_INF)
    m = Sm.max(axis=-1)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    e = np.where(valid, np.exp(Sm - m_safe[..., None]), 0.0)
    r = e.sum(axis=-1)
    with np.errstate(divide="ignore"):
        lse = m_safe + np.log(r)
    lse = np.where(r > 0, lse, _NEG_INF)
    lse = np.where(rows[:, None, :], lse, 0.0)
    return lse


# ---------------------------------------------------------------------------
# stage B: KL forward given the two LSE vectors
# ---------------------------------------------------------------------------

def _row_ok(rows, lse_s, lse_t):
    """ok(i) = row & lse_s != -inf & lse_t != -inf  (kernel_B.py:140-141)."""
    return rows[:, None, :] & (lse_s != _NEG_INF) & (lse_t != _NEG_INF)


def kl_rows(qs, ks, lse_s, qt, kt, lse_t, mask=None, causal=True,
            sm_scale_s=None, sm_scale_t=None):
    """Per-row KL terms [B,Hq,T] of stage B (kernel_B.py:206-216)."""
    qs = np.asarray(qs, dtype=np.float64)
    qt = np.asarray(qt, dtype=np.float64)
    B, Hq, T, Ds = qs.shape
    Dt = qt.shape[3]
    sm_scale_s = 1.0 / math.sqrt(Ds) if sm_scale_s is None else sm_scale_s
    sm_scale_t = 1.0 / math.sqrt(Dt) if sm_scale_t is None else sm_scale_t
    lse_s = np.asarray(lse_s, dtype=np.float64)
    lse_t = np.asarray(lse_t, dtype=np.float64)
    rows, valid = validity(B, T, mask, causal)
    ok = _row_ok(rows, lse_s, lse_t)
    valid = valid & ok[..., None]
    lse_s_safe = np.where(lse_s == _NEG_INF, 0.0, lse_s)
    lse_t_safe = np.where(lse_t == _NEG_INF, 0.0, lse_t)
    ls = np.where(valid, relation_logits(qs, ks, sm_scale_s) - lse_s_safe[..., None], 0.0)
    lt = np.where(valid, relation_logits(qt, kt, sm_scale_t) - lse_t_safe[..., None], 0.0)
    pt = np.where(valid, np.exp(lt), 0.0)
    acc = (pt * (lt - ls)).sum(axis=-1)
    return np.where(ok, acc, 0.0)


def kl_forward(qs, ks, lse_s, qt, kt, lse_t, mask=None, causal=True,
               sm_scale_s=None, sm_scale_t=None):
    """Stage B (kernel_B.py:105-218): the SUM over rows, as a float."""
    return float(kl_rows(qs, ks, lse_s, qt, kt, lse_t, mask, causal,
                         sm_scale_s, sm_scale_t).sum())


# ---------------------------------------------------------------------------
# stage C: gradients given the two LSE vectors
# ---------------------------------------------------------------------------

def kl_backward(qs, ks, lse_s, qt, kt, lse_t, mask=None, causal=True,
                sm_scale_s=None, sm_scale_t=None, d_cast=None):
    """Stage C (kernel_C.py:121-261): returns (dq [B,Hq,T,Ds], dk [B,Hkv_s,T,Ds]).

    ``d_cast`` in {None, 'bf16', 'f16'} emulates ``dval.to(qs.dtype)``
    (kernel_C.py:233); None keeps D exact (float64).
    """
    qs = np.asarray(qs, dtype=np.float64)
    ks = np.asarray(ks, dtype=np.float64)
    qt = np.asarray(qt, dtype=np.float64)
    B, Hq, T, Ds = qs.shape
    Hkv_s = ks.shape[1]
    Dt = qt.shape[3]
    sm_scale_s = 1.0 / math.sqrt(Ds) if sm_scale_s is None else sm_scale_s
    sm_scale_t = 1.0 / math.sqrt(Dt) if sm_scale_t is None else sm_scale_t
    lse_s = np.asarray(lse_s, dtype=np.float64)
    lse_t = np.asarray(lse_t, dtype=np.float64)
    rows, valid = validity(B, T, mask, causal)
    ok = _row_ok(rows, lse_s, lse_t)
    valid = valid & ok[..., None]
    lse_s_safe = np.where(lse_s == _NEG_INF, 0.0, lse_s)
    lse_t_safe = np.where(lse_t == _NEG_INF, 0.0, lse_t)
    ps = np.where(valid, np.exp(relation_logits(qs, ks, sm_scale_s) - lse_s_safe[..., None]), 0.0)
    pt = np.where(valid, np.exp(relation_logits(qt, kt, sm_scale_t) - lse_t_safe[..., None]), 0.0)
    dval = ps - pt
    if d_cast is not None:
        dval = round_to(dval.astype(np.float32), d_cast).astype(np.float64)
    gs = Hq // Hkv_s
    kmap = np.arange(Hq) // gs
    dq = sm_scale_s * np.matmul(dval, ks[:, kmap])
    dq = np.where(ok[..., None], dq, 0.0)
    dk = np.zeros((B, Hkv_s, T, Ds), dtype=np.float64)
    for h in range(Hq):
        dk[:, kmap[h]] += sm_scale_s * np.matmul(np.swapaxes(dval[:, h], -1, -2), qs[:, h])
    return dq, dk


# ---------------------------------------------------------------------------
# the autograd boundary
# ---------------------------------------------------------------------------

def attn_kl_align(qs, ks, qt, kt, mask=None, causal=True, sm_scale_s=None,
                  sm_scale_t=None, dloss=1.0, self_relation=None, d_cast=None):
    """``integration.py:6-73`` composed on the CPU.

    Returns ``(loss, dqs, dks, lse_s, lse_t)``.  When ``self_relation`` is
    true (the train.py call ``attn_kl_align(x, x, y, y)``), ``dqs`` is the
    summed gradient dq + dk of the shared input and ``dks`` is None.
    """
    Ds = np.asarray(qs).shape[3]
    Dt = np.asarray(qt).shape[3]
    sm_scale_s = 1.0 / math.sqrt(Ds) if sm_scale_s is None else sm_scale_s
    sm_scale_t = 1.0 / math.sqrt(Dt) if sm_scale_t is None else sm_scale_t
    lse_s = lse_stats(qs, ks, mask, causal, sm_scale_s)
    lse_t = lse_stats(qt, kt, mask, causal, sm_scale_t)
    loss = kl_forward(qs, ks, lse_s, qt, kt, lse_t, mask, causal, sm_scale_s, sm_scale_t)
    dq, dk = kl_backward(qs, ks, lse_s, qt, kt, lse_t, mask, causal,
                         sm_scale_s, sm_scale_t, d_cast=d_cast)
    dq = dq * dloss
    dk = dk * dloss
    if self_relation:
        return loss, dq + dk, None, lse_s, lse_t
    return loss, dq, dk, lse_s, lse_t


def materialized_kl(qs, ks, qt, kt, mask=None, causal=True, sm_scale_s=None,
                    sm_scale_t=None):
    """Independent formulation of ``integration.py:102-127``.

    log_softmax of the materialised logits masked with the dtype minimum,
    rows without a valid entry zeroed.  Row validity here is "any valid
    entry", which for consistent masks equals the mask itself.
    """
    qs = np.asarray(qs, dtype=np.float64)
    qt = np.asarray(qt, dtype=np.float64)
    B, Hq, T, Ds = qs.shape
    Dt = qt.shape[3]
    sm_scale_s = 1.0 / math.sqrt(Ds) if sm_scale_s is None else sm_scale_s
    sm_scale_t = 1.0 / math.sqrt(Dt) if sm_scale_t is None else sm_scale_t
    _, valid = validity(B, T, mask, causal)
    valid = np.broadcast_to(valid, (B, Hq, T, T))
    fmin = np.finfo(np.float64).min
    Ls = np.where(valid, relation_logits(qs, ks, sm_scale_s), fmin)
    Lt = np.where(valid, relation_logits(qt, kt, sm_scale_t), fmin)

    def log_softmax(x):
        mx = x.max(axis=-1, keepdims=True)
        y = x - mx
        return y - np.log(np.exp(y).sum(axis=-1, keepdims=True))

    lps = log_softmax(Ls)
    lpt = log_softmax(Lt)
    pt = np.exp(lpt)
    rows = valid.any(axis=-1, keepdims=True)
    lps = np.where(rows, lps, 0.0)
    lpt = np.where(rows, lpt, 0.0)
    pt = np.where(rows, pt, 0.0)
    return float((pt * (lpt - lps)).sum())


# ---------------------------------------------------------------------------
# linear-memory restatement of the self relation (train.py:380-402)
# ---------------------------------------------------------------------------

def self_relation_chunked(xs, xt, causal=True, sm_scale_s=None, sm_scale_t=None,
                          mask=None, chunk=256, dtype=np.float32, want_grad=True,
                          rows_subset=None):
    """Self relation KL(P_t || P_s) with P = softmax(a X X^T) for one [T,D] pair.

    Processes ``chunk`` query rows at a time, so memory is O(chunk * T)
    instead of O(T^2).  Returns ``(loss_sum, dX, lse_s, lse_t, kl_rows)``
    with ``dX = a_s (D + D^T) X_s`` (the q-is-k gradient; D = P_s - P_t).

    ``rows_subset`` (an int) restricts the forward to the first rows of the
    matrix (used to time a bounded CPU sample); dX is then None.
    """
    xs = np.asarray(xs, dtype=dtype)
    xt = np.asarray(xt, dtype=dtype)
    T, D = xs.shape
    sm_scale_s = 1.0 / math.sqrt(D) if sm_scale_s is None else sm_scale_s
    sm_scale_t = 1.0 / math.sqrt(xt.shape[1]) if sm_scale_t is None else sm_scale_t
    mb = np.ones(T, dtype=bool) if mask is None else (np.asarray(mask) != 0)
    n_rows = T if rows_subset is None else int(rows_subset)
    lse_s = np.zeros(T, dtype=np.float64)
    lse_t = np.zeros(T, dtype=np.float64)
    kl = np.zeros(T, dtype=np.float64)
    dX = np.zeros((T, D), dtype=dtype) if (want_grad and rows_subset is None) else None
    cols = np.arange(T)
    with np.errstate(divide="ignore", invalid="ignore"):
        _chunk_loop(xs, xt, mb, causal, sm_scale_s, sm_scale_t, chunk, dtype, n_rows, cols,
                    lse_s, lse_t, kl, dX)
    return float(kl.sum()), dX, lse_s, lse_t, kl


def _chunk_loop(xs, xt, mb, causal, sm_scale_s, sm_scale_t, chunk, dtype, n_rows, cols,
                lse_s, lse_t, kl, dX):
    T = xs.shape[0]
    for i0 in range(0, n_rows, chunk):
        i1 = min(n_rows, i0 + chunk)
        jmax = i1 if causal else T
        ridx = np.arange(i0, i1)
        valid = mb[i0:i1, None] & mb[None, :jmax]
        if causal:
            valid = valid & (cols[None, :jmax] <= ridx[:, None])
        Ss = (xs[i0:i1] @ xs[:jmax].T) * dtype(sm_scale_s)
        St = (xt[i0:i1] @ xt[:jmax].T) * dtype(sm_scale_t)
        Ss = np.where(valid, Ss, -np.inf)
        St = np.where(valid, St, -np.inf)
        ms = Ss.max(axis=1, keepdims=True)
        mt = St.max(axis=1, keepdims=True)
        ms = np.where(np.isfinite(ms), ms, 0)
        mt = np.where(np.isfinite(mt), mt, 0)
        es = np.exp(Ss - ms)
        et = np.exp(St - mt)
        ls = es.sum(axis=1, keepdims=True)
        lt = et.sum(axis=1, keepdims=True)
        lse_s_c = ms + np.log(ls)
        lse_t_c = mt + np.log(lt)
        ps = es / ls
        pt = et / lt
        logdiff = np.where(valid, (St - lse_t_c) - (Ss - lse_s_c), 0)
        kl_c = (pt * logdiff).sum(axis=1)
        rv = mb[i0:i1]
        lse_s[i0:i1] = np.where(rv, lse_s_c[:, 0], 0)
        lse_t[i0:i1] = np.where(rv, lse_t_c[:, 0], 0)
        kl[i0:i1] = np.where(rv, kl_c, 0)
        if dX is not None:
            Dm = np.where(valid & rv[:, None], ps - pt, 0).astype(dtype)
            dX[i0:i1] += dtype(sm_scale_s) * (Dm @ xs[:jmax])
            dX[:jmax] += dtype(sm_scale_s) * (Dm.T @ xs[i0:i1])


# ---------------------------------------------------------------------------
# flop / byte accounting (shared by bench and tests)
# ---------------------------------------------------------------------------

def relation_pairs(T, causal):
    """Number of (i, j) pairs per head: n(n+1)/2 causal, n^2 otherwise."""
    return T * (T + 1) // 2 if causal else T * T


def algorithmic_flops(B, H, T, D, causal=True):
    """12 * d * P per (b, h) relation for one fwd+bwd (2 GEMMs fwd, 4 bwd)."""
    return 12 * D * relation_pairs(T, causal) * B * H
