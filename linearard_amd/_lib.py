"""ctypes binding of ``liblinearard_amd.so`` (the C ABI in include/linearard_amd.h).

The library is loaded lazily on first use and fails loudly when it is
missing: there is no CPU or eager-PyTorch fallback anywhere in this package.
``torch`` is imported first on purpose: it owns the process's HIP runtime
(``libamdhip64.so.7``), which the library then shares, so torch streams and
device pointers are valid inside the library.
"""

from __future__ import annotations

import ctypes
import os
import re

import torch

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PACKAGE_DIR, "liblinearard_amd.so")
HEADER_PATH = os.path.join(os.path.dirname(PACKAGE_DIR), "include", "linearard_amd.h")

LARD_OK = 0
LARD_ERR_UNSUPPORTED = -2
DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
LOGITS_DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
MASK_CODES = {torch.bool: 1, torch.uint8: 1, torch.int32: 2, torch.int64: 3}


class Tensor4(ctypes.Structure):
    """``lard_tensor4``: a [B, H, T, D] device tensor view."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("size", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
        ("dtype", ctypes.c_int32),
    ]


class Mask(ctypes.Structure):
    """``lard_mask``: a [B, T] device attention mask."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("kind", ctypes.c_int32),
        ("size", ctypes.c_int64 * 2),
        ("stride", ctypes.c_int64 * 2),
    ]


class Logits(ctypes.Structure):
    """``lard_logits``: [B, K, V] logits of the kept positions."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("size", ctypes.c_int64 * 3),
        ("stride", ctypes.c_int64 * 3),
        ("dtype", ctypes.c_int32),
    ]


class Relation(ctypes.Structure):
    """``lard_relation``: one self relation of a batched loss."""

    _fields_ = [
        ("xs", Tensor4),
        ("xt", Tensor4),
        ("lse_s", ctypes.c_void_p),
        ("lse_t", ctypes.c_void_p),
        ("dxs", ctypes.c_void_p),
    ]


_T4P = ctypes.POINTER(Tensor4)
_MP = ctypes.POINTER(Mask)
_RP = ctypes.POINTER(Relation)
_LP = ctypes.POINTER(Logits)
_FP = ctypes.c_void_p  # float* device pointers are passed as addresses

# name -> (restype, argtypes); must cover every function include/linearard_amd.h declares.
SIGNATURES = {
    "lard_version": (ctypes.c_char_p, []),
    "lard_last_error": (ctypes.c_char_p, []),
    "lard_attn_kl_path": (ctypes.c_int, [_T4P, _T4P, _T4P, _T4P, ctypes.c_float, ctypes.c_float]),
    "lard_lse_stats": (ctypes.c_int, [_T4P, _T4P, _MP, ctypes.c_int, ctypes.c_float, _FP, ctypes.c_void_p]),
    "lard_kl_forward_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]),
    "lard_kl_forward": (ctypes.c_int, [_T4P, _T4P, _FP, _T4P, _T4P, _FP, _MP, ctypes.c_int, ctypes.c_float,
                                       ctypes.c_float, _FP, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "lard_kl_backward": (ctypes.c_int, [_T4P, _T4P, _FP, _T4P, _T4P, _FP, _MP, ctypes.c_int, ctypes.c_float,
                                        ctypes.c_float, _FP, _FP, ctypes.c_void_p]),
    "lard_attn_kl_forward_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 3),
    "lard_attn_kl_forward": (ctypes.c_int, [_T4P, _T4P, _T4P, _T4P, _MP, ctypes.c_int, ctypes.c_float,
                                            ctypes.c_float, _FP, _FP, _FP, ctypes.c_void_p, ctypes.c_size_t,
                                            ctypes.c_void_p]),
    "lard_attn_kl_forward_noalloc": (ctypes.c_int, [_T4P, _T4P, _T4P, _T4P, _MP, ctypes.c_int, ctypes.c_float,
                                                    ctypes.c_float, _FP, _FP, _FP, ctypes.c_void_p]),
    "lard_attn_kl_backward_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 5 + [ctypes.c_int]),
    "lard_attn_kl_backward": (ctypes.c_int, [_T4P, _T4P, _FP, _T4P, _T4P, _FP, _MP, ctypes.c_int, ctypes.c_float,
                                             ctypes.c_float, _FP, ctypes.c_int, _FP, _FP, ctypes.c_void_p,
                                             ctypes.c_size_t, ctypes.c_void_p]),
    "lard_attn_kl_forward_rowgrad_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 6),
    "lard_attn_kl_batched_rowgrad_workspace_bytes": (ctypes.c_size_t, [_RP, ctypes.c_int]),
    "lard_attn_kl_forward_rowgrad": (ctypes.c_int, [_T4P, _T4P, _T4P, _T4P, _MP, ctypes.c_int, ctypes.c_float,
                                                    ctypes.c_float, _FP, _FP, _FP, _FP, ctypes.c_void_p,
                                                    ctypes.c_size_t, ctypes.c_void_p]),
    "lard_attn_kl_backward_colgrad": (ctypes.c_int, [_T4P, _T4P, _FP, _T4P, _T4P, _FP, _MP, ctypes.c_int,
                                                     ctypes.c_float, ctypes.c_float, _FP, ctypes.c_int, _FP, _FP,
                                                     ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "lard_attn_kl_batched_workspace_bytes": (ctypes.c_size_t, [_RP, ctypes.c_int]),
    "lard_attn_kl_batched_forward_rowgrad": (ctypes.c_int, [_RP, ctypes.c_int, _MP, ctypes.c_int, ctypes.c_float,
                                                            ctypes.c_float, _FP, _FP, ctypes.c_void_p,
                                                            ctypes.c_size_t, ctypes.c_void_p]),
    "lard_attn_kl_batched_backward_colgrad": (ctypes.c_int, [_RP, ctypes.c_int, _MP, ctypes.c_int, ctypes.c_float,
                                                             ctypes.c_float, _FP, _FP, ctypes.c_void_p,
                                                             ctypes.c_size_t, ctypes.c_void_p]),
    "lard_attn_kl_batched_forward": (ctypes.c_int, [_RP, ctypes.c_int, _MP, ctypes.c_int, ctypes.c_float,
                                                    ctypes.c_float, _FP, _FP, ctypes.c_void_p, ctypes.c_size_t,
                                                    ctypes.c_void_p]),
    "lard_attn_kl_batched_backward": (ctypes.c_int, [_RP, ctypes.c_int, _MP, ctypes.c_int, ctypes.c_float,
                                                     ctypes.c_float, _FP, _FP, ctypes.c_void_p, ctypes.c_size_t,
                                                     ctypes.c_void_p]),
    "lard_rope_pair": (ctypes.c_int, [_T4P, _FP, _FP, ctypes.c_float, ctypes.c_float, ctypes.c_void_p,
                                      ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "lard_logits_kl_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64]),
    "lard_logits_kl_forward": (ctypes.c_int, [_LP, _LP, ctypes.c_float, _FP, _FP, _FP, _FP, ctypes.c_void_p,
                                              ctypes.c_size_t, ctypes.c_void_p]),
    "lard_logits_kl_backward": (ctypes.c_int, [_LP, _LP, ctypes.c_float, _FP, _FP, _FP, _FP, ctypes.c_int,
                                               ctypes.c_float, _LP, _LP, ctypes.c_void_p]),
    "lard_timing_enable": (ctypes.c_int, [ctypes.c_int]),
    "lard_timing_read": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_int64)]),
}

KERNEL_IDS = {"forward": 0, "row_grad": 1, "col_grad": 2, "logits_forward": 3, "logits_grad": 4,
              "forward_rowgrad": 5}

_LIB = None


def header_functions(path: str = HEADER_PATH):
    """Names of the functions declared in the public header."""
    with open(path, "r", encoding="utf-8") as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lard_[a-z0-9_]+)\s*\(", text)))


def lib():
    """Load and bind the library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c \"import __graft_entry__ as g; g.build()\"` "
                "(hipcc --offload-arch=gfx950); there is no fallback implementation")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != LARD_OK:
        msg = lib().lard_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def tensor4(t: torch.Tensor) -> Tensor4:
    d = Tensor4()
    d.data = t.data_ptr()
    for i in range(4):
        d.size[i] = t.shape[i]
        d.stride[i] = t.stride(i)
    d.dtype = DTYPE_CODES[t.dtype]
    return d


def logits_desc(t: torch.Tensor) -> Logits:
    """A [B, K, V] tensor (a [R, V] one is read as B = 1, K = R)."""
    if t.ndim == 2:
        t = t.unsqueeze(0)
    d = Logits()
    d.data = t.data_ptr()
    for i in range(3):
        d.size[i] = t.shape[i]
        d.stride[i] = t.stride(i)
    d.dtype = LOGITS_DTYPE_CODES[t.dtype]
    return d


def mask_desc(m) -> Mask:
    d = Mask()
    if m is None:
        d.data = None
        d.kind = 0
        return d
    d.data = m.data_ptr()
    d.kind = MASK_CODES[m.dtype]
    for i in range(2):
        d.size[i] = m.shape[i]
        d.stride[i] = m.stride(i)
    return d


def stream_of(t: torch.Tensor) -> int:
    """The current torch stream of the tensor's device, as a hipStream_t."""
    return torch.cuda.current_stream(t.device).cuda_stream
