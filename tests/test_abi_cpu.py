"""CPU-side checks of the C ABI library and the host layer (no GPU needed).

Nothing here launches a kernel: the library must load, bind every symbol the
public header declares, and reject invalid arguments before touching the GPU.
"""

import ctypes
import inspect
import os

import pytest
import torch

from linearard_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol():
    names = _lib.header_functions()
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must cover the header exactly"
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), n
    assert L.lard_version().decode().startswith("linearard_amd")


def test_abi_rejects_bad_arguments_without_a_gpu():
    L = _lib.lib()
    t = _lib.Tensor4()
    t.data = 16
    t.size[:] = [1, 2, 8, 24]
    t.stride[:] = [384, 192, 24, 1]
    t.dtype = 1
    m = _lib.Mask()
    rc = L.lard_lse_stats(ctypes.byref(t), ctypes.byref(t), ctypes.byref(m), 1, 0.1, 64, None)
    assert rc == -2 and b"supported set" in L.lard_last_error()
    t.size[3] = 16
    t.stride[:] = [256, 128, 16, 1]
    t.dtype = 7
    rc = L.lard_lse_stats(ctypes.byref(t), ctypes.byref(t), ctypes.byref(m), 1, 0.1, 64, None)
    assert rc == -2 and b"fp16/bf16/fp32" in L.lard_last_error()
    t.dtype = 0
    t.stride[3] = 2
    rc = L.lard_lse_stats(ctypes.byref(t), ctypes.byref(t), ctypes.byref(m), 1, 0.1, 64, None)
    assert rc == -1 and b"last-dim stride" in L.lard_last_error()
    t.stride[3] = 1
    t.data = 8  # misaligned
    rc = L.lard_lse_stats(ctypes.byref(t), ctypes.byref(t), ctypes.byref(m), 1, 0.1, 64, None)
    assert rc == -2 and b"aligned" in L.lard_last_error()
    t.data = 16
    m.kind = 9
    rc = L.lard_lse_stats(ctypes.byref(t), ctypes.byref(t), ctypes.byref(m), 1, 0.1, 64, None)
    assert rc == -1 and b"attn_mask dtype" in L.lard_last_error()
    m.kind = 0
    rc = L.lard_lse_stats(ctypes.byref(t), ctypes.byref(t), ctypes.byref(m), 1, float("nan"), 64, None)
    assert rc == -1 and b"sm_scale" in L.lard_last_error()
    # per-row KL terms (256-byte aligned) + 512 double partials of the loss sum
    assert L.lard_kl_forward_workspace_bytes(2, 3, 5) == 256 + 512 * 8
    assert L.lard_kl_forward_workspace_bytes(4, 32, 4096) == 4 * 32 * 4096 * 4 + 512 * 8
    assert L.lard_kl_forward_workspace_bytes(0, 3, 5) == 0
    # forward of the autograd path adds one validity byte per (padded) token and
    # the first two valid tokens of each sequence (two int32, 256-aligned)
    assert L.lard_attn_kl_forward_workspace_bytes(4, 32, 4096) == 4 * 32 * 4096 * 4 + 512 * 8 + 4 * 4096 + 256
    # backward: validity bytes, the first two valid tokens per sequence and 2
    # normalisers per (padded) row, or, when larger, the float32 path's two
    # double LSEs per row
    B, H, T, D = 2, 8, 1000, 64
    Tp = 1024
    tail = B * Tp + 256 + 2 * B * H * Tp * 4
    f64 = (2 * B * H * T * 8 + 255) // 256 * 256
    assert L.lard_attn_kl_backward_workspace_bytes(B, H, H, T, D, 1) == max(tail, f64)
    assert L.lard_attn_kl_backward_workspace_bytes(B, H, H, T, D, 0) == max(tail, f64)
    assert L.lard_attn_kl_backward_workspace_bytes(0, H, H, T, D, 0) == 0


def test_noalloc_forward_rejects_sizes_beyond_its_scratch_without_a_gpu():
    """The library's own workspace holds LARD_NOALLOC_SCRATCH_BYTES (16 MiB) per
    GPU: a forward needing more is refused before anything is launched."""
    L = _lib.lib()
    t = _lib.Tensor4()
    t.data = 256
    B, H, T, D = 1, 64, 65536, 128  # 4M rows: 16 MiB of row KL terms alone
    t.size[:] = [B, H, T, D]
    t.stride[:] = [H * T * D, T * D, D, 1]
    t.dtype = 1
    m = _lib.Mask()
    need = L.lard_attn_kl_forward_workspace_bytes(B, H, T)
    assert need > 16 << 20
    rc = L.lard_attn_kl_forward_noalloc(ctypes.byref(t), ctypes.byref(t), ctypes.byref(t), ctypes.byref(t),
                                        ctypes.byref(m), 1, 0.1, 0.1, 512, 1024, 2048, None)
    assert rc == -2 and b"scratch" in L.lard_last_error()


def test_batched_abi_rejects_bad_batches_without_a_gpu():
    L = _lib.lib()
    rels = (_lib.Relation * 2)()
    for r in range(2):
        for t in (rels[r].xs, rels[r].xt):
            t.data = 256
            t.size[:] = [1, 4 - 2 * r, 64, 128]
            t.stride[:] = [t.size[1] * 64 * 128, 64 * 128, 128, 1]
            t.dtype = 1
        rels[r].lse_s = rels[r].lse_t = rels[r].dxs = 512
    m = _lib.Mask()
    ws = L.lard_attn_kl_batched_workspace_bytes(rels, 2)
    # rows of both relations (KL terms, 256-aligned) + loss partials + validity
    # bytes + first two valid tokens + two normalisers per row
    rows = 1 * (4 + 2) * 64
    assert ws == rows * 4 + 512 * 8 + 256 + 256 + 2 * rows * 4
    assert L.lard_attn_kl_batched_workspace_bytes(None, 0) == 0
    rc = L.lard_attn_kl_batched_forward(rels, 0, ctypes.byref(m), 1, 0.1, 0.1, None, 1024, None, 0, None)
    assert rc == -1 and b"at least one relation" in L.lard_last_error()
    rels[1].xs.size[2] = rels[1].xt.size[2] = 32  # another T
    rc = L.lard_attn_kl_batched_forward(rels, 2, ctypes.byref(m), 1, 0.1, 0.1, None, 1024, None, 0, None)
    assert rc == -1 and b"share B and T" in L.lard_last_error()
    rels[1].xs.size[2] = rels[1].xt.size[2] = 64
    rc = L.lard_attn_kl_batched_forward(rels, 2, ctypes.byref(m), 1, 3e-7, 0.1, None, 1024, None, 0, None)
    assert rc == -2 and b"scales" in L.lard_last_error()
    for r in range(2):
        for t in (rels[r].xs, rels[r].xt):
            t.size[3] = 256
            t.stride[:] = [t.size[1] * 64 * 256, 64 * 256, 256, 1]
    rc = L.lard_attn_kl_batched_backward(rels, 2, ctypes.byref(m), 1, 0.1, 0.1, None, None, None, 0, None)
    assert rc == -2 and b"D <= 128" in L.lard_last_error()


def test_rope_abi_rejects_bad_arguments_without_a_gpu():
    L = _lib.lib()
    t = _lib.Tensor4()
    t.data = 256
    t.size[:] = [1, 2, 16, 8]
    t.stride[:] = [256, 128, 8, 1]
    t.dtype = 1
    rc = L.lard_rope_pair(ctypes.byref(t), 512, 512, 1.0, 1.0, None, 0, 1024, 2048, None)
    assert rc == -2 and b"multiple of 16" in L.lard_last_error()
    t.size[3] = 64
    t.stride[:] = [2048, 1024, 64, 1]
    rc = L.lard_rope_pair(ctypes.byref(t), None, 512, 1.0, 1.0, None, 0, 1024, 2048, None)
    assert rc == -1 and b"must not be NULL" in L.lard_last_error()
    rc = L.lard_rope_pair(ctypes.byref(t), 512, 512, 1.0, float("nan"), None, 0, 1024, 2048, None)
    assert rc == -1 and b"finite" in L.lard_last_error()


def _logits_desc(B=1, K=4, V=64, dtype=1, data=4096):
    d = _lib.Logits()
    d.data = data
    d.size[:] = [B, K, V]
    d.stride[:] = [K * V, V, 1]
    d.dtype = dtype
    return d


def test_logits_kl_abi_rejects_bad_arguments_without_a_gpu():
    L = _lib.lib()
    t, s = _logits_desc(), _logits_desc(data=8192)
    f = [16384, 16384 + 64, 16384 + 128, 16384 + 192]  # lse_t, lse_s, kl, loss (never dereferenced)
    ws = L.lard_logits_kl_workspace_bytes(4, 64)
    assert ws >= 4 * 32 and L.lard_logits_kl_workspace_bytes(0, 64) == 0

    def fwd(t, s, T=1.0, ws_bytes=ws, out=f):
        return L.lard_logits_kl_forward(ctypes.byref(t) if t is not None else None, ctypes.byref(s), T, *out,
                                        32768, ws_bytes, None)

    assert fwd(None, s) == -1 and b"must not be NULL" in L.lard_last_error()
    assert fwd(t, _logits_desc(V=32, data=8192)) == -1 and b"shape must match" in L.lard_last_error()
    assert fwd(t, _logits_desc(dtype=0, data=8192)) == -1 and b"dtype must match" in L.lard_last_error()
    assert fwd(_logits_desc(dtype=3), s) == -2 and b"fp16/bf16/fp32" in L.lard_last_error()
    bad = _logits_desc()
    bad.stride[2] = 2
    assert fwd(bad, s) == -1 and b"vocabulary stride" in L.lard_last_error()
    assert fwd(_logits_desc(data=4098), s) == -2 and b"16-byte" in L.lard_last_error()
    odd = _logits_desc(V=63)
    odd.stride[:] = [4 * 63, 63, 1]
    assert fwd(odd, _logits_desc(V=63, data=8192)) == -2 and b"16-byte" in L.lard_last_error()
    for T in (0.0, float("inf"), float("nan"), 1e-45):
        assert fwd(t, s, T=T) == -1 and b"temperature" in L.lard_last_error()
    assert fwd(t, s, ws_bytes=ws - 1) == -1 and b"workspace too small" in L.lard_last_error()
    assert fwd(t, s, out=[f[0], f[1], f[2], None]) == -1 and b"loss" in L.lard_last_error()

    g_bad = _logits_desc(dtype=2, data=65536)
    rc = L.lard_logits_kl_backward(ctypes.byref(t), ctypes.byref(s), 1.0, f[0], f[1], f[2], f[3], 0, 0.25,
                                   None, ctypes.byref(g_bad), None)
    assert rc == -1 and b"grad_s dtype" in L.lard_last_error()
    g = _logits_desc(data=65536)
    rc = L.lard_logits_kl_backward(ctypes.byref(t), ctypes.byref(s), 1.0, f[0], f[1], None, f[3], 0, 0.25,
                                   ctypes.byref(g), None, None)
    assert rc == -1 and b"kl_rows" in L.lard_last_error()
    rc = L.lard_logits_kl_backward(ctypes.byref(t), ctypes.byref(s), 1.0, f[0], f[1], f[2], None, 0, 0.25,
                                   None, ctypes.byref(g), None)
    assert rc == -1 and b"dloss" in L.lard_last_error()
    # no gradient requested: nothing to do, no GPU call
    assert L.lard_logits_kl_backward(ctypes.byref(t), ctypes.byref(s), 1.0, f[0], f[1], f[2], f[3], 0, 0.25,
                                     None, None, None) == 0


def test_distillation_loss_validates_its_lists_without_a_gpu():
    from linearard_amd.distill import distillation_loss

    x = torch.zeros((1, 2, 8, 16), dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="one tensor per layer"):
        distillation_loss([x, x], [x], [x], [x], [x], [x])
    with pytest.raises(AssertionError, match="one tensor per layer"):
        distillation_loss([], [], [], [], [], [])
    with pytest.raises(AssertionError, match="given together"):
        distillation_loss([x], [x], [x], [x], [x], [x], t_logits=torch.zeros((1, 2, 4)))


def test_python_wrappers_reject_cpu_tensors():
    from linearard_amd.attention_KL import kl_backward, kl_forward, lse_stats

    x = torch.zeros((1, 2, 8, 16), dtype=torch.bfloat16)
    l = torch.zeros((1, 2, 8))
    with pytest.raises(AssertionError, match="q/k must be on CUDA"):
        lse_stats(x, x)
    with pytest.raises(AssertionError, match="Q/K must be on CUDA"):
        kl_forward(x, x, l, x, x, l)
    with pytest.raises(AssertionError, match="Q/K must be on CUDA"):
        kl_backward(x, x, l, x, x, l)
    with pytest.raises(AssertionError, match="q must be a torch.Tensor"):
        lse_stats(None, x)


def test_wrappers_contain_no_math():
    """Equivalent of the reference's static_audit_wrapper (test_kernel_A.py:102-119):
    all arithmetic lives in the HIP library, none in the Python wrappers."""
    from linearard_amd.attention_KL import kernel_A, kernel_B, kernel_C

    banned = ["matmul", "einsum", "softmax", "logsumexp", "exp(", "log(", "sum(", "max(", "mean(",
              "reshape", "transpose"]
    for fn in (kernel_A.lse_stats, kernel_B.kl_forward, kernel_C.kl_backward):
        src = inspect.getsource(fn).lower()
        for key in banned:
            assert key not in src, f"{fn.__name__} contains {key}"


def test_no_runtime_compilation_fixed_instantiation_table():
    """The reference counts Triton JIT specialisations (test_kernel_A.py:127-203);
    here every kernel is compiled ahead of time, so the library's kernel table is
    fixed: 5 LSE + 25 KL + 25 dq + 25 dk instantiations (padded D in 16..256)."""
    path = os.path.join(ROOT, "linearard_amd", "csrc")
    srcs = [f for f in os.listdir(path) if f.endswith(".hip")]
    text = "".join(open(os.path.join(path, f)).read() for f in srcs)
    assert "hiprtc" not in text.lower()
    assert text.count("LARD_DP_CASES(X, 0)") >= 7


def test_drop_in_shim_names():
    from kernels.attention_KL import kernel_A, kernel_B, kernel_C
    from kernels.attention_KL.integration import AttnKLAlignFn, attn_kl_align

    assert kernel_A.lse_stats_triton is kernel_A.lse_stats
    assert kernel_B.kl_forward_triton is kernel_B.kl_forward
    assert kernel_C.kl_backward_triton is kernel_C.kl_backward
    assert kernel_A.SUPPORTED_HEAD_DIMS == (8, 16, 32, 64, 128, 256)
    assert callable(attn_kl_align) and issubclass(AttnKLAlignFn, torch.autograd.Function)


def test_timing_hook_validates_and_reads_empty_without_a_gpu():
    L = _lib.lib()
    total = ctypes.c_double(-1.0)
    count = ctypes.c_int64(-1)
    assert L.lard_timing_read(7, ctypes.byref(total), ctypes.byref(count)) == -1
    assert b"kernel id" in L.lard_last_error()
    assert L.lard_timing_read(0, None, ctypes.byref(count)) == -1
    assert L.lard_timing_enable(0) == 0
    for kid in _lib.KERNEL_IDS.values():  # nothing recorded: no HIP call is made
        assert L.lard_timing_read(kid, ctypes.byref(total), ctypes.byref(count)) == 0
        assert total.value == 0.0 and count.value == 0


def test_counter_summary_scales_by_the_calibration_copy(tmp_path):
    from linearard_amd import profiling

    head = ("Correlation_Id,Dispatch_Id,Agent_Id,Queue_Id,Process_Id,Thread_Id,Grid_Size,Kernel_Id,Kernel_Name,"
            "Workgroup_Size,LDS_Block_Size,Scratch_Size,VGPR_Count,Accum_VGPR_Count,SGPR_Count,Counter_Name,"
            "Counter_Value,Start_Timestamp,End_Timestamp\n")

    def row(d, name, counter, v):
        return f'{d},{d},A,1,1,1,1,1,"{name}",256,0,0,8,0,8,{counter},{v},0,1\n'

    fetch = tmp_path / "f.csv"
    write = tmp_path / "w.csv"
    # the calibration copy of 1 MiB reads as 512 counts (2 KiB per count); two
    # launches of the column kernel read 3000 and 1000 counts (mean 2000)
    fetch.write_text(head + row(1, "void at::native::neg_kernel_cuda(x)", "FETCH_SIZE", 512)
                     + row(2, "void lard::hot_bwd_kernel<128, true>(lard::HotArgs)", "FETCH_SIZE", 3000)
                     + row(3, "void lard::hot_bwd_kernel<128, true>(lard::HotArgs)", "FETCH_SIZE", 1000))
    write.write_text(head + row(1, "void at::native::neg_kernel_cuda(x)", "WRITE_SIZE", 1024)
                     + row(2, "void lard::hot_bwd_kernel<128, true>(lard::HotArgs)", "WRITE_SIZE", 100))
    out = profiling.traffic(str(fetch), str(write), 1, "cfg4")
    assert out["scale_fetch_bytes_per_count"] == 2048.0 and out["scale_write_bytes_per_count"] == 1024.0
    assert out["read_bytes"]["col_grad"] == 2000 * 2048.0
    assert out["bytes_per_launch"]["col_grad"] == 2000 * 2048.0 + 100 * 1024.0


def test_attn_kl_path_names_the_slower_paths_without_a_gpu():
    """lard_attn_kl_path classifies operands (nothing is launched): the
    throughput kernels, or the slower path and the condition behind it."""
    L = _lib.lib()

    def desc(D=128, dtype=1, T=64, H=2, row_stride=None):
        t = _lib.Tensor4()
        t.data = 4096
        t.size[:] = [1, H, T, D]
        rs = D if row_stride is None else row_stride
        t.stride[:] = [H * T * rs, T * rs, rs, 1]
        t.dtype = dtype
        return t

    def path(qs, qt, ss=0.1, st=0.1):
        rc = L.lard_attn_kl_path(ctypes.byref(qs), ctypes.byref(qs), ctypes.byref(qt), ctypes.byref(qt), ss, st)
        return rc, L.lard_last_error().decode()

    assert path(desc(), desc()) == (0, "")
    rc, why = path(desc(256), desc(256))
    assert rc == 1 and "head dim 256 > 128" in why
    rc, why = path(desc(64), desc(128))
    assert rc == 2 and "64 != teacher head dim 128" in why
    rc, why = path(desc(dtype=0), desc(dtype=1))
    assert rc == 2 and "dtypes differ" in why
    rc, why = path(desc(dtype=2), desc(dtype=2))
    assert rc == 3 and "float32" in why
    rc, why = path(desc(), desc(), ss=1e-7)
    assert rc == 1 and "scales" in why
    rc, why = path(desc(T=1 << 20, row_stride=2048), desc(T=1 << 20, row_stride=2048))
    assert rc == 1 and "2^30" in why
    rc, why = path(desc(D=24), desc(D=24))
    assert rc == -2 and "supported set" in why  # invalid operands: an error, as for the compute calls
    # the alignment checks of the compute calls, with their error codes
    rc, why = path(desc(dtype=2), desc(dtype=1))
    assert rc == -2 and "float32 on both sides" in why
    rc, why = path(desc(dtype=1), desc(dtype=2))
    assert rc == -2 and "float32 on both sides" in why
    for kw in ({"T": 128}, {"H": 4}):
        rc, why = path(desc(), desc(**kw))
        assert rc == -1 and "B/Hq/T must align" in why
