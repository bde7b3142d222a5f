"""Static checks of the compiled gfx950 kernels (CPU; hipcc cross-compiles).

* No kernel of any source writes through the scalar data cache.
* The HBM->LDS copy sequence is the only user of M0 in the throughput
  kernels (hot.hip, hot_fwdq.hip): the copies write M0 from inline asm while
  the compiler reserves it.
* The fused row-gradient forward (hot_fwdq.hip) issues its MFMAs as inline
  asm; on every control-flow path of every instantiation, MFMA results are
  left alone for the gfx950 wait states and no VALU write of an MFMA operand
  comes within 2 wait states before it (tests/isa_check.py).
* The checker itself catches planted violations.
"""

import os

import pytest

from tests import isa_check as C

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "linearard_amd", "csrc")
HAVE_HIPCC = os.path.exists(C.HIPCC)
needs_hipcc = pytest.mark.skipif(not HAVE_HIPCC, reason="hipcc not installed")


@pytest.fixture(scope="module")
def asm_dir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("isa"))


_ASM = {}


def _kernels(src, asm_dir):
    """Kernels of one source's gfx950 assembly (compiled once per session)."""
    if src not in _ASM:
        _ASM[src] = C.kernels(C.device_asm(os.path.join(CSRC, src), asm_dir))
    return _ASM[src]


SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


@needs_hipcc
@pytest.mark.parametrize("src", SOURCES)
def test_no_writes_through_the_scalar_cache(asm_dir, src):
    ks = _kernels(src, asm_dir)
    errs = [e for name, body in ks.items() for e in C.check_no_scalar_writes(name, body)]
    assert not errs, "\n".join(errs[:20])


@needs_hipcc
@pytest.mark.parametrize("src", ["hot.hip", "hot_fwdq.hip"])
def test_m0_only_in_the_copy_sequence(asm_dir, src):
    ks = _kernels(src, asm_dir)
    assert ks, "no kernels found"
    errs = [e for name, body in ks.items() for e in C.check_m0(name, body)]
    assert not errs, "\n".join(errs[:20])
    # the copies are there (the check is not vacuous)
    assert any("global_load_lds_dwordx4" in t for body in ks.values() for _, t in body)


@needs_hipcc
def test_fused_forward_mfma_wait_states(asm_dir):
    ks = _kernels("hot_fwdq.hip", asm_dir)
    fused = {n: b for n, b in ks.items() if "hot_fwdq" in n}
    assert len(fused) == 16, sorted(fused)  # {16, 32, 64, 128} x {bf16, f16} x {single, batch}
    errs = [e for name, body in fused.items() for e in C.check_mfma_hazards(name, body)]
    assert not errs, "\n".join(errs[:20])


def _body(lines):
    out = []
    for ln in lines:
        if ln.endswith(":"):
            out.append(("label", ln[:-1]))
        else:
            out.append(("inst", ln))
    return out


def test_checker_catches_planted_hazards():
    mfma = "v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]"
    # result read too soon
    assert C.check_mfma_hazards("k", _body([mfma, "v_add_f32_e32 v30, v3, v31", "s_endpgm"]))
    # result read after enough wait states
    assert not C.check_mfma_hazards("k", _body([mfma, "s_nop 7", "s_nop 7", "s_nop 3", "v_add_f32_e32 v30, v3, v31",
                                                "s_endpgm"]))
    # the next MFMA of the same chain may follow directly
    assert not C.check_mfma_hazards("k", _body([mfma, mfma, "s_nop 7", "s_nop 7", "s_nop 3", "s_endpgm"]))
    # another MFMA reading the result as an A operand may not
    assert C.check_mfma_hazards("k", _body([mfma, "v_mfma_f32_32x32x16_bf16 v[40:55], v[0:3], v[20:23], 0",
                                            "s_nop 7", "s_nop 7", "s_nop 3", "s_endpgm"]))
    # a VALU write of an operand right before the MFMA
    assert C.check_mfma_hazards("k", _body(["v_mov_b32_e32 v17, 0", mfma, "s_nop 7", "s_nop 7", "s_nop 3",
                                            "s_endpgm"]))
    # ... and one wait state apart is still too close, two is enough
    assert C.check_mfma_hazards("k", _body(["v_mov_b32_e32 v17, 0", "s_nop 0", mfma, "s_nop 7", "s_nop 7",
                                            "s_nop 3", "s_endpgm"]))
    assert not C.check_mfma_hazards("k", _body(["v_mov_b32_e32 v17, 0", "s_nop 1", mfma, "s_nop 7", "s_nop 7",
                                                "s_nop 3", "s_endpgm"]))
    # an operand written in a predecessor block: by the branch's block and by fall-through
    assert C.check_mfma_hazards("k", _body(["v_mov_b32_e32 v17, 0", "s_cbranch_scc1 .LBB0_1", "s_nop 7",
                                            ".LBB0_1:", mfma, "s_nop 7", "s_nop 7", "s_nop 3", "s_endpgm"]))
    assert C.check_mfma_hazards("k", _body(["s_cbranch_scc1 .LBB0_1", "v_mov_b32_e32 v17, 0",
                                            ".LBB0_1:", mfma, "s_nop 7", "s_nop 7", "s_nop 3", "s_endpgm"]))
    # ... and far enough on both paths
    assert not C.check_mfma_hazards("k", _body(["v_mov_b32_e32 v17, 0", "s_nop 0", "s_cbranch_scc1 .LBB0_1",
                                                "s_nop 1", ".LBB0_1:", mfma, "s_nop 7", "s_nop 7", "s_nop 3",
                                                "s_endpgm"]))
    # AGPR accumulators, read back too early along a branch target
    acc = "v_mfma_f32_32x32x16_bf16 a[0:15], v[16:19], v[20:23], a[0:15]"
    assert C.check_mfma_hazards("k", _body([acc, "s_cbranch_scc1 .LBB0_2", "s_nop 7", "s_nop 7", "s_nop 7",
                                            ".LBB0_2:", "v_accvgpr_read_b32 v1, a4", "s_endpgm"]))
    # a scalar store and a scalar atomic
    assert C.check_no_scalar_writes("k", _body(["s_store_dword s4, s[0:1], 0x0"]))
    assert C.check_no_scalar_writes("k", _body(["s_atomic_add s4, s[0:1], 0x0"]))
    assert not C.check_no_scalar_writes("k", _body(["s_load_dword s4, s[0:1], 0x0", "global_store_dword v0, v1, off"]))
    # M0 outside the copy sequence, and an implicit reader
    assert C.check_m0("k", _body(["s_mov_b32 m0, s4", "ds_read_b32 v0, v1"]))
    assert C.check_m0("k", _body(["s_sendmsg sendmsg(MSG_INTERRUPT)"]))
    assert not C.check_m0("k", _body(["s_mov_b32 m0, s4", "s_nop 0", "global_load_lds_dwordx4 v1, s[2:3]"]))
