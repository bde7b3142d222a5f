"""Static checks on the gfx950 assembly of the throughput kernels (CPU only).

Three properties of the device code, checked on its assembly:

* No writes through the scalar data cache anywhere (every kernel of every
  source): device code writes memory through vector stores only.

Two hazards the compiler cannot police for code it did not write itself:

* M0.  The HBM->LDS copies (``lds_async16``, inline asm) write M0, which the
  compiler reserves.  The kernels are correct only while nothing else in them
  uses M0: every instruction that names ``m0`` must be that copy sequence
  (``s_mov_b32 m0, ...`` / ``s_nop 0`` / ``global_load_lds_dwordx4``), and no
  instruction that reads M0 implicitly (movrel, gpr_idx, sendmsg, GWS,
  ``*_addtid``, interpolation) may appear at all.

* MFMA dependencies.  The fused forward (``hot_fwdq_*``) issues its MFMAs as
  inline asm, so the compiler inserts none of the wait states that the
  gfx950 matrix unit requires around them.  The checks, on every control-flow
  path, in wait states (one per instruction, N + 1 for ``s_nop N``):
    - an MFMA result (VGPR or AGPR) is not touched by any other instruction
      for ``RESULT_WAIT`` wait states, except by the next MFMA of the same
      accumulation chain (source C == destination, exactly);
    - no VALU instruction writes an MFMA source register in the
      ``OPERAND_WAIT`` wait states before it, on any path into it (across
      branches and labels).

Used by ``tests/test_isa.py``; nothing in the product imports it.
"""

from __future__ import annotations

import os
import re
import subprocess

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

# gfx950, 8-pass XDL (v_mfma_f32_32x32x16_*): result -> VALU / memory read or
# write needs 11 + 1 wait states and 16-pass ones 19; checking 19 covers both.
RESULT_WAIT = 19
# VALU write of a VGPR -> MFMA reads it: 2 wait states.
OPERAND_WAIT = 2

# Writes through the scalar data cache (scalar stores and atomics, the
# cache's write-back and discard): none may appear in any kernel.
SCALAR_WRITE = re.compile(r"^(s_store|s_buffer_store|s_scratch_store|s_atomic|s_buffer_atomic|s_dcache_wb"
                          r"|s_dcache_discard)")

IMPLICIT_M0 = re.compile(r"^(v_movrel|s_movrel|s_set_gpr_idx|s_sendmsg|ds_gws|v_interp|ds_\w*addtid|s_ttracedata)")


def device_asm(src: str, out_dir: str) -> str:
    """gfx950 assembly of one HIP source (compiled like the Makefile does)."""
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-S", src, "-o", out]
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    with open(out, "r", encoding="utf-8") as f:
        return f.read()


def kernels(asm: str) -> dict:
    """kernel name -> list of (kind, text): kind 'label' or 'inst'."""
    out = {}
    cur = None
    for line in asm.split("\n"):
        m = re.match(r"^(_Z\w+):", line)
        if m:
            cur = m.group(1)
            out[cur] = []
            continue
        if cur is None:
            continue
        t = line.split(";")[0].strip()
        if not t:
            continue
        if t.startswith(".Lfunc_end") or t.startswith(".size"):
            cur = None
            continue
        lm = re.match(r"^(\.L\w+|\d+):$", t)
        if lm:
            out[cur].append(("label", lm.group(1)))
        elif not t.startswith("."):
            out[cur].append(("inst", t))
    return out


def _regs(tok: str):
    """Registers named by one operand: a set of ('v'|'a'|'s', index)."""
    tok = tok.strip()
    m = re.match(r"^\|?-?\|?([vas])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"^\|?-?\|?([vas])(\d+)\b", tok)
    if m:
        return {(m.group(1), int(m.group(2)))}
    return set()


def _operands(inst: str):
    parts = inst.split(None, 1)
    if len(parts) == 1:
        return parts[0], []
    ops = [o.strip() for o in re.split(r",(?![^\[]*\])", parts[1])]
    return parts[0], ops


def _wait_states(inst: str) -> int:
    op, ops = _operands(inst)
    if op == "s_nop":
        return int(ops[0], 0) + 1
    return 1


def _touches(inst: str, regs) -> bool:
    _, ops = _operands(inst)
    for o in ops:
        if _regs(o) & regs:
            return True
    return False


def check_m0(name: str, body) -> list:
    errs = []
    insts = [t for k, t in body if k == "inst"]
    for i, t in enumerate(insts):
        op, ops = _operands(t)
        if IMPLICIT_M0.match(op):
            errs.append(f"{name}: {t!r} reads M0 implicitly")
        if any(o == "m0" for o in ops):
            ok = (op == "s_mov_b32" and ops[0] == "m0" and i + 2 < len(insts) and insts[i + 1] == "s_nop 0"
                  and insts[i + 2].startswith("global_load_lds_dwordx4"))
            if not ok:
                errs.append(f"{name}: {t!r} uses M0 outside the HBM->LDS copy sequence")
    return errs


def check_no_scalar_writes(name: str, body) -> list:
    return [f"{name}: {t!r} writes through the scalar data cache" for k, t in body
            if k == "inst" and SCALAR_WRITE.match(_operands(t)[0])]


def _successors(body, pos):
    """Positions control may reach right after the instruction at pos."""
    kind, t = body[pos]
    op, ops = _operands(t)
    labels = {text: i for i, (k, text) in enumerate(body) if k == "label"}

    def target(lbl):
        if re.match(r"^\d+f$", lbl):  # numeric local label, forward
            want = lbl[:-1]
            for j in range(pos + 1, len(body)):
                if body[j] == ("label", want):
                    return j
            raise ValueError(f"no forward label {lbl}")
        return labels[lbl]

    if op == "s_endpgm":
        return []
    if op == "s_branch":
        return [target(ops[0])]
    if op.startswith("s_cbranch"):
        return [pos + 1, target(ops[0])]
    if op.startswith("s_setpc") or op.startswith("s_swappc"):
        raise ValueError(f"indirect branch {t!r}")
    return [pos + 1]


def _scan_result(body, start, regs, chain_dst):
    """Smallest wait-state distance from the MFMA at start to an instruction
    touching regs (None if none within RESULT_WAIT on any path)."""
    worst = None
    stack = [(s, 0) for s in _successors(body, start)]
    seen = {}
    while stack:
        pos, dist = stack.pop()
        if pos >= len(body) or dist >= RESULT_WAIT:
            continue
        if seen.get(pos, 1 << 30) <= dist:
            continue
        seen[pos] = dist
        kind, t = body[pos]
        if kind == "inst":
            op, ops = _operands(t)
            if _touches(t, regs):
                if op.startswith("v_mfma") and len(ops) >= 4 and ops[0] == chain_dst and ops[3] == chain_dst:
                    continue  # the next MFMA of the same accumulation chain
                worst = dist if worst is None else min(worst, dist)
                continue
            step = _wait_states(t)
        else:
            step = 0
        for s in _successors(body, pos) if kind == "inst" else [pos + 1]:
            stack.append((s, dist + step))
    return worst


def _predecessors(body):
    """position -> positions control may come from directly (fall-through
    from the previous instruction unless that ends the path, and every branch
    whose target is that label)."""
    preds = {i: [] for i in range(len(body))}
    for j, (kind, t) in enumerate(body):
        succ = _successors(body, j) if kind == "inst" else [j + 1]
        for s2 in succ:
            if s2 < len(body):
                preds[s2].append(j)
    return preds


def _scan_operand_writes(body, preds, i, srcs):
    """Wait states between VALU writes of srcs and the MFMA at i, on every
    path into it, for writes closer than OPERAND_WAIT: [(position, distance)]."""
    hits = []
    stack = [(p, 0) for p in preds[i]]
    seen = set()
    while stack:
        pos, ws = stack.pop()
        if ws >= OPERAND_WAIT or (pos, ws) in seen:
            continue
        seen.add((pos, ws))
        kind, t = body[pos]
        step = 0
        if kind == "inst":
            op, ops = _operands(t)
            if op.startswith("v_") and not op.startswith("v_mfma") and ops and _regs(ops[0]) & srcs:
                hits.append((pos, ws))
                continue
            step = _wait_states(t)
        for p in preds[pos]:
            stack.append((p, ws + step))
    return hits


def check_mfma_hazards(name: str, body) -> list:
    errs = []
    preds = _predecessors(body)
    for i, (kind, t) in enumerate(body):
        if kind != "inst" or not t.startswith("v_mfma"):
            continue
        op, ops = _operands(t)
        dst = _regs(ops[0])
        d = _scan_result(body, i, dst, ops[0])
        if d is not None:
            errs.append(f"{name}: result of {t!r} (#{i}) is touched {d} wait states later (< {RESULT_WAIT})")
        # VALU writes of the sources within OPERAND_WAIT before, on every path
        srcs = set()
        for o in ops[1:4]:
            srcs |= _regs(o)
        for pos, ws in _scan_operand_writes(body, preds, i, srcs):
            errs.append(f"{name}: {body[pos][1]!r} writes an operand of {t!r} {ws} wait states before it")
    return errs
