"""Every MFMA result is read only after the matrix core has written it (CPU only).

A 32x32 or 16x16 MFMA writes its result registers over several passes, and
an instruction that reads them (an accumulator read, an LDS or global store,
a VALU operation) must come enough wait states later; the compiler inserts
``s_nop`` for that.  Once, behind a branch that skipped a prefetch, it read
two accumulators one instruction after the last MFMA of a chain and waited
only afterwards, so a few RVQ codes came out wrong.  This test compiles every
``csrc/*.hip`` to gfx950 assembly with the library's flags and follows every
control-flow path from each MFMA to the first non-MFMA instruction reading
one of its result registers, counting wait states (an ``s_nop N`` counts
N + 1, any other instruction 1, branches followed both ways); each such read
must come at least passes + 1 wait states after the MFMA.  (The compiler's
own straight-line waits are passes + 2; the bad read had 1.)  Passes per
instruction on gfx950, from the MFMA busy cycles the counters report (4 per
pass): 32x32x2 f32 16, 32x32x16 bf16 8, 16x16x4 f32 8, 16x16x32 bf16 4.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

import pytest

from conftest import REPO

sys.path.insert(0, str(REPO / "fast-mimi_amd"))
import build_native  # noqa: E402  (the library's own compile flags)

HIPCC = build_native.HIPCC
CSRC = REPO / "fast-mimi_amd" / "csrc"
OUT = REPO / "fast-mimi_amd" / "_build" / "isa"
PASSES = {"v_mfma_f32_32x32x2_f32": 16, "v_mfma_f32_32x32x16_bf16": 8,
          "v_mfma_f32_16x16x4_f32": 8, "v_mfma_f32_16x16x32_bf16": 4}
MARGIN = 1
_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_STORES = ("ds_write", "buffer_store", "global_store", "flat_store", "scratch_store", "global_atomic",
           "buffer_atomic")
_LOADS = ("ds_read", "global_load", "buffer_load", "flat_load", "scratch_load")


def _regs(text: str) -> set:
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out |= {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


def _functions(path):
    """(name, [(opcode, operands)], {label: index}) per function of an assembly file."""
    funcs, cur = [], None
    for line in open(path):
        s = line.split(";")[0].rstrip()
        if not s.strip():
            continue
        if re.match(r"^_Z\w+:$", s):
            cur = (s[:-1], [], {})
            funcs.append(cur)
            continue
        if cur is None:
            continue
        if s.startswith(".Lfunc_end"):
            cur = None
            continue
        m = re.match(r"^(\.LBB\w+):", s)
        if m:
            cur[2][m.group(1)] = len(cur[1])
            continue
        t = s.strip()
        if not t.startswith("."):
            op, _, rest = t.partition(" ")
            cur[1].append((op, rest.strip()))
    return funcs


def _reads_writes(op: str, rest: str):
    if op.startswith("s_") or not rest:
        return set(), set()
    ops = [o.strip() for o in re.split(r",(?![^\[]*\])", rest)]
    if op.startswith(_STORES):
        return _regs(" ".join(ops)), set()
    return _regs(" ".join(ops[1:])), _regs(ops[0])


def _early_reads(name, ins, labels):
    found = []
    for i, (op, rest) in enumerate(ins):
        if op not in PASSES:
            continue
        need = PASSES[op] + MARGIN
        stack, seen = [(i + 1, 0, frozenset(_regs(rest.split(",")[0])))], set()
        while stack:
            j, ws, live = stack.pop()
            while j < len(ins) and ws < need and live and (j, ws, live) not in seen:
                seen.add((j, ws, live))
                op2, rest2 = ins[j]
                if op2.startswith("v_mfma"):
                    live = live - _regs(rest2.split(",")[0])  # a chained MFMA takes over
                else:
                    rd, wr = _reads_writes(op2, rest2)
                    if rd & live:
                        found.append(f"{name}: {op} #{i} read by {op2} #{j} after {ws} wait states "
                                     f"(needs {need})")
                    live = live - wr
                ws += int(rest2.split()[0]) + 1 if op2 == "s_nop" else 1
                if op2 == "s_branch":
                    j = labels[rest2.split()[0]]
                    continue
                if op2.startswith("s_cbranch"):
                    stack.append((labels[rest2.split()[0]], ws, live))
                if op2 in ("s_endpgm", "s_setpc_b64"):
                    break
                j += 1
    return found


def _assemble(src):
    out = OUT / (src.stem + ".s")
    cmd = [HIPCC, *build_native.FLAGS, "-I", str(CSRC), "-S", "--cuda-device-only", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_no_mfma_result_is_read_early():
    OUT.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        files = list(pool.map(_assemble, sorted(CSRC.glob("*.hip"))))
    found, mfmas = [], 0
    for path in files:
        for name, ins, labels in _functions(path):
            mfmas += sum(op in PASSES for op, _ in ins)
            found += _early_reads(name, ins, labels)
    assert mfmas > 1000, "no MFMAs found: the assembly parser no longer matches the compiler's output"
    assert not found, "\n".join(found[:20])


def test_the_check_catches_a_read_behind_a_branch():
    """The path walk sees a read on the taken side of a branch."""
    ins = [("v_mfma_f32_32x32x2_f32", "a[0:15], v1, v2, a[0:15]"),
           ("s_cbranch_scc1", ".LBB0_2"),
           ("s_nop", "15"), ("s_nop", "1"),
           ("v_accvgpr_read_b32", "v3, a15")]
    assert _early_reads("k", ins, {".LBB0_2": 4})
    assert not _early_reads("k", ins[:1] + ins[2:], {})
