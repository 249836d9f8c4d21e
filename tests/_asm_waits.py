"""Static check of the library's gfx950 assembly: no instruction may read or overwrite a
VGPR whose LDS or vector-memory load can still be in flight.

Kernels here issue LDS reads from inline asm and wait for them with hand-counted
``s_waitcnt`` statements.  Such a wait orders memory operations only: the compiler may
still schedule a plain VALU use of the loaded registers above it unless the wait (or an
empty asm after it) names those registers.  This module replays each kernel's
instructions in program order, modelling the two in-order counters:

* every ``ds_*`` instruction (and ``s_load``, which also counts in lgkmcnt) joins the LDS
  queue, every vector-memory load / store / LDS copy joins the VMEM queue;
* ``s_waitcnt lgkmcnt(N)`` / ``vmcnt(N)`` retire all but the newest N entries of a queue;
* any instruction whose sources or destinations meet the destination registers of a
  queued (not yet retired) load issued from inline asm is reported.

Loads the compiler emitted itself are waited for by the compiler; they take part in the
counting but are not checked (the file-order walk would otherwise report uses on the
other side of a branch).  Branches are followed in file order: the loop bodies with
hand-counted waits are straight-line after unrolling.
"""
from __future__ import annotations

import re
import subprocess
from typing import Iterable

_RANGE = re.compile(r"([vas])\[(\d+):(\d+)\]")
_SINGLE = re.compile(r"([vas])(\d+)")


def _regs(tok: str) -> set:
    tok = tok.strip()
    m = _RANGE.fullmatch(tok)
    if m:
        return {f"{m.group(1)}{r}" for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    return {tok} if _SINGLE.fullmatch(tok) else set()


def _all_regs(toks: Iterable[str]) -> set:
    out = set()
    for t in toks:
        out |= _regs(t)
    return out


def kernels(asm: str) -> dict:
    """Kernel symbol -> list of (instruction, from inline asm) (comments and directives dropped)."""
    out, cur, in_asm = {}, None, False
    for line in asm.splitlines():
        if re.match(r"^_Z\w+:", line):
            cur = line.split(":")[0]
            out[cur] = []
            continue
        if cur is None:
            continue
        if line.startswith(".Lfunc_end"):
            cur = None
            continue
        if ";;#ASMSTART" in line:
            in_asm = True
            continue
        if ";;#ASMEND" in line:
            in_asm = False
            continue
        s = line.split(";")[0].strip()
        if s and not s.startswith(".") and not s.endswith(":"):
            out[cur].append((s, in_asm))
    return out


def inflight_uses(instrs: list) -> list:
    """Instructions that touch registers of an inline-asm load that may still be in flight.

    ``instrs``: instruction strings (all treated as inline asm) or (instruction, from_asm) pairs.
    """
    lds, vm, issues = [], [], []
    for n, item in enumerate(instrs):
        s, tracked = (item, True) if isinstance(item, str) else item
        parts = s.split(None, 1)
        op = parts[0]
        args = [a.split()[0] for a in re.split(r",\s*", parts[1]) if a.strip()] if len(parts) > 1 else []
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", s)
            if m:
                k = int(m.group(1))
                lds = lds[len(lds) - k:] if 0 < k < len(lds) else ([] if k == 0 else lds)
            m = re.search(r"vmcnt\((\d+)\)", s)
            if m:
                k = int(m.group(1))
                vm = vm[len(vm) - k:] if 0 < k < len(vm) else ([] if k == 0 else vm)
            continue
        if op.startswith("s_"):
            if op.startswith("s_load") or op.startswith("s_buffer_load"):
                lds.append((set(), n, s))
            continue
        dst, src = set(), set()
        is_lds_copy = op.startswith("global_load_lds") or (op.startswith("buffer_load") and " lds" in s)
        if op.startswith("ds_write") or op.startswith("global_store") or op.startswith("buffer_store") or is_lds_copy:
            src = _all_regs(args)
        elif op.startswith("ds_") or op.startswith("global_load") or op.startswith("buffer_load") \
                or op.startswith("flat_load") or op.startswith("v_"):
            if args:
                dst, src = _regs(args[0]), _all_regs(args[1:])
        for regs, at, text in lds + vm:
            hit = regs & (src | dst)
            if hit:
                issues.append(f"{s}  touches {sorted(hit)[:4]} of in-flight [{text}] (instr {at})")
        if op.startswith("ds_"):
            lds.append((dst if tracked else set(), n, s))
        elif op.startswith(("global_load", "buffer_load", "flat_load", "global_store", "buffer_store")):
            vm.append((set() if is_lds_copy or not tracked else dst, n, s))
    return issues


def device_asm(source: str, include_dirs: list, hipcc: str = "/opt/rocm/bin/hipcc") -> str:
    """gfx950 device assembly of one HIP source, with the library's flags."""
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-S", "--cuda-device-only", "-o", "-", source]
    cmd[1:1] = [f"-I{d}" for d in include_dirs]
    res = subprocess.run(cmd, capture_output=True, text=True, check=True)
    return res.stdout
