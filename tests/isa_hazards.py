"""Scan gfx950 assembly for uses of a VGPR whose load is still in flight.

The page-streaming decode kernel issues its K loads as inline assembly (the
compiler's own wait analysis would stall the pipeline) and waits for them
with explicit ``s_waitcnt vmcnt`` instructions.  That is only correct if the
compiler never reads, copies or overwrites such a register before the wait:
a register copy at a branch join, for instance, would move stale data.  This
module walks a kernel's instructions in order, keeps the queue of
outstanding vector-memory operations that ``vmcnt`` counts (loads in order,
stores and direct-to-LDS loads as entries without registers) and reports
every instruction that touches a destination register of a load that no
wait has retired yet.  The walk is linear (branches are read in layout
order, a path ends at each s_endpgm), which is exact for the straight-line
pipeline of that kernel.
"""
from __future__ import annotations

import re

_VMEM_LOAD = ("buffer_load", "global_load", "scratch_load", "flat_load")
_VMEM_OTHER = ("buffer_store", "global_store", "scratch_store", "flat_store", "buffer_atomic", "global_atomic")


def _vregs(token: str) -> set[int]:
    m = re.match(r"v\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", token)
    return {int(m.group(1))} if m else set()


def kernel_lines(asm: str, symbol: str) -> list[str]:
    """The kernel's instructions, entry to the end of the function (every
    s_endpgm of its early exits included)."""
    lines = asm.split("\n")
    start = next(i for i, l in enumerate(lines) if l.startswith(symbol + ":"))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
    return lines[start:end]


def in_flight_uses(lines: list[str]) -> list[str]:
    """Instructions that touch a register of a load not yet waited for."""
    pending: list[set[int]] = []
    found = []
    for raw in lines:
        text = raw.split(";")[0].strip()
        if not text or text.startswith(".") or text.endswith(":"):
            continue
        op = text.split()[0]
        if op == "s_endpgm":  # a path ends; the next instruction starts another
            pending.clear()
            continue
        args = [a.strip() for a in text[len(op):].split(",")]
        wait = re.match(r"s_waitcnt\s+(?:.*\s)?vmcnt\((\d+)\)", text)
        if wait:
            keep = int(wait.group(1))
            del pending[:max(0, len(pending) - keep)]
            continue
        touched = set()
        for a in args:
            if a:
                touched |= _vregs(a.split()[0])
        if op.startswith(_VMEM_LOAD):
            dst = set() if text.endswith(" lds") else _vregs(args[0])
            srcs = set().union(*(_vregs(a.split()[0]) for a in args[1:] if a)) if len(args) > 1 else set()
            if any((dst | srcs) & p for p in pending):
                found.append(text)
            pending.append(dst)
            continue
        if op.startswith(_VMEM_OTHER):
            if any(touched & p for p in pending):
                found.append(text)
            pending.append(set())
            continue
        if any(touched & p for p in pending):
            found.append(text)
    return found


# ---------------------------------------------------------------------------
# VALU write of an SGPR followed too closely by a vector-memory instruction
# that reads it.  gfx9-family parts (gfx950 included) need 5 wait states
# between a VALU instruction that writes an SGPR (v_readlane,
# v_readfirstlane, a VOP3 compare or carry-out) and a VMEM instruction that
# reads that SGPR as its resource descriptor, soffset or saddr; otherwise the
# memory instruction can use the old value.  The compiler pads its own
# instructions, but not a VMEM instruction written as inline assembly: there
# a stale descriptor base sends the access to an unrelated address.

_VMEM_ANY = ("buffer_", "global_", "flat_", "scratch_")
_VALU_SGPR_CARRY = ("v_add_co", "v_sub_co", "v_subrev_co", "v_addc_co", "v_subb_co", "v_subbrev_co",
                    "v_div_scale", "v_mad_u64", "v_mad_i64")
VMEM_SGPR_WAIT_STATES = 5


def _sregs(token: str) -> set[int]:
    m = re.match(r"s\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", token)
    return {int(m.group(1))} if m else set()


def vmem_sgpr_hazards(lines: list[str]) -> list[tuple[str, int]]:
    """(VMEM instruction, wait states since the VALU write) for every VMEM
    instruction that reads an SGPR written by a VALU instruction fewer than
    5 wait states earlier.  Linear walk in layout order; a label resets
    nothing (conservative across fall-through), s_nop N counts N + 1."""
    recent: list[tuple[set[int], int]] = []
    found = []
    for raw in lines:
        text = raw.split(";")[0].strip()
        if not text or text.startswith(".") or text.endswith(":"):
            continue
        op = text.split()[0]
        args = [a.strip() for a in text[len(op):].split(",")]
        if op.startswith(_VMEM_ANY):
            reads = set()
            for a in args:
                if a:
                    reads |= _sregs(a.split()[0])
            for written, states in recent:
                if written & reads and states < VMEM_SGPR_WAIT_STATES:
                    found.append((text, states))
        m = re.match(r"s_nop\s+(\d+)", text)
        step = int(m.group(1)) + 1 if m else 1
        recent = [(w, s + step) for w, s in recent if s + step < VMEM_SGPR_WAIT_STATES]
        if op.startswith("v_") and args and args[0]:
            dst = _sregs(args[0].split()[0])
            if len(args) > 1 and op.startswith(_VALU_SGPR_CARRY):
                dst |= _sregs(args[1].split()[0])
            if dst:
                recent.append((dst, 0))
    return found


_RET_ATOMIC = re.compile(r"^(global|buffer|flat)_atomic_\S+\s.*\bsc0\b")
_SC1_STORE = re.compile(r"^(global|buffer|flat)_store\S*\s.*\bsc1\b")
_SC1_LOAD = re.compile(r"^(global|buffer|flat)_load\S*\s.*\bsc1\b")
_VMCNT0 = re.compile(r"^s_waitcnt\s.*\bvmcnt\(0\)")


def _instructions(lines: list[str]) -> list[str]:
    out = []
    for raw in lines:
        text = raw.split(";")[0].strip()
        if text and not text.startswith(".") and not text.endswith(":"):
            out.append(text)
    return out


def split_kv_order(lines: list[str]) -> tuple[list[str], int]:
    """The split-KV arrival protocol in a kernel's instructions (layout
    order).  For every returning atomic (an arrival): the device-coherent
    (sc1) partial stores before it must be complete -- an s_waitcnt
    vmcnt(0) and a workgroup barrier between the last of them and the
    atomic -- and the first sc1 load after it (a merge reading the
    partials) must come after an s_waitcnt vmcnt(0) (the atomic's returned
    count) and a barrier (its broadcast to the workgroup).  Returns the
    violations and the number of (arrival, merge load) pairs checked."""
    ins = _instructions(lines)
    bad, pairs = [], 0
    for i, t in enumerate(ins):
        if not _RET_ATOMIC.match(t):
            continue
        stores = [j for j in range(i) if _SC1_STORE.match(ins[j])]
        if stores:
            between = ins[stores[-1] + 1:i]
            if not any(_VMCNT0.match(x) for x in between) or "s_barrier" not in between:
                bad.append(f"arrival '{t}' not preceded by a wait and a barrier after '{ins[stores[-1]]}'")
        load = next((k for k in range(i + 1, len(ins)) if _SC1_LOAD.match(ins[k])), None)
        if load is not None:
            pairs += 1
            between = ins[i + 1:load]
            if not any(_VMCNT0.match(x) for x in between) or "s_barrier" not in between:
                bad.append(f"merge load '{ins[load]}' issued before the arrival '{t}' returned")
    return bad, pairs


def kernel_symbols(asm: str) -> list[str]:
    """Names of the kernel functions in an assembly listing."""
    return re.findall(r"^\s*\.type\s+(\S+),@function", asm, flags=re.M)
