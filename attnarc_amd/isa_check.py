"""Check of the compiled decode kernels for early reads of in-flight loads.

The streaming kernels issue some loads from inline asm and wait for them
later (``s_waitcnt``), so that the memory latency overlaps other work. The
compiler does not know such a load is in flight. If it copies or spills the
destination register before the wait (a ``v_writelane_b32`` of an SGPR, a
``s_mov_b32``, any read), the copy holds the register's old contents. If it
writes the register, the load can land after that write and overwrite it.
Either way a wrong block ID or wrong data follows. A stale block ID addresses
the DMA out of bounds.

This tool compiles ``paged_decode_attention.hip`` to gfx950 assembly and
scans every kernel. For each load that stands inside an inline-asm region and
returns into registers (scalar ``s_load_dword*`` / ``s_buffer_load_dword*``,
vector ``global_load_dword*`` / ``buffer_load_dword*`` without the LDS
variant), it reports any instruction on a path from the load (through
branches and loop back-edges) that names a destination register before a
wait that completes the load: ``lgkmcnt(0)`` for scalar loads, which may
return out of order, and ``vmcnt(N)`` with at least N vector loads issued
after it for vector loads, which return in order.

Usage: ``python -m attnarc_amd.isa_check`` (about 2.5 minutes of compile),
or ``python -m attnarc_amd.isa_check FILE.s`` to scan assembly already made.
Exit status 1 when a hazard is found.
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile

_SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "paged_decode_attention.hip")
_INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")

_SCALAR_LOAD = re.compile(r"\s*(s_load_dword\w*|s_buffer_load_dword\w*)\s+(s\[\d+:\d+\]|s\d+),")
_VECTOR_LOAD = re.compile(r"\s*(global_load_dword\w*|buffer_load_dword\w*)\s+(v\[\d+:\d+\]|v\d+),")
_FUNC = re.compile(r"^(_Z\S+):")


def _reg_set(spec: str, kind: str) -> set[int]:
    m = re.fullmatch(kind + r"\[(\d+):(\d+)\]", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(kind + r"(\d+)", spec)
    return {int(m.group(1))} if m else set()


def _named(text: str, kind: str) -> set[int]:
    regs: set[int] = set()
    for m in re.finditer(kind + r"\[(\d+):(\d+)\]", text):
        regs |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\b" + kind + r"(\d+)\b", text):
        regs.add(int(m.group(1)))
    return regs


_VM_LOAD = re.compile(r"\s*(global_load\w*|buffer_load\w*|flat_load\w*)\b")
_WAIT = re.compile(r"\s*s_waitcnt\b(.*)")
_BRANCH = re.compile(r"\s*(s_branch|s_cbranch_\w+)\s+(\S+)")
_LABEL = re.compile(r"^(\.?[A-Za-z_][\w.$]*):")


def _wait_count(args: str, counter: str) -> int | None:
    """The N of ``counter(N)`` in an s_waitcnt's operands, or None."""
    m = re.search(counter + r"\((\d+)\)", args)
    return int(m.group(1)) if m else None


def _covers(kind: str, n: int, loads_after: int) -> bool:
    """Whether a wait for counter value n completes the load. Vector loads
    return in issue order, so vmcnt(n) completes every load with at least n
    loads issued after it; scalar loads may return out of order, so only
    lgkmcnt(0) completes a given one."""
    return n == 0 if kind == "s" else loads_after >= n


def scan(asm: str, window: int = 600) -> list[str]:
    """Hazards in ``asm`` (AMDGPU assembly text), one line of text each.

    From each inline-asm load into registers, every path is followed
    (branches to labels, taken and not taken, loop back-edges included) up to
    ``window`` instructions, counting the vector loads issued after it, until
    a wait completes the load; an instruction on the way that names a
    destination register is a hazard."""
    lines = asm.split("\n")
    labels = {}
    for i, line in enumerate(lines):
        m = _LABEL.match(line)
        if m:
            labels[m.group(1)] = i
    found: list[str] = []
    func = None
    in_asm = False
    for i, line in enumerate(lines):
        m = _FUNC.match(line)
        if m:
            func = m.group(1)
        if ";;#ASMSTART" in line:
            in_asm = True
        elif ";;#ASMEND" in line:
            in_asm = False
        if not in_asm:
            continue
        code = line.split(";")[0]
        ms, mv = _SCALAR_LOAD.match(code), _VECTOR_LOAD.match(code)
        if ms:
            kind, counter, dest = "s", "lgkmcnt", _reg_set(ms.group(2), "s")
        elif mv and "lds" not in code:
            kind, counter, dest = "v", "vmcnt", _reg_set(mv.group(2), "v")
        else:
            continue
        hit = _follow(lines, labels, i + 1, kind, counter, dest, window)
        if hit is not None:
            found.append(f"{func}: line {i + 1}: {code.strip()} -> line {hit + 1}: {lines[hit].split(';')[0].strip()}")
    return found


_ANDN2_VCC = re.compile(r"\s*s_andn2_b64\s+vcc,\s*exec,\s*(s\[\d+:\d+\])")


def _never_taken(lines, j) -> bool:
    """A branch the compiler emits with a constant condition: ``s_cbranch_vccnz``
    right after ``vcc = exec & ~s[a:b]`` where s[a:b] was last set to -1 in
    code reachable only by falling through from there (no label between:
    vcc = 0). The compiler writes this for a loop exit whose other side is
    decided elsewhere."""
    code = lines[j].split(";")[0]
    if "s_cbranch_vccnz" not in code:
        return False
    k = j - 1
    while k >= 0 and not lines[k].split(";")[0].strip():
        k -= 1
    m = _ANDN2_VCC.match(lines[k].split(";")[0]) if k >= 0 else None
    if not m:
        # one scalar move may sit between the two
        k -= 1
        m = _ANDN2_VCC.match(lines[k].split(";")[0]) if k >= 0 else None
        if not m:
            return False
    reg = m.group(1)
    for i in range(k - 1, max(-1, k - 200), -1):
        c = lines[i].split(";")[0]
        if _LABEL.match(lines[i]):  # a join: other paths may set the register
            return False
        if reg in c and re.match(r"\s*s_\w+\s+" + re.escape(reg) + r",", c):
            return bool(re.match(r"\s*s_mov_b64\s+" + re.escape(reg) + r",\s*-1\s*$", c))
    return False


def _follow(lines, labels, start, kind, counter, dest, window):
    """First line on any path from ``start`` that names a register of
    ``dest`` before a wait completes the load, or None."""
    best: dict[int, int] = {}  # line -> fewest loads-after seen there (revisit only with fewer)
    stack = [(start, 0, 0)]  # (line, loads issued after the load, instructions walked)
    while stack:
        j, after, steps = stack.pop()
        while j < len(lines) and steps < window:
            if j in best and best[j] <= after:
                break
            best[j] = after
            line = lines[j]
            if _FUNC.match(line) or ".Lfunc_end" in line:
                break
            code = line.split(";")[0]
            if not code.strip() or _LABEL.match(line):
                j += 1
                continue
            steps += 1
            w = _WAIT.match(code)
            if w:
                n = _wait_count(w.group(1), counter)
                if n is not None and _covers(kind, n, after):
                    break
            if _named(code, kind) & dest:
                return j
            if _VM_LOAD.match(code):
                after += 1
            b = _BRANCH.match(code)
            if b:
                target = labels.get(b.group(2))
                if target is not None and not _never_taken(lines, j):
                    stack.append((target, after, steps))
                if b.group(1) == "s_branch":
                    break  # unconditional: only the target continues
            if code.strip().startswith("s_endpgm"):
                break
            j += 1
    return None


def compile_asm(out_path: str) -> None:
    cmd = ["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", f"-I{_INCLUDE}", "--offload-device-only", "-S", _SRC, "-o", out_path]
    subprocess.run(cmd, check=True, stderr=subprocess.DEVNULL)


def main(argv: list[str]) -> int:
    if argv:
        asm = open(argv[0]).read()
    else:
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "paged_decode_attention.s")
            compile_asm(path)
            asm = open(path).read()
    found = scan(asm)
    for line in found:
        print(line)
    loads = sum(1 for ln in asm.split("\n") if _SCALAR_LOAD.match(ln.split(";")[0]) or _VECTOR_LOAD.match(ln.split(";")[0]))
    print(f"{len(found)} early reads or writes of in-flight loads ({loads} loads in the assembly)")
    return 1 if found else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
