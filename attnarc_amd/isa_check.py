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
variant), it reports any later instruction that names a destination register
before the next wait on that load's counter (``lgkmcnt`` for scalar loads,
``vmcnt`` for vector loads).

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


def scan(asm: str, window: int = 600) -> list[str]:
    """Hazards in ``asm`` (AMDGPU assembly text), one line of text each."""
    lines = asm.split("\n")
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
        for j in range(i + 1, min(i + window, len(lines))):
            later = lines[j].split(";")[0]
            if "s_waitcnt" in later and counter in later:
                break
            if _named(later, kind) & dest:
                found.append(f"{func}: line {i + 1}: {code.strip()} -> line {j + 1}: {later.strip()}")
                break
    return found


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
