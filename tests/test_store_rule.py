"""CPU check of the rule the step runner's acquire-only fence mode rests on,
on the device code objects as built: every global store of the library's
kernels is an agent-scope (sc1) store -- except the streaming-read probe's
sink, which only the host reads -- and no store is left between a kernel's
last full wait (s_waitcnt vmcnt(0)) and an s_endpgm.  Read from the AMD
disassembly of the code objects this repository builds."""
import functools
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from _util import pkg

OBJDUMP = shutil.which("llvm-objdump") or "/opt/rocm/llvm/bin/llvm-objdump"
STORE = re.compile(r"^(global|buffer|flat)_(store|atomic)\w*")
HOST_READ_ONLY = ("read_probe_kernel",)  # kernels whose stores only the host reads


@functools.lru_cache(maxsize=None)
def _disassemble(path: Path) -> dict:
    out = subprocess.run([OBJDUMP, "-d", str(path)], capture_output=True, text=True,
                         check=True).stdout
    funcs, name = {}, None
    for line in out.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:", line)
        if m:
            name = m.group(1)
            funcs[name] = []
            continue
        ins = line.strip().split("//")[0].strip()
        if name and ins:
            funcs[name].append(ins)
    return funcs


def _code_objects():
    build = pkg("native.build")
    paths = build.code_object_paths()
    if not Path(OBJDUMP).exists() or not all(p.exists() for p in paths):
        pytest.skip("llvm-objdump or the built code objects are missing")
    return paths


def plain_stores(funcs: dict) -> list:
    """(kernel, instruction) of every global store without sc1."""
    return [(name, ins) for name, lines in funcs.items()
            if not any(h in name for h in HOST_READ_ONLY)
            for ins in lines if STORE.match(ins) and not re.search(r"\bsc1\b", ins)]


def unwaited_ends(funcs: dict) -> tuple:
    """(number of s_endpgm, kernels with a store after the last vmcnt(0)
    wait before one of them), scanning back from each s_endpgm."""
    ends, late = 0, []
    for name, lines in funcs.items():
        for i, ins in enumerate(lines):
            if not ins.startswith("s_endpgm"):
                continue
            ends += 1
            for prev in reversed(lines[:i]):
                if prev.startswith("s_endpgm") or (prev.startswith("s_waitcnt")
                                                    and "vmcnt(0)" in prev):
                    break
                if STORE.match(prev) and not any(h in name for h in HOST_READ_ONLY):
                    late.append(name)
                    break
    return ends, late


def test_the_scan_finds_planted_mistakes():
    funcs = {"ok": ["global_store_short v0, v1, s[2:3] sc1", "s_waitcnt vmcnt(0)", "s_endpgm"],
             "plain": ["global_store_dword v0, v1, s[2:3]", "s_waitcnt vmcnt(0)", "s_endpgm"],
             "late": ["global_store_dword v0, v1, s[2:3] sc1", "s_endpgm"]}
    assert plain_stores(funcs) == [("plain", "global_store_dword v0, v1, s[2:3]")]
    assert unwaited_ends(funcs) == (3, ["late"])


def test_every_store_is_agent_scope():
    plain = [(p.name, n[:80], ins) for p in _code_objects()
             for n, ins in plain_stores(_disassemble(p))]
    assert not plain, f"stores without sc1: {plain[:5]}"


def test_stores_complete_before_every_kernel_end():
    ends, late = 0, []
    for path in _code_objects():
        e, l = unwaited_ends(_disassemble(path))
        ends += e
        late += [(path.name, n[:80]) for n in l]
    assert ends > 100
    assert not late, f"a store not waited for before s_endpgm: {late[:5]}"
