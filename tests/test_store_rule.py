"""CPU check of the rule the step runner's acquire-only fence mode rests on,
on the device code objects as built: every global store of the library's
kernels is an agent-scope (sc1) store, and on every control-flow path from a
store to an s_endpgm there is a full wait (s_waitcnt vmcnt(0): on gfx9
targets vmcnt counts stores too).  Read from the AMD disassembly of the code
objects this repository builds; the scan follows branches (s_branch,
s_cbranch_*), so a store in a block that jumps to a shared s_endpgm is
checked on that path too."""
import functools
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from _util import pkg

OBJDUMP = shutil.which("llvm-objdump") or "/opt/rocm/llvm/bin/llvm-objdump"
STORE = re.compile(r"^(global|buffer|flat)_(store|atomic)\w*")
HEADER = re.compile(r"^([0-9a-f]+) <(.+)>:")
# "<mnemonic ...>  // <address>: <encoding> [<function+0xoffset>]"
COMMENT = re.compile(r"//\s*([0-9A-Fa-f]+):[^<]*(?:<(.+)\+0x([0-9a-f]+)>)?")


@functools.lru_cache(maxsize=None)
def _disassemble(path: Path) -> dict:
    """kernel name -> [(address, instruction, branch target address or None)]."""
    out = subprocess.run([OBJDUMP, "-d", str(path)], capture_output=True, text=True,
                         check=True).stdout
    funcs, name, base = {}, None, 0
    for line in out.splitlines():
        m = HEADER.match(line)
        if m:
            base, name = int(m.group(1), 16), m.group(2)
            funcs[name] = []
            continue
        if not name or "//" not in line:
            continue
        ins = line.split("//")[0].strip()
        c = COMMENT.search(line)
        if not ins or not c:
            continue
        target = base + int(c.group(3), 16) if c.group(2) == name else None
        funcs[name].append((int(c.group(1), 16), ins, target))
    return funcs


def _code_objects():
    build = pkg("native.build")
    paths = build.code_object_paths()
    have = Path(OBJDUMP).exists() and all(p.exists() for p in paths)
    if not have:
        if build.LIB.exists():  # a built library whose rule cannot be checked is a failure
            pytest.fail(f"libsmx.so is built but llvm-objdump ({OBJDUMP}) or a code object "
                        f"({[str(p) for p in paths if not p.exists()]}) is missing")
        pytest.skip("nothing is built")
    return paths


def plain_stores(funcs: dict) -> list:
    """(kernel, instruction) of every global store without sc1."""
    return [(name, ins) for name, lines in funcs.items()
            for _, ins, _ in lines if STORE.match(ins) and not re.search(r"\bsc1\b", ins)]


def _successors(lines, i, index):
    _, ins, target = lines[i]
    if ins.startswith("s_endpgm"):
        return []
    nxt = [i + 1] if i + 1 < len(lines) else []
    if ins.startswith("s_branch"):
        return [index[target]] if target in index else []
    if ins.startswith("s_cbranch"):
        return nxt + ([index[target]] if target in index else [])
    return nxt


def unwaited_ends(funcs: dict) -> tuple:
    """(number of s_endpgm, kernels where some path from a store reaches an
    s_endpgm without an s_waitcnt vmcnt(0) between them).  Forward dataflow
    over the kernel's control-flow graph: a store sets "pending", a full
    wait clears it, a join is pending if any incoming path is."""
    ends, late = 0, []
    for name, lines in funcs.items():
        index = {addr: i for i, (addr, _, _) in enumerate(lines)}
        n = len(lines)
        pending_in = [False] * n
        work = list(range(n))
        while work:
            i = work.pop()
            ins = lines[i][1]
            if STORE.match(ins):
                out = True
            elif ins.startswith("s_waitcnt") and "vmcnt(0)" in ins:
                out = False
            else:
                out = pending_in[i]
            for j in _successors(lines, i, index):
                if out and not pending_in[j]:
                    pending_in[j] = True
                    work.append(j)
        for i, (_, ins, _) in enumerate(lines):
            if ins.startswith("s_endpgm"):
                ends += 1
                if pending_in[i] and name not in late:
                    late.append(name)
    return ends, late


def _lines(*ins):
    """Planted kernels: instructions at 4-byte addresses, "-> k" marking a
    branch to instruction k."""
    out = []
    for i, s in enumerate(ins):
        tgt = None
        if " -> " in s:
            s, k = s.split(" -> ")
            tgt = 4 * int(k)
        out.append((4 * i, s, tgt))
    return out


def test_the_scan_finds_planted_mistakes():
    funcs = {"ok": _lines("global_store_short v0, v1, s[2:3] sc1", "s_waitcnt vmcnt(0)",
                          "s_endpgm"),
             "plain": _lines("global_store_dword v0, v1, s[2:3]", "s_waitcnt vmcnt(0)",
                             "s_endpgm"),
             "late": _lines("global_store_dword v0, v1, s[2:3] sc1", "s_endpgm"),
             # the fall-through path waits; the branch reaches a second s_endpgm
             # with the store still in flight
             "branchy": _lines("global_store_dword v0, v1, s[2:3] sc1", "s_cbranch_scc1 -> 4",
                               "s_waitcnt vmcnt(0)", "s_endpgm", "s_endpgm"),
             # a loop whose back edge carries a store past the wait to the exit
             "loop": _lines("s_waitcnt vmcnt(0)", "s_cbranch_scc0 -> 4",
                            "global_store_dword v0, v1, s[2:3] sc1", "s_branch -> 1",
                            "s_endpgm"),
             # every path waits: the branch target waits before its end
             "branchy_ok": _lines("global_store_dword v0, v1, s[2:3] sc1", "s_cbranch_scc1 -> 4",
                                  "s_waitcnt vmcnt(0)", "s_endpgm",
                                  "s_waitcnt vmcnt(0) lgkmcnt(0)", "s_endpgm")}
    assert plain_stores(funcs) == [("plain", "global_store_dword v0, v1, s[2:3]")]
    ends, late = unwaited_ends(funcs)
    assert ends == 8
    assert sorted(late) == ["branchy", "late", "loop"]


def test_the_parser_reads_branch_targets():
    paths = _code_objects()
    funcs = _disassemble(paths[0])
    branches = [(name, t) for name, lines in funcs.items() for _, ins, t in lines
                if ins.startswith(("s_branch", "s_cbranch"))]
    assert branches and all(t is not None for _, t in branches)
    addrs = {name: {a for a, _, _ in lines} for name, lines in funcs.items()}
    assert all(t in addrs[name] for name, t in branches)


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
    assert not late, f"a store not waited for before s_endpgm on some path: {late[:5]}"
