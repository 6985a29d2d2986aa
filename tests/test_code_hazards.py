"""Wait states around the LDS-DMA loads of the built library (no GPU needed).

The kernels issue their global -> LDS loads (`global_load_lds_dword*`) from inline assembly, and
the compiler inserts no wait states for an instruction it cannot see. The gfx9 / CDNA ISA needs:
- five wait states between a VALU instruction that writes an SGPR (v_readfirstlane, v_readlane,
  a compare or carry-out with an SGPR destination) and a memory instruction that reads that
  SGPR, here the load's scalar base address or M0 (its LDS address); without them the load can
  use the register's previous value, i.e. a wrong address;
- one wait state between an SALU write of M0 and an LDS DMA that reads it.

This test disassembles the gfx950 code objects of build/libcuflash_attn.so with ROCm's
llvm-objdump and checks every LDS-DMA load against both rules, walking back from the load
through every control-flow predecessor (fall-through and branches into the window) until five
wait states are covered. It first checks itself on hand-written listings with and without each
hazard.

The forward and backward LDS-DMA helpers (common.hpp: lds_dma16_async, lds_dma16_async_s,
lds_dma4_async) carry a single `s_nop 0`, which covers the SALU write of M0 only. They are safe
because every base address and LDS address handed to them today is an SALU value (kernel
arguments, wave-uniform loop counters, readfirstlane of a uniform expression the compiler
places on the scalar unit). A future call site whose base comes from a lane (v_readlane,
v_readfirstlane of a divergent value) would need the five-wait-state form that decode.hip's
helpers use; this test is what catches such a call site, so it must stay in the CPU suite.
"""

from __future__ import annotations

import os
import re
import struct
import subprocess

import pytest

from conftest import REPO

LIB = os.path.join(REPO, "build", "libcuflash_attn.so")
LLVM = "/opt/rocm/llvm/bin"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

_INSN = re.compile(r"^\s+([a-z_0-9]+)\s*(.*?)\s*//\s*([0-9A-Fa-f]+):")
_SREG = re.compile(r"^s\[(\d+):(\d+)\]$|^s(\d+)$")
# VALU instructions whose second operand is an SGPR destination (carry or condition out).
_SDST1 = ("_co_", "v_div_scale", "v_mad_u64_u32", "v_mad_i64_i32")


def _regs(tok: str) -> set:
    tok = tok.strip()
    if tok == "m0":
        return {"m0"}
    m = _SREG.match(tok)
    if not m:
        return set()
    if m.group(3) is not None:
        return {int(m.group(3))}
    return set(range(int(m.group(1)), int(m.group(2)) + 1))


def _operands(text: str) -> list:
    return [t for t in (x.strip() for x in text.split(",")) if t]


def _first_token(op: str) -> str:
    return op.split()[0] if op else ""


def _sgpr_writes(mnem: str, ops: list) -> set:
    """SGPRs (and M0) that an instruction writes, for the kinds these rules concern."""
    if not ops:
        return set()
    if mnem.startswith("v_"):
        out = _regs(_first_token(ops[0]))
        if any(k in mnem for k in _SDST1) and len(ops) > 1:
            out |= _regs(_first_token(ops[1]))
        return out
    if mnem.startswith("s_") and _first_token(ops[0]) == "m0":
        return {"m0"}
    return set()


def parse(listing: str) -> list:
    """[(address, mnemonic, operands)] in layout order."""
    out = []
    for line in listing.splitlines():
        m = _INSN.match(line)
        if m:
            out.append((int(m.group(3), 16), m.group(1), _operands(m.group(2))))
    return out


def find_hazards(insns: list) -> tuple:
    """(number of LDS-DMA loads, [description of each violation])."""
    index = {a: i for i, (a, _, _) in enumerate(insns)}
    preds = {i: [] for i in range(len(insns))}
    for i, (addr, mnem, ops) in enumerate(insns):
        ends = mnem in ("s_branch", "s_endpgm", "s_setpc_b64") or mnem.startswith("s_trap")
        if i + 1 < len(insns) and not ends:
            preds[i + 1].append(i)
        if mnem == "s_branch" or mnem.startswith("s_cbranch_"):
            simm = int(_first_token(ops[0]), 0)
            simm = simm - 65536 if simm >= 32768 else simm
            target = addr + 4 + 4 * simm
            if target in index:
                preds[index[target]].append(i)

    def cost(i):
        mnem, ops = insns[i][1], insns[i][2]
        return int(_first_token(ops[0]), 0) + 1 if mnem == "s_nop" else 1

    loads = 0
    bad = []
    for i, (addr, mnem, ops) in enumerate(insns):
        if not mnem.startswith("global_load_lds"):
            continue
        loads += 1
        reads = {"m0"}
        if len(ops) > 1:
            reads |= _regs(_first_token(ops[1]))
        seen = set()
        stack = [(p, 0) for p in preds[i]]  # (instruction, wait states between it and the load)
        while stack:
            j, ws = stack.pop()
            if (j, ws) in seen or ws >= 5:
                continue
            seen.add((j, ws))
            jm, jo = insns[j][1], insns[j][2]
            w = _sgpr_writes(jm, jo) & reads
            if w and jm.startswith("v_"):
                bad.append(f"{addr:#x} {mnem} {', '.join(ops)}: {jm} at {insns[j][0]:#x} writes "
                           f"{sorted(map(str, w))} {ws} wait states before it (5 needed)")
            elif w and ws < 1:
                bad.append(f"{addr:#x} {mnem}: {jm} at {insns[j][0]:#x} writes M0 right before it")
            stack.extend((p, ws + cost(j)) for p in preds[j])
    return loads, bad


def _listing(lines):
    """A listing in llvm-objdump's format from (mnemonic and operands) strings."""
    return "\n".join(f"\t{text:<58}// {0x1000 + 4 * i:012X}: 00000000" for i, text in enumerate(lines))


def test_checker_finds_planted_hazards():
    hazard = ["s_mov_b32 m0, 0", "v_readfirstlane_b32 s5, v9", "v_readfirstlane_b32 s4, v8",
              "s_nop 0", "global_load_lds_dwordx4 v93, s[4:5] nt"]
    assert find_hazards(parse(_listing(hazard)))[0] == 1
    assert len(find_hazards(parse(_listing(hazard)))[1]) == 2
    fixed = hazard[:3] + ["s_nop 4"] + hazard[4:]
    assert find_hazards(parse(_listing(fixed))) == (1, [])
    # M0 written by the SALU right before the load; a VALU-written M0 three states before.
    assert len(find_hazards(parse(_listing(["s_mov_b32 m0, s3",
                                            "global_load_lds_dwordx4 v[2:3], off"])))[1]) == 1
    assert len(find_hazards(parse(_listing(["v_readfirstlane_b32 m0, v1", "s_nop 1",
                                            "global_load_lds_dwordx4 v[2:3], off"])))[1]) == 1
    # A carry-out SGPR of a VALU add used as the base.
    assert len(find_hazards(parse(_listing(["v_add_co_u32_e64 v1, s[6:7], v2, v3", "s_nop 2",
                                            "global_load_lds_dwordx4 v1, s[6:7]"])))[1]) == 1
    # The hazard reached only through a branch into the load's block: branch at 0x100c jumps
    # 3 instructions ahead (+4 + 4 * 2) to the load at 0x1018; the fall-through path is clean.
    branchy = ["v_readfirstlane_b32 s4, v8", "s_mov_b32 m0, 0", "s_nop 0", "s_branch 2",
               "s_mov_b32 s4, s9", "s_nop 4", "global_load_lds_dwordx4 v93, s[4:5]"]
    loads, bad = find_hazards(parse(_listing(branchy)))
    assert loads == 1 and len(bad) == 1 and "0x1000" in bad[0]
    # A VALU that only reads the SGPR is no hazard.
    assert find_hazards(parse(_listing(["v_lshl_add_u64 v[8:9], v[2:3], 0, s[4:5]",
                                        "s_nop 0", "global_load_lds_dwordx4 v9, s[4:5]"]))) == (1, [])


def _code_objects(tmp_path):
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}",
                    LIB, str(tmp_path / "lib.tmp")], check=True, capture_output=True)
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(BUNDLE_MAGIC), data)]
    objs = []
    for n, start in enumerate(starts):
        off = start + len(BUNDLE_MAGIC)
        (count,) = struct.unpack_from("<Q", data, off)
        off += 8
        for _ in range(count):
            entry_off, size, tlen = struct.unpack_from("<QQQ", data, off)
            off += 24
            triple = data[off:off + tlen].decode()
            off += tlen
            if "gfx950" in triple and size > 0:
                path = tmp_path / f"dev{n}.co"
                path.write_bytes(data[start + entry_off:start + entry_off + size])
                objs.append(path)
    return objs


def test_lds_dma_loads_of_the_built_library(tmp_path):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    if not os.path.exists(os.path.join(LLVM, "llvm-objdump")):
        pytest.skip("ROCm llvm-objdump not installed")
    objs = _code_objects(tmp_path)
    assert objs, "no gfx950 code object in the library"
    total = 0
    problems = []
    for co in objs:
        dis = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", str(co)],
                             check=True, capture_output=True, text=True).stdout
        loads, bad = find_hazards(parse(dis))
        total += loads
        problems += bad
    # Forward, backward and decode kernels: well over a thousand load sites.
    assert total > 1000, total
    assert not problems, "\n".join(problems[:20])
