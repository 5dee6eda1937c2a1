"""Scans the built library's gfx950 machine code for one hardware hazard.

A VALU instruction that rewrites the data registers of a vector-memory store of
more than 64 bits, as the very next instruction, can change the data the store
writes: on MI355X the first dword of some lanes of a 128-bit buffer store took
the value the next instruction wrote (wrong split-k partial tiles in a few
outputs per launch).  The compiler inserts no wait for buffer stores with a
register soffset, so the library's kernels keep such data registers unwritten
for two wait states themselves.  This test disassembles the library's own code
objects (built here from this repository's sources) and fails on any store of
more than 64 bits followed directly by a VALU write of one of its data
registers.  CPU only: it needs the built library and llvm-objdump.
"""

import os
import re
import shutil
import struct
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(os.path.dirname(HERE), "flash-train_amd", "flash_train", "libflash_train.so")
ROCM_LLVM = "/opt/rocm/llvm/bin"
STORE = re.compile(r"^(buffer|global|flat|scratch)_store_(dwordx3|dwordx4|b96|b128)\b")


def tool(name: str):
    path = os.path.join(ROCM_LLVM, name)
    return path if os.path.exists(path) else shutil.which(name)


def code_objects(so: str) -> list:
    """The gfx950 code objects of every offload bundle in the library's .hip_fatbin section."""
    out = subprocess.run([tool("llvm-readelf"), "-S", "-W", so], capture_output=True, text=True, check=True).stdout
    m = re.search(r"\.hip_fatbin\s+PROGBITS\s+[0-9a-f]+\s+([0-9a-f]+)\s+([0-9a-f]+)", out)
    assert m, "no .hip_fatbin section"
    off, size = int(m.group(1), 16), int(m.group(2), 16)
    with open(so, "rb") as f:
        f.seek(off)
        data = f.read(size)
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    objs, pos = [], 0
    while (i := data.find(magic, pos)) >= 0:
        (entries,) = struct.unpack_from("<Q", data, i + len(magic))
        p = i + len(magic) + 8
        for _ in range(entries):
            e_off, e_size, t_size = struct.unpack_from("<QQQ", data, p)
            p += 24
            triple = data[p:p + t_size].decode()
            p += t_size
            if "gfx950" in triple:
                objs.append(data[i + e_off:i + e_off + e_size])
        pos = i + 1
    return objs


def vregs(op: str) -> set:
    op = op.strip()
    m = re.match(r"v\[(\d+):(\d+)\]$", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op)
    return {int(m.group(1))} if m else set()


def hazards(disasm: str) -> list:
    """(store, next instruction) pairs where the next instruction is a VALU writing a data VGPR."""
    insts = []
    for line in disasm.splitlines():
        line = line.split("//")[0].strip()
        if not line or line.endswith(":") or line.startswith((".", "Disassembly")) or "file format" in line:
            continue
        insts.append(line)
    found = []
    for a, b in zip(insts, insts[1:]):
        mnem, _, ops = a.partition(" ")
        if not STORE.match(mnem):
            continue
        operands = [o.strip() for o in ops.split(",")]
        data = vregs(operands[0] if mnem.startswith("buffer") else operands[1])
        nm, _, nops = b.partition(" ")
        if nm.startswith("v_") and nops:
            dst = vregs(nops.split(",")[0])
            if dst & data:
                found.append((a, b))
    return found


def test_no_valu_write_of_store_data_right_after_a_wide_store():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing; run `python flash-train_amd/build.py`")
    if tool("llvm-objdump") is None or tool("llvm-readelf") is None:
        pytest.skip("llvm-objdump / llvm-readelf not available")
    objs = code_objects(LIB)
    assert objs, "no gfx950 code objects in the library"
    bad, stores = [], 0
    with tempfile.TemporaryDirectory() as tmp:
        for i, obj in enumerate(objs):
            path = os.path.join(tmp, f"co{i}.o")
            with open(path, "wb") as f:
                f.write(obj)
            dis = subprocess.run([tool("llvm-objdump"), "-d", "--no-show-raw-insn", "--mcpu=gfx950", path],
                                 capture_output=True, text=True, check=True).stdout
            stores += sum(1 for line in dis.splitlines() if STORE.match(line.strip()))
            bad += hazards(dis)
    assert stores > 0, "found no wide stores at all: the disassembly was not parsed"
    assert not bad, bad[:5]


def test_the_scan_flags_the_pattern():
    dis = "\n".join([
        "\tbuffer_store_dwordx4 v[0:3], v7, s[8:11], s2 offen",
        "\tv_cndmask_b32_e64 v0, v6, v5, s[0:1]",
        "\tbuffer_store_dwordx4 v[4:7], v7, s[8:11], s2 offen",
        "\ts_nop 1",
        "\tv_mov_b32_e32 v4, v9",
        "\tglobal_store_dwordx4 v2, v[8:11], s[0:1]",
        "\tv_mov_b32_e32 v2, 0",
    ])
    found = hazards(dis)
    assert len(found) == 1 and found[0][1].startswith("v_cndmask_b32_e64 v0")
