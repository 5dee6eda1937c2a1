"""Scans the built library's gfx950 machine code for a hardware hazard and the deep-k split protocol.

Store-data hazard: a VALU instruction that rewrites the data registers of a
vector-memory store of more than 64 bits too soon after the store can change
the data the store writes: on MI355X the first dword of some lanes of a
128-bit buffer store took the value the next instruction wrote (wrong split-k
partial tiles in a few outputs per launch).  The compiler inserts no wait for
buffer stores with a register soffset, so the library's kernels keep such data
registers unwritten for two wait states themselves (`s_nop 1`).  The scan
counts wait states after every wide store (`s_nop N` gives N + 1, any other
instruction 1) and fails on a VALU write of a data register before two have
passed.

Deep-k protocol: the in-launch split-k reduction of the deep-k kernel relies on
agent-scope (L2-coherent across XCDs) encodings of its partial-tile stores and
loads, on a returning atomic for the arrival count, and on a full vector-memory
wait before the arrival; the scan checks each in the built code.

CPU only: it needs the built library and llvm-objdump.
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


def instructions(disasm: str) -> list:
    """The instruction lines of an llvm-objdump listing, comments and labels dropped."""
    insts = []
    for line in disasm.splitlines():
        line = line.split("//")[0].strip()
        if not line or line.endswith(":") or line.startswith((".", "Disassembly")) or "file format" in line:
            continue
        insts.append(line)
    return insts


def wait_states(inst: str) -> int:
    """Wait states an instruction provides: `s_nop N` gives N + 1, anything else 1."""
    m = re.match(r"s_nop\s+(\d+)", inst)
    return int(m.group(1)) + 1 if m else 1


# A wide store's data VGPRs must not be rewritten by a VALU within this many
# wait states of the store (gfx940+ hazard on the store-data read).
STORE_DATA_WAIT_STATES = 2


def hazards(disasm: str) -> list:
    """(store, instruction) pairs where a VALU writes a data VGPR of a wide store too soon after it."""
    insts = instructions(disasm)
    found = []
    for i, a in enumerate(insts):
        mnem, _, ops = a.partition(" ")
        if not STORE.match(mnem):
            continue
        operands = [o.strip() for o in ops.split(",")]
        data = vregs(operands[0] if mnem.startswith("buffer") else operands[1])
        elapsed = 0
        for b in insts[i + 1:]:
            if elapsed >= STORE_DATA_WAIT_STATES:
                break
            nm, _, nops = b.partition(" ")
            if nm.startswith("v_") and nops and vregs(nops.split(",")[0]) & data:
                found.append((a, b))
                break
            elapsed += wait_states(b)
    return found


def disassemble_all(so: str) -> list:
    """llvm-objdump listings of every gfx950 code object in the library."""
    out = []
    with tempfile.TemporaryDirectory() as tmp:
        for i, obj in enumerate(code_objects(so)):
            path = os.path.join(tmp, f"co{i}.o")
            with open(path, "wb") as f:
                f.write(obj)
            out.append(subprocess.run([tool("llvm-objdump"), "-d", "--no-show-raw-insn", "--mcpu=gfx950", path],
                                      capture_output=True, text=True, check=True).stdout)
    return out


def function_body(disasm: str, needle: str) -> str:
    """The listing of the first function whose symbol contains `needle`, up to the next symbol."""
    lines, body, inside = disasm.splitlines(), [], False
    for line in lines:
        if re.match(r"^[0-9a-f]+ <.*>:$", line):
            if inside:
                break
            inside = needle in line
            continue
        if inside:
            body.append(line)
    return "\n".join(body)


def deepk_protocol_violations(body: str) -> list:
    """Checks the deep-k kernel's last-arrival split-k protocol in its gfx950 code.

    The kernel (csrc/gemm/deepk_tile.hpp, `deepk_gemm_body`) publishes its
    64x64 partial tile with agent-scope relaxed stores, waits for them
    (`s_waitcnt vmcnt(0)`), meets its workgroup at a barrier, and counts its
    arrival with one atomic add that returns the old value; the last arrival
    reads the other partials with agent-scope relaxed loads and resets the
    counter with an agent-scope store.  On gfx950 an agent-scope access is a
    plain global access with the `sc1` bit (it misses the XCD's own L2 on
    loads and writes through it on stores), which is what makes a partial
    written on one XCD readable on another without a cache writeback or
    invalidate.  A relaxed read-modify-write at workgroup or agent scope is
    the same returning atomic (`sc0` = return the old value, no `sc1`); a
    system-scope one adds `sc1`.  Returns the violations found (empty = the
    protocol is intact).
    """
    insts = instructions(body)
    bad = []
    atom = [i for i, x in enumerate(insts) if x.startswith("global_atomic_add ")]
    if len(atom) != 1:
        return [f"expected one arrival atomic, found {len(atom)}"]
    ia = atom[0]
    if not re.search(r"\bsc0\b", insts[ia]) or re.search(r"\bsc1\b", insts[ia]):
        bad.append(f"arrival atomic is not an agent-scope returning add: {insts[ia]}")
    pre = [(i, x) for i, x in enumerate(insts[:ia]) if re.match(r"global_store_dword(x2|x3|x4|)\b", x)]
    if len(pre) != 8:
        bad.append(f"expected 8 64-bit partial stores before the arrival, found {len(pre)}: {[x for _, x in pre]}")
    for _, x in pre:
        if not x.startswith("global_store_dwordx2 ") or not re.search(r"\bsc1\b", x):
            bad.append(f"partial store is not an agent-scope 64-bit store: {x}")
    if pre:
        last = pre[-1][0]
        tail = insts[last + 1:ia]
        w = next((j for j, x in enumerate(tail) if x.startswith("s_waitcnt") and (
            "vmcnt(0)" in x or re.fullmatch(r"s_waitcnt\s+0", x))), None)
        b = next((j for j, x in enumerate(tail) if x.startswith("s_barrier")), None)
        if w is None or b is None or w > b:
            bad.append("no s_waitcnt vmcnt(0) then s_barrier between the partial stores and the arrival")
    gathers = [x for x in insts[ia + 1:] if x.startswith("global_load_dwordx2 ")]
    if len(gathers) < 8:
        bad.append(f"expected the last arrival's 64-bit partial loads, found {len(gathers)}")
    for x in gathers:
        if not re.search(r"\bsc1\b", x):
            bad.append(f"partial load is not agent-scope: {x}")
    resets = [x for x in insts[ia + 1:] if x.startswith("global_store_dword ")]
    if len(resets) != 1 or not re.search(r"\bsc1\b", resets[0]):
        bad.append(f"expected one agent-scope 32-bit counter reset, found {resets}")
    return bad


def built_listings() -> list:
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing; run `python flash-train_amd/build.py`")
    if tool("llvm-objdump") is None or tool("llvm-readelf") is None:
        pytest.skip("llvm-objdump / llvm-readelf not available")
    listings = disassemble_all(LIB)
    assert listings, "no gfx950 code objects in the library"
    return listings


def test_no_valu_write_of_store_data_right_after_a_wide_store():
    bad, stores = [], 0
    for dis in built_listings():
        stores += sum(1 for line in dis.splitlines() if STORE.match(line.strip()))
        bad += hazards(dis)
    assert stores > 0, "found no wide stores at all: the disassembly was not parsed"
    assert not bad, bad[:5]


def test_deepk_split_protocol_in_the_built_code():
    bodies = [function_body(dis, "deepk_gemm") for dis in built_listings()]
    bodies = [b for b in bodies if b.strip()]
    assert len(bodies) == 1, "expected the deep-k kernel in exactly one code object"
    assert deepk_protocol_violations(bodies[0]) == []


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


def test_the_scan_counts_wait_states():
    weak = "\n".join([
        "\tbuffer_store_dwordx4 v[0:3], v7, s[8:11], s2 offen",
        "\ts_nop 0",
        "\tv_mov_b32_e32 v1, v9",
    ])
    assert len(hazards(weak)) == 1
    salu = "\n".join([
        "\tglobal_store_dwordx4 v2, v[8:11], s[0:1]",
        "\ts_mov_b32 s4, 0",
        "\tv_mov_b32_e32 v9, 0",
    ])
    assert len(hazards(salu)) == 1
    enough = "\n".join([
        "\tglobal_store_dwordx4 v2, v[8:11], s[0:1]",
        "\ts_mov_b32 s4, 0",
        "\ts_mov_b32 s5, 0",
        "\tv_mov_b32_e32 v9, 0",
    ])
    assert hazards(enough) == []


PROTOCOL_OK = """
\tglobal_store_dwordx2 v162, v[14:15], s[0:1] sc1
\tglobal_store_dwordx2 v162, v[16:17], s[0:1] offset:2048 sc1
\tglobal_store_dwordx2 v[22:23], v[10:11], off offset:-4096 sc1
\tglobal_store_dwordx2 v[20:21], v[12:13], off offset:2048 sc1
\tglobal_store_dwordx2 v[22:23], v[6:7], off sc1
\tglobal_store_dwordx2 v[22:23], v[8:9], off offset:2048 sc1
\tglobal_store_dwordx2 v[18:19], v[2:3], off sc1
\tglobal_store_dwordx2 v[18:19], v[4:5], off offset:2048 sc1
\ts_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)
\ts_barrier
\tglobal_atomic_add v1, v1, v18, s[14:15] sc0
\ts_waitcnt vmcnt(0)
\ts_barrier
""" + "".join(f"\tglobal_load_dwordx2 v[{2*i}:{2*i+1}], v[0:1], off sc1\n" for i in range(8)) + """
\tglobal_store_dword v0, v0, s[0:1] sc1
\tglobal_store_dwordx4 v1, v[4:7], s[2:3]
"""


def test_the_protocol_check_flags_plain_accesses():
    assert deepk_protocol_violations(PROTOCOL_OK) == []
    cases = {
        "plain partial store": ("global_store_dwordx2 v[18:19], v[2:3], off sc1", "global_store_dwordx2 v[18:19], v[2:3], off"),
        "plain partial load": ("global_load_dwordx2 v[6:7], v[0:1], off sc1", "global_load_dwordx2 v[6:7], v[0:1], off"),
        "plain counter reset": ("global_store_dword v0, v0, s[0:1] sc1", "global_store_dword v0, v0, s[0:1]"),
        "non-atomic arrival": ("global_atomic_add v1, v1, v18, s[14:15] sc0", "global_load_dword v1, v18, s[14:15]"),
        "system-scope arrival": ("global_atomic_add v1, v1, v18, s[14:15] sc0", "global_atomic_add v1, v1, v18, s[14:15] sc0 sc1"),
        "no wait before the arrival": ("\ts_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)\n\ts_barrier\n\tglobal_atomic", "\ts_barrier\n\tglobal_atomic"),
    }
    for name, (old, new) in cases.items():
        assert old in PROTOCOL_OK, name
        assert deepk_protocol_violations(PROTOCOL_OK.replace(old, new, 1)), name
