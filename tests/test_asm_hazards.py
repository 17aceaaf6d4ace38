"""Wait-state checks over the gfx950 machine code of the built libpraghip.so.

The kernels use inline asm in two places where the compiler's hazard
recognizer cannot see a dependency:
* the carry-out products (modarith.hpp): a v_mad_u64_u32 writes its carry
  into an SGPR pair as a lane mask and a v_addc_co_u32 of another asm
  statement reads it as carry-in;
* the share GEMM's LDS DMA (gemm.hip): a scalar write of M0 followed by a
  global_load_lds_dwordx4 that reads it.

This test disassembles the library's own gfx950 code objects (llvm-objdump
from the ROCm toolchain) and checks, in straight-line code, every reader of
these two kinds against the last writer of its register:
* a VALU write of an SGPR lane mask (carry-out, compare result) is followed
  by at least two wait states before a VALU reads it as carry-in or select;
  the compiler leaves exactly that for its own code (s_nop 1, or s_nop 0 plus
  one instruction), so the same rule checks the asm and the compiler alike;
* a write of M0 is followed by at least one wait state before an LDS DMA.

A third check covers the LDS exchanges between transform passes (barrier,
writes, barrier, reads, barrier).  The compiler does not count s_barrier as
a memory access when it sinks loads into a successor block: with the values
read first used after a branch, it once moved an exchange's reads below the
barrier that follows them (a faster wave's next writes then raced them).
The exchange now pins its reads with an empty asm memory clobber; the test
checks that every barrier ending a run of LDS writes is followed by LDS reads
before the next barrier.
"""
import os
import re
import shutil
import struct
import subprocess

import pytest

from praghip import _lib

LLVM = "/opt/rocm/llvm/bin"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(LLVM, "llvm-objdump")),
                                reason="llvm-objdump of the ROCm toolchain not found")


def gfx950_code_objects(fatbin: bytes):
    """Code objects for gfx950 in a .hip_fatbin section: one clang offload
    bundle per translation unit (magic, entry count, then offset / size /
    triple per entry)."""
    out, pos = [], 0
    while True:
        i = fatbin.find(BUNDLE_MAGIC, pos)
        if i < 0:
            return out
        (count,) = struct.unpack_from("<Q", fatbin, i + 24)
        p = i + 32
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            p += 24
            triple = fatbin[p:p + tlen].decode()
            p += tlen
            if triple.endswith("gfx950"):
                out.append(fatbin[i + off:i + off + size])
        pos = i + len(BUNDLE_MAGIC)


@pytest.fixture(scope="module")
def machine_code(tmp_path_factory):
    d = tmp_path_factory.mktemp("isa")
    fat = d / "fat.bin"
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), "--dump-section", f".hip_fatbin={fat}", _lib.LIB_PATH,
                    str(d / "stripped")], check=True)
    objects = gfx950_code_objects(fat.read_bytes())
    assert len(objects) >= 7, "one code object per HIP source"
    text = []
    for k, co in enumerate(objects):
        path = d / f"co{k}"
        path.write_bytes(co)
        r = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", str(path)],
                           capture_output=True, text=True, check=True)
        text.append(r.stdout)
    shutil.rmtree(d, ignore_errors=True)
    return parse("\n".join(text))


def parse(text):
    """[(mnemonic, operands, line)], with ('FUNC', [], name) at each symbol."""
    out = []
    for line in text.splitlines():
        line = line.strip()
        if line.endswith(">:"):
            out.append(("FUNC", [], line))
            continue
        m = re.match(r"^([a-z_][a-z0-9_.]*)\s*(.*?)\s*//", line)
        if m:
            rest = m.group(2)
            out.append((m.group(1), [x.strip() for x in rest.split(",")] if rest else [], line))
    return out


def sgprs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    if m:
        return {int(m.group(1))}
    if tok == "vcc":
        return {"vcc_lo", "vcc_hi"}
    return {tok} if tok in ("vcc_lo", "vcc_hi", "m0") else set()


CARRY_OUT = re.compile(r"v_(add|sub|subrev|addc|subb|subbrev)_co_u32_e64$|v_mad_[ui]64_[ui]32$|v_div_scale_f(32|64)$")
CARRY_E32 = re.compile(r"v_(add|sub|subrev|addc|subb|subbrev)_co_u32_e32$")
MASK_IN_E64 = re.compile(r"v_cndmask_b32_e64$|v_(addc|subb|subbrev)_co_u32_e64$")
MASK_IN_E32 = re.compile(r"v_cndmask_b32_e32$|v_(addc|subb|subbrev)_co_u32_e32$")


def sgpr_defs(op, ops):
    """SGPRs (and M0, VCC) an instruction writes, and whether a VALU writes them."""
    d = set()
    if op.startswith("v_"):
        if CARRY_OUT.match(op) and len(ops) > 1:
            d |= sgprs(ops[1])
        elif (op.startswith("v_cmp") or op.startswith("v_readfirstlane") or op.startswith("v_readlane")) and ops:
            d |= sgprs(ops[0])
        if op.endswith("_e32") and (op.startswith("v_cmp") or CARRY_E32.match(op)):
            d |= {"vcc_lo", "vcc_hi"}
        return d, True
    if op.startswith("s_") and ops and not (op in ("s_nop", "s_waitcnt", "s_barrier") or op.startswith("s_cbranch")
                                            or op.startswith("s_cmp") or op.startswith("s_bitcmp")
                                            or op.startswith("s_set") or op.startswith("s_sleep")):
        d |= sgprs(ops[0])
    return d, False


def wait_states(op, ops):
    return int(ops[0], 0) + 1 if op == "s_nop" else 1


def block_start(op):
    return op == "FUNC" or op.startswith("s_cbranch") or op in ("s_branch", "s_setpc_b64")


def last_writer(code, i, regs):
    """Wait states between instruction i and the last writer of any of regs
    in the same straight-line run, and whether that writer is a VALU (None
    when no writer is found before a branch or label)."""
    ws = 0
    for j in range(i - 1, max(i - 128, -1), -1):
        op, ops, _ = code[j]
        if block_start(op):
            return None
        d, valu = sgpr_defs(op, ops)
        if d & regs:
            return ws, valu, j
        ws += wait_states(op, ops)
    return None


def test_lane_mask_reads_have_two_wait_states(machine_code):
    reads = bad = 0
    worst = []
    for i, (op, ops, line) in enumerate(machine_code):
        if MASK_IN_E64.match(op):
            regs = sgprs(ops[-1])
        elif MASK_IN_E32.match(op):
            regs = {"vcc_lo", "vcc_hi"}
        else:
            continue
        if not regs:
            continue
        reads += 1
        w = last_writer(machine_code, i, regs)
        if w and w[1] and w[0] < 2:
            bad += 1
            worst.append((machine_code[w[2]][2], line))
    # the carry-out products alone put thousands of asm carry reads here
    assert reads > 10000
    assert bad == 0, worst[:5]


def test_carry_out_products_are_in_the_library(machine_code):
    """The asm carry chain (v_mad_u64_u32 writing an SGPR carry that a
    v_addc_co_u32 reads) is present, so the check above covers it."""
    chains = 0
    for i, (op, ops, _) in enumerate(machine_code):
        if op == "v_addc_co_u32_e64" and len(ops) == 5:
            w = last_writer(machine_code, i, sgprs(ops[4]))
            if w and machine_code[w[2]][0] == "v_mad_u64_u32":
                chains += 1
    assert chains > 1000


def test_m0_write_precedes_lds_dma_by_one_wait_state(machine_code):
    dmas = bad = 0
    worst = []
    for i, (op, ops, line) in enumerate(machine_code):
        if not (op.startswith("global_load_lds") or (op.startswith("buffer_load") and " lds" in line)):
            continue
        dmas += 1
        w = last_writer(machine_code, i, {"m0"})
        if w and w[0] < 1:
            bad += 1
            worst.append((machine_code[w[2]][2], line))
    assert dmas > 0  # the share GEMM's DMA kernel
    assert bad == 0, worst[:5]


def test_exchange_reads_stay_between_barriers(machine_code):
    """Barrier, LDS writes, barrier, LDS reads, barrier: the reads stay before
    the third barrier (straight-line code; a branch ends the run)."""
    exchanges = bad = 0
    worst = []
    after_writes = False  # the last barrier ended a run of LDS writes
    last_lds = None
    func = None
    for op, ops, line in machine_code:
        if op == "FUNC":
            func, after_writes, last_lds = line, False, None
            continue
        if block_start(op):
            after_writes, last_lds = False, None
            continue
        if op.startswith("ds_"):
            kind = "r" if "read" in op else ("w" if "write" in op else "o")
            if after_writes and kind == "r":
                after_writes = False
                exchanges += 1
            last_lds = kind
        elif op == "s_barrier":
            if after_writes:
                bad += 1
                worst.append(func)
            after_writes = last_lds == "w"
            last_lds = None
    assert exchanges > 50  # the transforms' cross-wave exchanges
    assert bad == 0, worst[:5]
