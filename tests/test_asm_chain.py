"""The decode-step dataflow kernel (k_chain) keeps a ring of tile buffers in registers, loaded by inline asm and waited
for by an explicit s_waitcnt fused with each slot's use (p8x_step.hip, ChSlot). The compiler treats an asm output as
available at once: were it to read a ring register (a copy, a spill, any use) between the load and the wait, that read
would see the register before the load returned. This test compiles the unit to gfx950 assembly with the library's
flags and checks, over the compute waves' code, that every read of a ring register follows, in its basic block, the
wait that names it (the load and wait asm carry a comment with their registers). CPU only (hipcc cross-compiles)."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from test_asm_ordering import CSRC, HIPCC, hipflags

RING = 6   # kChRing in p8x_step.hip
DEST_FIRST = ("v_", "buffer_load", "global_load", "ds_read", "scratch_load", "s_")


def regs(tok):
    """register numbers of a VGPR operand token: v5 -> {5}, v[4:7] -> {4, 5, 6, 7}"""
    m = re.fullmatch(r"v(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def kernel_body(asm, name_prefix):
    lines = asm.splitlines()
    start = next(i for i, ln in enumerate(lines) if ln.startswith(name_prefix) and ":" in ln)
    end = next(i for i in range(start, len(lines)) if lines[i].strip().startswith("s_endpgm"))
    return lines[start:end + 1]


def tagged(ln, tag):
    """registers named by a `; ring <tag> ...` comment on this line"""
    m = re.search(r";\s*ring " + tag + r"\s+(.*)$", ln)
    if not m:
        return None
    out = set()
    for t in m.group(1).split():
        out |= regs(t)
    return out


def unwaited_reads(body):
    """(ring registers, reads of a ring register that is not ready), scanning the code from the first ring load to the
    end of the last block with a ring wait. A register is free until its first ring load; from then on it is ready
    only after a wait that names it, until the end of that basic block or its next load (the loop's back edge makes a
    slot's next use precede its load in the text, so readiness never carries across a label)."""
    ring, first, last = set(), None, None
    for i, ln in enumerate(body):
        r = tagged(ln, "load")
        if r is not None:
            ring |= r
            first = i if first is None else first
        if tagged(ln, "wait") is not None:
            last = i
    bad, loaded, ready = [], set(), set()
    if first is None:
        return ring, bad
    end = next((k for k in range(last + 1, len(body)) if re.match(r"^\.LBB\w*:", body[k])), len(body))
    for ln in body[first:end]:
        s = ln.split(";")[0].strip()
        if re.match(r"^\.LBB\w*:", ln):
            ready = set()
            continue
        w = tagged(ln, "wait")
        if w is not None:
            ready |= w
            continue
        r = tagged(ln, "load")
        if r is not None:
            loaded |= r
            ready -= r
            continue
        if not s or s.startswith((".", "s_")):
            continue
        ops = [t.rstrip(",") for t in s.split()[1:]]
        srcs = ops[1:] if s.startswith(DEST_FIRST) and not s.startswith(("v_cmp", "v_cmpx")) else ops
        for t in srcs:
            if regs(t) & loaded - ready:
                bad.append(s)
                break
    return ring, bad


def test_scanner_flags_an_early_read():
    """negative control: a read between a ring load and its wait is reported, one after the wait is not"""
    body = ["k:", "buffer_load_dwordx4 v[6:9], v1, s[8:11], s2 offen offset:512 nt ; ring load v[2:5] v[6:9]",
            "v_mov_b32_e32 v65, v7", "s_waitcnt vmcnt(10) ; ring wait v[2:5] v[6:9]", "v_and_b32_e32 v70, 3, v7",
            ".LBB0_1:", "v_and_b32_e32 v71, 3, v8", "s_waitcnt vmcnt(10) ; ring wait v[2:5] v[6:9]"]
    ring, bad = unwaited_reads(body)
    assert ring == set(range(2, 10))
    assert bad == ["v_mov_b32_e32 v65, v7", "v_and_b32_e32 v71, 3, v8"]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_chain_ring_registers_read_only_after_wait():
    out = tempfile.mkdtemp(prefix="p8x_asm_")
    try:
        dst = os.path.join(out, "step.s")
        cmd = [HIPCC] + hipflags() + ["--cuda-device-only", "-S", os.path.join(CSRC, "p8x_step.hip"), "-o", dst]
        r = subprocess.run(cmd, capture_output=True, timeout=900)
        assert r.returncode == 0, r.stderr.decode()[-2000:]
        body = kernel_body(open(dst).read(), "_ZN3p8x7k_chain")
        ring, bad = unwaited_reads(body)
        assert len(ring) == 8 * RING, sorted(ring)   # two 16-byte loads per slot
        assert bad == [], bad[:10]
        waits = [ln for ln in body if tagged(ln, "wait") is not None]
        assert len(waits) >= RING and all(f"vmcnt({2 * (RING - 1)})" in ln for ln in waits)
    finally:
        shutil.rmtree(out, ignore_errors=True)
