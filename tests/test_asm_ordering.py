"""The K-chunk fix-up publishes partial rows to another workgroup (possibly on another XCD): agent-scope stores,
then an arrival counter RMW. The stores must be complete (s_waitcnt vmcnt(0)) before the RMW is issued, or the
last arrival can read a stale partial. This test compiles the units that hold fix-up kernels to gfx950 assembly
(with the library's own flags) and checks that no atomic add follows an sc1 store without a vmcnt(0) wait between.
CPU only (hipcc cross-compiles)."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "pingala8-llm_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
# the single-call row-group kernel (one and two columns, K split), the task kernel (K-chunk fix-up) and the
# one-launch step (K-chunk fix-up, stage barrier)
UNITS = ["p8x_gemv_w.hip", "p8x_gemv_rgm.hip", "p8x_gemv_q81.hip", "p8x_step.hip"]


def hipflags():
    """HIPFLAGS from the library Makefile (continuation lines joined), with the architecture filled in"""
    txt = open(os.path.join(CSRC, "Makefile")).read().replace("\\\n", " ")
    m = re.search(r"^HIPFLAGS\s*=\s*(.*)$", txt, re.M)
    return m.group(1).replace("$(ARCH)", "gfx950").split()


def unordered_publications(asm_lines):
    """(atomic adds, atomic adds issued while an sc1 store may still be outstanding), scanning in program order"""
    pending, n, bad = False, 0, 0
    for ln in asm_lines:
        s = ln.strip()
        if re.match(r"(global|buffer)_store_\w+ .*\bsc1\b", s):
            pending = True
        elif s.startswith("s_waitcnt") and "vmcnt(0)" in s:
            pending = False
        elif re.match(r"(global|buffer)_atomic_add", s):
            n += 1
            bad += pending
        elif s.startswith(".Lfunc_end"):
            pending = False
    return n, bad


def test_scanner_flags_a_store_then_atomic():
    """negative control: the scanner catches the sequence the fix removed"""
    bad_seq = ["global_store_dword v[10:11], v20, off sc1", "global_atomic_add v2, v3, v48, s[36:37] sc0"]
    good_seq = [bad_seq[0], "s_waitcnt vmcnt(0)", bad_seq[1]]
    assert unordered_publications(bad_seq) == (1, 1)
    assert unordered_publications(good_seq) == (1, 0)


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_fixup_stores_complete_before_arrival():
    out = tempfile.mkdtemp(prefix="p8x_asm_")
    try:
        procs = {}
        for u in UNITS:
            cmd = [HIPCC] + hipflags() + ["--cuda-device-only", "-S", os.path.join(CSRC, u), "-o", os.path.join(out, u + ".s")]
            procs[u] = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)
        total = 0
        for u, p in procs.items():
            _, err = p.communicate(timeout=600)
            assert p.returncode == 0, err.decode()[-2000:]
            n, bad = unordered_publications(open(os.path.join(out, u + ".s")).read().splitlines())
            assert bad == 0, f"{u}: {bad} of {n} atomic adds follow an sc1 store without s_waitcnt vmcnt(0)"
            total += n
        assert total > 0   # the fix-up kernels were compiled
    finally:
        shutil.rmtree(out, ignore_errors=True)
