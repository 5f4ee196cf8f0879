"""The launch-timeline analysis build (make timeline) on the GPU: a two-layer dependent step replayed from a graph
records one stamp row per row-group workgroup, in launch order (run in a child process: the timeline library is a
separate build of the same sources and must not replace the product library in this process)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "pingala8-llm_amd")


@pytest.mark.skipif(not os.path.exists(os.path.join(PKG, "p8x", "libp8x_timeline.so")), reason="timeline library not built")
def test_timeline_two_layers():
    r = subprocess.run([sys.executable, "-m", "p8x.timeline", "--layers", "2", "--replays", "3"], cwd=PKG,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.splitlines()
    assert lines[0].startswith("9 launches"), lines[0]   # 2 layers x 4 launches + the head
    kinds = [ln.split("|")[1].strip() for ln in lines if ln.startswith("| ") and not ln.startswith("| launch")]
    assert kinds == ["q/k/v", "o", "gate/up+swiglu", "down", "head"], kinds


@pytest.mark.skipif(not os.path.exists(os.path.join(PKG, "p8x", "libp8x_timeline.so")), reason="timeline library not built")
def test_timeline_eager_two_layers():
    r = subprocess.run([sys.executable, "-m", "p8x.timeline", "--layers", "2", "--replays", "2", "--eager"], cwd=PKG,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.splitlines()
    assert lines[0].startswith("9 launches"), lines[0]
    assert any(ln.startswith("kernel-argument fields in") for ln in lines), lines


@pytest.mark.skipif(not os.path.exists(os.path.join(PKG, "p8x", "libp8x_timeline.so")), reason="timeline library not built")
def test_timeline_gemm_phases():
    """the prompt GEMM's per-wave phases: one record per k_mm wave, phases that add up to no more than the wave"""
    r = subprocess.run([sys.executable, "-m", "p8x.timeline", "--gemm", "--tokens", "64", "--replays", "2"], cwd=PKG,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = r.stdout
    assert out.count(" waves, ") == 2, out
    for name in ("ffn_up", "ffn_down"):
        assert name in out, out
    for phase in ("prologue", "products", "barrier waits", "stores", "wave total"):
        assert phase in out, out
