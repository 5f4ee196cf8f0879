"""Where a row-group GEMV launch spends its time: per-workgroup timestamps over the dependency-respecting decode step.

Needs the timeline build (`make -C pingala8-llm_amd/csrc timeline` -> p8x/libp8x_timeline.so): thread 0 of every
k_gemv_rg workgroup records s_memrealtime (100 MHz) at its start, when the kernel-argument fields are in, when its first
loads are in (the timeline build waits for them there), after the coset table and the activation quantization, after
the workgroup barrier, after its tiles, and at its end. The chain replayed from one HIP graph is the one bench.py's
dependent_step measures: per layer {q,k,v} -> o -> {gate,up}+swiglu -> down, then the head shards, each launch reading
its producer's output (Llama-3.1-8B shapes, class-3 tensors).

    python -m p8x.timeline [--layers 32]

prints, per kind of launch, the median and maximum over workgroups of each stamp (us from the launch's first
workgroup start), averaged over the launches of that kind, and the gap from the previous launch's last workgroup end
to this launch's first workgroup start.

    python -m p8x.timeline --step [--layers 32]

runs the same chain as one step object (the dataflow kernel for these class-3 tensors) and prints, per kind of stage,
where a stage's time goes: sync wave 0 of every workgroup records s_memrealtime at the start of its input phase, when
its input blocks are polled and quantized into LDS, after the workgroup barrier that starts the compute phase, after
the one that ends it, and after its epilogue (partial rows summed, outputs published); compute wave 0 records when its
tiles of the stage are done. Per stage: the median / maximum over the workgroups with work of each phase, and the
stage's span (last epilogue end of the previous stage to last epilogue end of this one).
"""
import argparse
import ctypes
import os
import sys

import numpy as np

import p8x

STAMPS = ["start", "args in", "loads in", "table+quant", "barrier", "tiles", "end"]


STEP_PHASES = ["input", "to compute", "compute", "to epilogue", "epilogue"]


def step_timeline(args, L):
    """per-stage records of the step kernel (see the module docstring)"""
    root = os.path.dirname(os.path.dirname(p8x.HERE))
    sys.path.insert(0, root)
    import bench
    tensors, kinds, _ = bench.build_stack(args.layers, "c3", 0)
    nl = args.layers
    layer = [tensors[7 * l:7 * l + 7] for l in range(nl)]
    head = tensors[7 * nl:]
    x0 = p8x.DeviceBuffer.from_numpy(np.random.default_rng(9).standard_normal(layer[0][0].K).astype(np.float32))
    stages, cur = [], x0
    for q, k, v, o, gate, up, down in layer:
        yq, yk, yv = (p8x.DeviceBuffer(4 * t.rows) for t in (q, k, v))
        yo, yg, yd = p8x.DeviceBuffer(4 * o.rows), p8x.DeviceBuffer(4 * gate.rows), p8x.DeviceBuffer(4 * down.rows)
        stages += [([q, k, v], cur, [yq, yk, yv]), ([o], yq, [yo]), ([gate, up], yo, None, yg), ([down], yg, [yd])]
        cur = yd
    stages.append((head, cur, [p8x.DeviceBuffer(4 * t.rows) for t in head]))
    step = p8x.Step(stages)
    info = step.info()
    st = p8x.Stream()
    for _ in range(args.replays):
        step.run(st)
    st.sync()
    step.run(st)
    st.sync()
    step.check()
    G, nst = info["grid"], info["stages"]
    buf = np.zeros((nst, G, 8), np.uint64)
    n = ctypes.c_uint()
    p8x.check(L.p8x_timeline_read(buf.ctypes.data, buf.nbytes, ctypes.byref(n)), "p8x_timeline_read")
    step.release()
    if args.dump:
        np.save(args.dump, buf)
    rec = buf.astype(np.int64)
    t0 = rec[:, :, 0].min()
    names = ["q/k/v", "o", "gate/up+swiglu", "down"]
    rows = {}
    prev_end = rec[0, :, 0].min()
    for s in range(nst):
        r = rec[s]
        act = r[:, 6] > 0
        kind = names[s % 4] if s < 4 * nl else "head"
        ph = [r[act, 1] - r[act, 0], r[act, 2] - r[act, 1], r[act, 5] - r[act, 2], r[act, 3] - r[act, 5], r[act, 4] - r[act, 3]]
        end = r[act, 4].max()
        span = end - prev_end
        prev_end = end
        rows.setdefault(kind, []).append([np.median(x) / 100.0 for x in ph] + [x.max() / 100.0 for x in ph] + [span / 100.0, act.sum()])
    total = (rec[:, :, 4].max() - t0) / 100.0
    print(f"step kernel ({info['kernel']}): {nst} stages, {G} workgroups, {total:.1f} us from the first workgroup's start "
          "to the last epilogue end; us per phase")
    print("| stage | workgroups with work | " + " | ".join(STEP_PHASES) + " | stage span |")
    print("|---|---|" + "---|" * 6)
    for kind, v in rows.items():
        m = np.mean(np.array(v, np.float64), axis=0)
        cells = [f"{m[j]:.2f} / {m[5 + j]:.2f}" for j in range(5)]
        print(f"| {kind} | {int(m[11])} | " + " | ".join(cells) + f" | {m[10]:.2f} |")
    print("(each phase cell: median / maximum over the workgroups with work, averaged over the stages of that kind; "
          "stage span: from the previous stage's last epilogue end to this stage's last epilogue end)")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--replays", type=int, default=20, help="untimed graph replays before the recorded one")
    ap.add_argument("--step", action="store_true", help="the one-launch step kernel instead of the graph of launches")
    ap.add_argument("--dump", default=None, help="with --step: save the raw records [stage][workgroup][8] to this .npy file")
    args = ap.parse_args()
    p8x.LIB_PATH = os.path.join(p8x.HERE, "libp8x_timeline.so")
    L = p8x.lib()
    if not hasattr(L, "p8x_timeline_read"):
        raise p8x.P8xError(f"{p8x.LIB_PATH} is not the timeline build")
    L.p8x_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint)]
    p8x.check(L.p8x_timeline_reset(), "p8x_timeline_reset")   # allocates the record buffer before any capture
    if args.step:
        step_timeline(args, L)
        return
    root = os.path.dirname(os.path.dirname(p8x.HERE))
    sys.path.insert(0, root)
    import bench
    tensors, kinds, _ = bench.build_stack(args.layers, "c3", 0)
    nl = args.layers
    layer = [tensors[7 * l:7 * l + 7] for l in range(nl)]
    head = tensors[7 * nl:]
    x0 = p8x.DeviceBuffer.from_numpy(np.random.default_rng(9).standard_normal(layer[0][0].K).astype(np.float32))
    plan, cur = [], x0
    for q, k, v, o, gate, up, down in layer:
        yq, yk, yv = (p8x.DeviceBuffer(4 * t.rows) for t in (q, k, v))
        yo, yg, yd = p8x.DeviceBuffer(4 * o.rows), p8x.DeviceBuffer(4 * gate.rows), p8x.DeviceBuffer(4 * down.rows)
        plan.append(((q, k, v), cur, (yq, yk, yv), (o, yq, yo), (gate, up, yo, yg), (down, yg, yd)))
        cur = yd
    yh = [p8x.DeviceBuffer(4 * t.rows) for t in head]

    def enqueue(s):
        for qkv, xin, yqkv, (o, xo, yo), (gate, up, xg, yg), (down, xd, yd) in plan:
            p8x.mul_mat_vec_multi_dev(list(qkv), xin, list(yqkv), stream=s)
            o.mul_mat_vec_dev(xo, yo, stream=s)
            p8x.mul_mat_vec_glu_dev(gate, up, xg, yg, stream=s)
            down.mul_mat_vec_dev(xd, yd, stream=s)
        p8x.mul_mat_vec_multi_dev(head, cur, yh, stream=s)

    st = p8x.Stream()
    graph = p8x.Graph(enqueue, st)
    for _ in range(args.replays):
        graph.launch(st)
    st.sync()
    p8x.check(L.p8x_timeline_reset(), "p8x_timeline_reset")
    graph.launch(st)
    st.sync()
    nrec = 65536
    buf = np.zeros((nrec, 8), np.uint64)
    n = ctypes.c_uint()
    p8x.check(L.p8x_timeline_read(buf.ctypes.data, buf.nbytes, ctypes.byref(n)), "p8x_timeline_read")
    graph.release()
    rec = buf[:min(n.value, nrec)].astype(np.int64)
    # records in arrival order; launches on one stream do not overlap, so consecutive runs of `grid` records are
    # one launch each
    grid = rec[:, 0] & 0xFFFFFFFF
    launches, i = [], 0
    while i < len(rec):
        launches.append(rec[i:i + grid[i], 1:8])
        i += int(grid[i])
    names = ["q/k/v", "o", "gate/up+swiglu", "down"]
    rows = {}
    prev_end = None
    for li, t in enumerate(launches):
        kind = names[li % 4] if li < 4 * nl else "head"
        base = t[:, 0].min()
        med = [(np.median(t[:, j]) - base) / 100.0 for j in range(7)]
        mx = [(t[:, j].max() - base) / 100.0 for j in range(7)]
        gap = (base - prev_end) / 100.0 if prev_end is not None else np.nan
        prev_end = t[:, 6].max()
        rows.setdefault(kind, []).append(med + mx + [gap, len(t)])
    print(f"{len(launches)} launches, {len(rec)} workgroup records; us from the launch's first workgroup start")
    print("| launch | workgroups | " + " | ".join(STAMPS[1:]) + " | gap before |")
    print("|---|---|" + "---|" * 7)
    for kind, v in rows.items():
        m = np.nanmean(np.array(v, np.float64), axis=0)
        cells = [f"{m[j]:.2f} / {m[7 + j]:.2f}" for j in range(1, 7)]
        print(f"| {kind} | {int(m[15])} | " + " | ".join(cells) + f" | {m[14]:.2f} |")
    print("(each cell: median / maximum over the workgroups, averaged over the launches of that kind)")


if __name__ == "__main__":
    main()
