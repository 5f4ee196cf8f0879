"""Where a row-group GEMV launch spends its time: per-workgroup timestamps over the dependency-respecting decode step.

Needs the timeline build (`make -C pingala8-llm_amd/csrc timeline` -> p8x/libp8x_timeline.so): thread 0 of every
k_gemv_rg workgroup records s_memrealtime (100 MHz) at its start, when the kernel-argument fields are in, when its first
loads are in (the timeline build waits for them there), after the coset table and the activation quantization, after
the workgroup barrier, after its tiles, and at its end. The chain replayed from one HIP graph is the one bench.py's
dependent_step measures: per layer {q,k,v} -> o -> {gate,up}+swiglu -> down, then the head shards, each launch reading
its producer's output (Llama-3.1-8B shapes, class-3 tensors).

    python -m p8x.timeline [--layers 32] [--eager]

prints, per kind of launch, the median and maximum over workgroups of each stamp (us from the launch's first
workgroup start), averaged over the launches of that kind, and the gap from the previous launch's last workgroup end
to this launch's first workgroup start.

    python -m p8x.timeline --step [--layers 32]

runs the same chain as one step object (k_step: one cooperative launch, a grid barrier between stages) and prints,
per kind of stage, where a stage's time goes: thread 0 of every workgroup records s_memrealtime at its stage start,
when its first virtual workgroup's input is in LDS, at the end of its virtual workgroups, when its stores are
complete, after its arrival and when it sees the release; within the first virtual workgroup also when its
activation loads are in (the timeline build waits for them there), when its tile prefetch is issued, when its
quantization is done, and, for its first round of row groups, when its tiles are done, the partial rows exchanged
and the epilogue done. Per stage: the median / maximum over workgroups of each phase, and the stage's span (the
previous stage's last release to this stage's last release).

    python -m p8x.timeline --gemm [--tokens 512]

times one p8x_mul_mat call per Llama-3.1-8B FFN shape (bf16 tokens, after warm-up calls): lane 0 of every k_mm wave
records s_memrealtime at its start, after its prologue (first x' half-block, payload and coset table in, first
barrier), summed over the half-blocks the time of its products (the x' writes of the next half-block included) and of
its barrier waits, at the end of its K loop and when its output stores have completed. Prints the median and maximum
over waves of each phase.
"""
import argparse
import ctypes
import os
import sys

import numpy as np

import p8x

STAMPS = ["start", "args in", "loads in", "table+quant", "barrier", "tiles", "end"]


BARRIER_PHASES = ["input", "tiles + epilogue", "stores done", "arrival", "release wait", "to next stage"]


def barrier_timeline(rec, info, nl):
    """per-stage phases of the grid-barrier step kernel: thread 0 of every workgroup records its stage start, its first
    virtual workgroup's input in LDS, the end of its virtual workgroups, its stores complete, its arrival done and the
    release seen"""
    nst, G = info["stages"], info["grid"]
    names = ["q/k/v", "o", "gate/up+swiglu", "down"]
    rows = {}
    prev_end = None
    for s in range(nst - 1):   # the last stage has no barrier after it
        r, nxt = rec[s], rec[s + 1]
        act = (r[:, 6] & 0xFFFF) > 0
        kind = names[s % 4] if s < 4 * nl else "head"
        ph = [r[act, 1] - r[act, 0], r[act, 2] - r[act, 1], r[:, 3] - r[:, 2], r[:, 4] - r[:, 3], r[:, 5] - r[:, 4], nxt[:, 0] - r[:, 5]]
        end = r[:, 5].max()
        span = (end - prev_end) if prev_end is not None else np.nan
        prev_end = end
        rows.setdefault(kind, []).append([np.median(x) / 100.0 for x in ph] + [x.max() / 100.0 for x in ph] + [span / 100.0, act.sum()])
    total = (rec[nst - 1, :, 0].max() - rec[0, :, 0].min()) / 100.0
    nph = len(BARRIER_PHASES)
    print(f"step kernel (barrier): {nst} stages, {G} workgroups, {total:.1f} us from the first workgroup's start to the last "
          "stage's start; us per phase")
    print("| stage | workgroups with work | " + " | ".join(BARRIER_PHASES) + " | stage span |")
    print("|---|---|" + "---|" * (nph + 1))
    for kind, v in rows.items():
        m = np.nanmean(np.array(v, np.float64), axis=0)
        cells = [f"{m[j]:.2f} / {m[nph + j]:.2f}" for j in range(nph)]
        print(f"| {kind} | {int(m[2 * nph + 1])} | " + " | ".join(cells) + f" | {m[2 * nph]:.2f} |")
    print("(each phase cell: median / maximum over the workgroups (input, tiles: those with work), averaged over the stages "
          "of that kind; stage span: from the previous stage's last release to this stage's last release)")
    # inside the first virtual workgroup: 16-bit tick counts packed into rec[6] (from the stage start) and rec[7]
    # (quantization from the stage start, the rest from the input in LDS)
    sub = {}
    for s in range(nst - 1):
        r = rec[s]
        act = (r[:, 6] & 0xFFFF) > 0
        f6, f7 = r[act, 6], r[act, 7]
        field = lambda v, sh: ((v >> sh) & 0xFFFF) / 100.0
        inp = (r[act, 1] - r[act, 0]) / 100.0
        vals = [field(f6, 16), field(f6, 32), field(f7, 0), inp, inp + field(f7, 16), inp + field(f7, 32), inp + field(f7, 48)]
        kind = names[s % 4] if s < 4 * nl else "head"
        sub.setdefault(kind, []).append([np.median(v) for v in vals])
    print()
    print("| stage | activations in | tile prefetch issued | quantized | input in LDS (all waves) | tiles done | "
          "partials exchanged | epilogue done |")
    print("|---|---|---|---|---|---|---|---|")
    for kind, v in sub.items():
        m = np.mean(np.array(v, np.float64), axis=0)
        print(f"| {kind} | " + " | ".join(f"{x:.2f}" for x in m) + " |")
    print("(us from the stage start, thread 0 of the first virtual workgroup, median over workgroups with work; the "
          "timeline build waits for the activation loads where it records them)")


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
    barrier_timeline(buf.astype(np.int64), info, nl)


def gemm_timeline(args, L):
    rng = np.random.default_rng(3)
    N = args.tokens
    for name, rows, K in (("ffn_up 4096->14336", 14336, 4096), ("ffn_down 14336->4096", 4096, 14336)):
        t = p8x.Tensor(p8x.synth_random(rows + K, rows, K, nd=8), rows, K)
        u = rng.standard_normal((N, K)).astype(np.float32).view(np.uint32).astype(np.uint64)
        xb = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        xd, yd = p8x.DeviceBuffer.from_numpy(xb), p8x.DeviceBuffer(4 * N * rows)
        st = p8x.Stream()
        for _ in range(args.replays):
            t.mul_mat_dev(xd, p8x.BF16, N, yd, stream=st)
        st.sync()
        p8x.check(L.p8x_timeline_reset(), "p8x_timeline_reset")
        t.mul_mat_dev(xd, p8x.BF16, N, yd, stream=st)
        st.sync()
        buf = np.zeros((65536, 8), np.uint64)
        n = ctypes.c_uint()
        p8x.check(L.p8x_timeline_read(buf.ctypes.data, buf.nbytes, ctypes.byref(n)), "p8x_timeline_read")
        r = buf[:min(n.value, 65536)].astype(np.int64)
        blocks = r[:, 0] & 0xFFFF
        us = lambda v: v / 100.0
        phases = [("prologue", r[:, 2] - r[:, 1]), ("products", r[:, 3]), ("barrier waits", r[:, 4]),
                  ("stores", r[:, 6] - r[:, 5]), ("wave total", r[:, 6] - r[:, 1])]
        print(f"{name}, {N} tokens: {len(r)} waves, {int(r[0, 7])} workgroups, {sorted(set(blocks.tolist()))} K blocks each; "
              f"kernel span {us(r[:, 6].max() - r[:, 1].min()):.2f} us")
        for label, v in phases:
            print(f"  {label:14s} median {us(np.median(v)):7.2f} us   max {us(v.max()):7.2f} us")
        print(f"  products per half-block (median) {us(np.median(r[:, 3] / (2 * blocks))):.3f} us")
        xd.free(); yd.free(); st.release(); t.release()


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--replays", type=int, default=20, help="untimed graph replays before the recorded one")
    ap.add_argument("--step", action="store_true", help="the one-launch step kernel instead of the graph of launches")
    ap.add_argument("--eager", action="store_true", help="the launches enqueued one by one instead of replayed from a graph")
    ap.add_argument("--dump", default=None, help="with --step: save the raw records [stage][workgroup][8] to this .npy file")
    ap.add_argument("--gemm", action="store_true", help="the prompt GEMM's k_mm waves instead of the decode step")
    ap.add_argument("--tokens", type=int, default=512, help="with --gemm: tokens per call")
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
    if args.gemm:
        gemm_timeline(args, L)
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
    graph = None if args.eager else p8x.Graph(enqueue, st)
    for _ in range(args.replays):
        enqueue(st) if args.eager else graph.launch(st)
    st.sync()
    p8x.check(L.p8x_timeline_reset(), "p8x_timeline_reset")
    enqueue(st) if args.eager else graph.launch(st)
    st.sync()
    nrec = 65536
    buf = np.zeros((nrec, 8), np.uint64)
    n = ctypes.c_uint()
    p8x.check(L.p8x_timeline_read(buf.ctypes.data, buf.nbytes, ctypes.byref(n)), "p8x_timeline_read")
    if graph:
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
    print("| launch | workgroups | " + " | ".join(STAMPS) + " | gap before |")
    print("|---|---|" + "---|" * 8)
    for kind, v in rows.items():
        m = np.nanmean(np.array(v, np.float64), axis=0)
        cells = [f"{m[j]:.2f} / {m[7 + j]:.2f}" for j in range(0, 7)]
        print(f"| {kind} | {int(m[15])} | " + " | ".join(cells) + f" | {m[14]:.2f} |")
    print("(each cell: median / maximum over the workgroups, averaged over the launches of that kind; start: when the "
          "workgroup began, the dispatch ramp of the launch)")
    # per workgroup, from its own start: how long its kernel-argument fields took (args in - start)
    own = {}
    for li, t in enumerate(launches):
        kind = names[li % 4] if li < 4 * nl else "head"
        own.setdefault(kind, []).append(np.median((t[:, 1] - t[:, 0]) / 100.0))
    print("kernel-argument fields in, from each workgroup's own start (median over workgroups, mean over launches): " +
          ", ".join(f"{k} {np.mean(v):.2f} us" for k, v in own.items()))


if __name__ == "__main__":
    main()
