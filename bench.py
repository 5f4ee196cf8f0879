#!/usr/bin/env python3
"""Benchmark: batch-1 fused decode + GEMV over the Llama-3.1-8B-shaped Pingala-8 linear stack on one MI355X.

Workload (one step): 32 layers x (q 4096x4096, k 1024x4096, v 1024x4096, o 4096x4096, gate 14336x4096,
up 14336x4096, down 4096x14336) + lm_head 128256x4096 as 4 row-shards of 32064 rows (the format keeps
rows < 32768). Every linear runs the reference's GEMV path: activation prep (x' = FWHT(x sg / c) / 16,
8-bit per 128 columns) then the fused decode + GEMV kernel with un-permute and clamp delta. Random-valid
class-3 weights (the reference's timing arm) on synthetic N(0, 1) activations, all resident in HBM before
the timed region. value = packed weight stream bytes (M + S + D) per step x steps / wall time.

roofline: the fused GEMV kernel, algorithmic bytes = the packed stream of each launch, durations from HIP
events bracketing every GEMV launch on the stream it runs on. cpu_baseline: the reference's own CPU core
(oracle/_ref, built from its patch) running its two-phase GEMV driver on bounded samples (the stack's first 10
layers at 16 and 8 threads, x16 and q8 activations; one tensor or layer of the other configurations).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "pingala8-llm_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

import p8x  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense fp16/bf16 MFMA, MI355X
LLAMA_LAYER = [("attn_q", 4096, 4096), ("attn_k", 1024, 4096), ("attn_v", 1024, 4096), ("attn_output", 4096, 4096),
               ("ffn_gate", 14336, 4096), ("ffn_up", 14336, 4096), ("ffn_down", 4096, 14336)]
HEAD_SHARDS = [("lm_head", 32064, 4096)] * 4
QWEN3_14B_LAYER = [("attn_q", 5120, 5120), ("attn_k", 1024, 5120), ("attn_v", 1024, 5120), ("attn_output", 5120, 5120),
                   ("ffn_gate", 17408, 5120), ("ffn_up", 17408, 5120), ("ffn_down", 5120, 17408)]
QWEN3_4B_LAYER = [("attn_q", 4096, 2560), ("attn_k", 1024, 2560), ("attn_v", 1024, 2560), ("attn_output", 2560, 4096),
                  ("ffn_gate", 9728, 2560), ("ffn_up", 9728, 2560), ("ffn_down", 2560, 9728)]
CLASS_C3 = (0, 0, 0, 1, 0, 0, 0, 0)
# B4 class mix per tensor kind (logs/cs_lfull_transcode.log): attn_v class 6, ffn_down 78.1% c3 / 12.5% c4 / 9.4% c2
CLASS_B4 = {"attn_v": (0, 0, 0, 0, 0, 0, 1, 0), "ffn_down": (0, 0, 0.094, 0.781, 0.125, 0, 0, 0)}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# linears that read the same input share its rotation (one column scale c per input, one sign vector per model)
SHARED_INPUT = [("attn_q", "attn_k", "attn_v"), ("attn_output",), ("ffn_gate", "ffn_up"), ("ffn_down",)]


def build_stack(layers, mix, keep_host_layers):
    """the stack's tensors (device), their kinds, and the host slots of the first keep_host_layers layers (the CPU
    baseline's sample)"""
    tensors, kinds, host0 = [], [], []
    seed = 1
    signs = None
    groups = [[(f"blk.{l}.{k}", r, K) for (k, r, K) in LLAMA_LAYER if k in grp] for l in range(layers) for grp in SHARED_INPUT]
    groups.append([(f"output.{i}", r, K) for i, (_, r, K) in enumerate(HEAD_SHARDS)])
    for grp in groups:
        slots = []
        for name, rows, K in grp:
            kind = name.split(".")[-1] if name.startswith("blk") else "lm_head"
            cp = CLASS_B4.get(kind, CLASS_C3) if mix == "b4" else CLASS_C3
            slots.append(p8x.synth_random(seed, rows, K, class_p=cp, nd=1))
            seed += 1
        if signs is None:
            o = p8x.side_offsets(slots[0].size, grp[0][1], grp[0][2], 1)
            signs = slots[0][o["SG"]:o["SG"] + 256].copy()
        p8x.share_input(slots, [(r, K) for _, r, K in grp], signs_from=signs)
        for slot, (name, rows, K) in zip(slots, grp):
            tensors.append(p8x.Tensor(slot, rows, K))
            kinds.append(name.split(".")[-1] if name.startswith("blk") else "lm_head")
            if name.startswith("blk.") and int(name.split(".")[1]) < keep_host_layers:
                host0.append((slot, rows, K))
    return tensors, kinds, host0


def stream_bytes_of(slot, rows, K):
    """packed weight stream (payload D + scales S + tile words M) of a host slot"""
    nt = (rows // 32) * (K // 256)
    kb = int(np.frombuffer(slot[-32:].tobytes(), np.uint32)[2])
    return kb - ((2064 + 68 * nt + 15) & ~15) + 68 * nt


def host_l3():
    """the host's last-level cache as lscpu reports it (e.g. '256 MiB (8 instances)')"""
    import subprocess
    try:
        for ln in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if ln.strip().startswith("L3"):
                return ln.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return "unknown"


def cpu_baseline(host_stack, seconds):
    """The reference's own CPU core (oracle/_ref: vr-native-cpu-core.h compiled from its patch, driven by a pthread
    restatement of its two-phase vrc_tg GEMV) on bounded samples: the Llama-3.1-8B stack's first layers (larger than
    the host's last-level cache), at 16 threads (this box's CPU share) and 8 (the reference paper's setting), in the
    reference's default x16 activation mode and in q8; then one tensor or layer of the other configurations.
    Returns the headline object (stack sample, x16, 16 threads) with every run listed under "runs"."""
    import oracle as O
    variant = O.best_ref_variant()
    if not O.ref_available(variant):
        return None
    core = O.RefCore(variant)
    rng = np.random.default_rng(7)

    def run(name, slots, planes, nth, secs):
        pool = O.RefPool(core, nth)
        refs = [core.open(sl, r, K) for (sl, r, K) in slots]
        xs = [rng.standard_normal(K).astype(np.float32) for (_, _, K) in slots]
        ys = [np.zeros(r, np.float32) for (_, r, _) in slots]
        nbytes = sum(stream_bytes_of(sl, r, K) for (sl, r, K) in slots)
        pool.gemv_seq(refs, xs, ys, planes=planes)   # warm
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < secs:
            pool.gemv_seq(refs, xs, ys, planes=planes)
            n += 1
        dt = time.perf_counter() - t0
        pool.close()
        for r in refs:
            r.close()
        res = {"sample": name, "mode": "x16" if planes == 2 else "q8", "threads": nth, "MB": round(nbytes / 1e6, 1),
               "passes": n, "ms_per_pass": round(dt / n * 1e3, 3), "GB/s": round(nbytes * n / dt / 1e9, 3)}
        log("cpu baseline:", json.dumps(res))
        return res

    ncpu = os.cpu_count() or 1
    threads = [t for t in (16, 8) if t <= ncpu] or [ncpu]
    nl = len(host_stack) // 7
    stack_name = f"llama3.1-8b layers 0-{nl - 1} ({7 * nl} linears)"
    runs = [run(stack_name, host_stack, planes, nth, seconds / 4) for nth in threads for planes in (2, 1)]
    cfgs = [("4096 x 4096 (one tensor)", [(4096, 4096)]),
            ("qwen3-4b one layer", [(r, K) for (_, r, K) in QWEN3_4B_LAYER]),
            ("qwen3-14b one layer", [(r, K) for (_, r, K) in QWEN3_14B_LAYER])]
    for name, shapes in cfgs:
        slots = [(p8x.synth_random(7000 + i, r, K, nd=1), r, K) for i, (r, K) in enumerate(shapes)]
        runs.append(run(name, slots, 2, threads[0], seconds / 8))
    head = runs[0]
    return {"value": head["GB/s"], "unit": "GB/s", "cores": head["threads"], "kind": "reference",
            "sample": f"{stack_name}, {head['MB']} MB packed (host L3: {host_l3()}), {head['passes']} passes, "
                      f"x16 activations (the reference's default CPU mode), {head['threads']} threads; "
                      f"reference core vr-native-cpu-core.h built {core.isa}",
            "runs": runs}


def timed_steps(run, stream, warmup, steps):
    """ms per call of run(), calls back to back after warmup, HIP events around the whole run"""
    for _ in range(warmup):
        run()
    stream.sync()
    e0, e1 = p8x.Event(), p8x.Event()
    e0.record(stream)
    for _ in range(steps):
        run()
    e1.record(stream)
    stream.sync()
    return e0.elapsed_ms(e1) / steps


def measure_qwen14b_columns(stream, steps, col_list=(1, 2, 4, 8), kernel=p8x.GEMV_KERNEL_AUTO):
    """Qwen3-14B (40 layers, 280 linears, all class 3) streamed by one grouped launch per step at 1/2/4/8
    activation columns sharing the weights: GB/s of the weight stream and columns (tokens) per second. kernel: the
    fused launch's kernel for more than one column (the plan's choice by default; p8x_gemv_batch_create_ex)"""
    plan = [(r, K) for _ in range(40) for (_, r, K) in QWEN3_14B_LAYER]
    tensors = [p8x.Tensor(p8x.synth_random(1000 + i, r, K, nd=1), r, K) for i, (r, K) in enumerate(plan)]
    stream_bytes = sum(t.stream_bytes for t in tensors)
    rng = np.random.default_rng(5)
    out = {"workload": "qwen3-14b linear stack: 40 x (q,k,v,o,gate,up,down), class 3, one grouped launch per step",
           "stream_bytes_per_step": int(stream_bytes)}
    for n in col_list:
        xs = {K: p8x.DeviceBuffer.from_numpy(rng.standard_normal(n * K).astype(np.float32)) for K in sorted({t.K for t in tensors})}
        ys = [p8x.DeviceBuffer(4 * n * t.rows) for t in tensors]
        batch = p8x.GemvBatch(tensors, [xs[t.K] for t in tensors], ys, ncols=n, kernel=kernel if n > 1 else p8x.GEMV_KERNEL_AUTO)
        ms = timed_steps(lambda: batch.run(stream), stream, 40, steps)
        out[f"batch_{n}"] = {"ms_per_step": round(ms, 4), "GB/s": round(stream_bytes / (ms * 1e-3) / 1e9, 1),
                             "tokens_per_s": round(n / (ms * 1e-3), 1)}
        log(f"qwen3-14b batch {n}: {ms * 1e3:.1f} us/step, {stream_bytes / (ms * 1e-3) / 1e9:.0f} GB/s")
        batch.release()
        for b in list(xs.values()) + ys:
            b.free()
    for t in tensors:
        t.release()
    return out


def measure_quantized_4096(stream, steps, copies=128):
    """one 4096 x 4096 W quantized by the host encoder (N(0, 0.02^2) with 0.1% of entries x10, seeded c16 in
    [0.5, 2) and Hadamard signs, clamp delta above fp16(1.001 max|W|)); single p8x_mul_mat_vec calls back to back
    over 128 distinct device copies (555 MB, so the MALL does not hold the weights)"""
    rng = np.random.default_rng(1)
    W = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    W[rng.random(W.shape) < 0.001] *= 10
    c16 = rng.uniform(0.5, 2.0, 4096).astype(np.float16).view(np.uint16)
    slot = p8x.quantize_tensor(W, c16=c16, sign_seed=3)
    tensors = [p8x.Tensor(slot, 4096, 4096) for _ in range(copies)]
    x = p8x.DeviceBuffer.from_numpy(rng.standard_normal(4096).astype(np.float32))
    y = p8x.DeviceBuffer(4 * 4096)

    def rnd(act):
        def f():
            for t in tensors:
                t.mul_mat_vec_dev(x, y, act=act, stream=stream)
        return f

    ms = timed_steps(rnd(p8x.ACT_Q8_128), stream, 5, steps) / copies
    ms1 = timed_steps(rnd(p8x.ACT_Q8_1), stream, 5, steps) / copies
    b = tensors[0].stream_bytes
    for t in tensors:
        t.release()
    log(f"quantized 4096x4096: {ms * 1e3:.2f} us per call (q8 per 128 columns), {ms1 * 1e3:.2f} us (block_q8_1)")
    return {"workload": f"one 4096 x 4096 class-3 tensor from the host encoder, {copies} device copies in rotation, "
                        "single p8x_mul_mat_vec calls back to back", "stream_bytes": int(b),
            "us_per_call": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
            "q8_1": {"us_per_call": round(ms1 * 1e3, 2), "GB/s": round(b / (ms1 * 1e-3) / 1e9, 1),
                     "activations": "ggml block_q8_1 (per 32 columns), quantized in the call"}}


def measure_qwen4b_layer(stream, steps, copies=20):
    """Qwen3-4B one layer (7 linears, 26 MB), batch 1, rotating over 20 distinct copies (> 512 MB, so the MALL
    does not hold the weights): one grouped launch per layer, and one p8x_mul_mat_vec call per linear"""
    tensors = [[p8x.Tensor(p8x.synth_random(5000 + 7 * c + i, r, K, nd=1), r, K) for i, (_, r, K) in enumerate(QWEN3_4B_LAYER)]
               for c in range(copies)]
    layer_bytes = sum(t.stream_bytes for t in tensors[0])
    rng = np.random.default_rng(6)
    xs = {K: p8x.DeviceBuffer.from_numpy(rng.standard_normal(K).astype(np.float32)) for K in (2560, 4096, 9728)}
    ys = [[p8x.DeviceBuffer(4 * t.rows) for t in layer] for layer in tensors]
    batches = [p8x.GemvBatch(layer, [xs[t.K] for t in layer], y) for layer, y in zip(tensors, ys)]

    def grouped():
        for b in batches:
            b.run(stream)

    def per_linear():
        for layer, y in zip(tensors, ys):
            for t, yb in zip(layer, y):
                t.mul_mat_vec_dev(xs[t.K], yb, stream=stream)

    g_ms = timed_steps(grouped, stream, 10, steps) / copies
    l_ms = timed_steps(per_linear, stream, 10, steps) / copies
    log(f"qwen3-4b layer: grouped {g_ms * 1e3:.1f} us, per-linear {l_ms * 1e3:.1f} us per layer")
    for b in batches:
        b.release()
    for layer, y in zip(tensors, ys):
        for t in layer:
            t.release()
        for b in y:
            b.free()
    for b in xs.values():
        b.free()
    return {"workload": f"qwen3-4b one layer (q,k,v,o,gate,up,down), batch 1, {copies} distinct copies in rotation",
            "stream_bytes_per_layer": int(layer_bytes),
            "grouped_launch": {"us_per_layer": round(g_ms * 1e3, 2), "GB/s": round(layer_bytes / (g_ms * 1e-3) / 1e9, 1)},
            "per_linear_launches": {"us_per_layer": round(l_ms * 1e3, 2), "GB/s": round(layer_bytes / (l_ms * 1e-3) / 1e9, 1)}}


def measure_per_linear(tensors, kinds, xs, ybufs, stream, step_bytes, pl_steps, graph_replay=True):
    """the drop-in pattern: one p8x_mul_mat_vec call (a single launch) per linear, as a MUL_MAT hook would issue"""
    def step_linear_on(s):
        for i, t in enumerate(tensors):
            t.mul_mat_vec_dev(xs[t.K], ybufs[i], stream=s)

    def step_linear(events=None):
        for i, t in enumerate(tensors):
            if events is not None:
                events[2 * i].record(stream)
            t.mul_mat_vec_dev(xs[t.K], ybufs[i], stream=stream)
            if events is not None:
                events[2 * i + 1].record(stream)

    for _ in range(5):   # past the GPU's settling phase (tens of milliseconds of load)
        step_linear()
    stream.sync()
    e0, e1 = p8x.Event(), p8x.Event()
    e0.record(stream)
    for _ in range(pl_steps):
        step_linear()
    e1.record(stream)
    stream.sync()
    pl_ms = e0.elapsed_ms(e1) / pl_steps
    evs = [[p8x.Event() for _ in range(2 * len(tensors))] for _ in range(pl_steps)]
    for s_ in range(pl_steps):
        step_linear(evs[s_])
    stream.sync()
    kern_ms = np.zeros(len(tensors))
    for s_ in range(pl_steps):
        for i in range(len(tensors)):
            kern_ms[i] += evs[s_][2 * i].elapsed_ms(evs[s_][2 * i + 1])
    kern_ms /= pl_steps
    bytes_per = np.array([t.stream_bytes for t in tensors], np.float64)
    per_kind = {}
    for k in dict.fromkeys(kinds):
        idx = [i for i, kk in enumerate(kinds) if kk == k]
        per_kind[k] = {"GB/s": round(bytes_per[idx].sum() / (kern_ms[idx].sum() * 1e-3) / 1e9, 1),
                       "us_per_call": round(float(kern_ms[idx].mean() * 1e3), 2),
                       "MB_per_call": round(float(bytes_per[idx].mean() / 1e6), 3)}
    log("per-linear p8x_mul_mat_vec calls, per kind:", json.dumps(per_kind))
    per_linear = {"GB/s": round(step_bytes / (pl_ms * 1e-3) / 1e9, 1), "ms_per_step": round(pl_ms, 4),
                  "launches_per_step": len(tensors), "per_kind": per_kind}
    if graph_replay:
        # the same step captured once in a HIP graph and replayed (how a graph-capturing host issues it)
        graph = p8x.Graph(lambda s: step_linear_on(s), stream)
        g_ms = timed_steps(lambda: graph.launch(stream), stream, 5, pl_steps)
        graph.release()
        log(f"per-linear calls replayed from a HIP graph: {g_ms * 1e3:.0f} us/step")
        per_linear["graph_replay"] = {"GB/s": round(step_bytes / (g_ms * 1e-3) / 1e9, 1), "ms_per_step": round(g_ms, 4)}
    return per_linear


def measure_dependent_step(tensors, kinds, stream, steps, graph_replay=True):
    """A batch-1 decode step that respects the data dependencies of the model: per layer, q/k/v as one launch on the
    layer input (p8x_mul_mat_vec_multi), o on q's output, the gated FFN input silu(gate x) * (up x) as one launch on
    o's output (p8x_mul_mat_vec_glu), down on that (the next layer's input); then the head shards as one launch on
    the last down's output. Each product's activations are its producer's outputs, so nothing overlaps across
    launches; captured once in a HIP graph and replayed. (Values shrink from layer to layer without the model's
    norms; the products' work does not depend on them.)"""
    nl = sum(1 for k in kinds if k == "attn_q")
    layer = [tensors[7 * l:7 * l + 7] for l in range(nl)]
    head = tensors[7 * nl:]
    rng = np.random.default_rng(9)
    x0 = p8x.DeviceBuffer.from_numpy(rng.standard_normal(layer[0][0].K).astype(np.float32))
    bufs, plan = [x0], []
    cur = x0
    for q, k, v, o, gate, up, down in layer:
        yq, yk, yv = p8x.DeviceBuffer(4 * q.rows), p8x.DeviceBuffer(4 * k.rows), p8x.DeviceBuffer(4 * v.rows)
        yo, yg, yd = p8x.DeviceBuffer(4 * o.rows), p8x.DeviceBuffer(4 * gate.rows), p8x.DeviceBuffer(4 * down.rows)
        bufs += [yq, yk, yv, yo, yg, yd]
        plan.append(((q, k, v), cur, (yq, yk, yv), (o, yq, yo), (gate, up, yo, yg), (down, yg, yd)))
        cur = yd
    yh = [p8x.DeviceBuffer(4 * t.rows) for t in head]
    bufs += yh

    def enqueue(s):
        for qkv, xin, yqkv, (o, xo, yo), (gate, up, xg, yg), (down, xd, yd) in plan:
            p8x.mul_mat_vec_multi_dev(list(qkv), xin, list(yqkv), stream=s)
            o.mul_mat_vec_dev(xo, yo, stream=s)
            p8x.mul_mat_vec_glu_dev(gate, up, xg, yg, stream=s)
            down.mul_mat_vec_dev(xd, yd, stream=s)
        p8x.mul_mat_vec_multi_dev(head, cur, yh, stream=s)

    eager_ms = timed_steps(lambda: enqueue(stream), stream, 3, steps)
    g_ms = None
    if graph_replay:
        graph = p8x.Graph(enqueue, stream)
        g_ms = timed_steps(lambda: graph.launch(stream), stream, 3, steps)
        graph.release()
    # the same chain as one cooperative launch (p8x_step): stages separated by grid barriers
    chain = []
    for qkv, xin, yqkv, (o, xo, yo), (gate, up, xg, yg), (down, xd, yd) in plan:
        chain += [(list(qkv), xin, list(yqkv)), ([o], xo, [yo]), ([gate, up], xg, None, yg), ([down], xd, [yd])]
    chain.append((head, cur, yh))
    step = p8x.Step(chain)
    s_ms = timed_steps(lambda: step.run(stream), stream, 3, steps)
    step.check()
    sinfo = step.info()
    step.release()
    step_bytes = sum(t.stream_bytes for t in tensors)
    launches = 4 * nl + 1
    gtxt = f"graph {g_ms * 1e3:.0f} us" if g_ms is not None else "graph not replayed"
    log(f"dependent step: eager {eager_ms * 1e3:.0f} us, {gtxt} ({launches} launches), "
        f"one launch {s_ms * 1e3:.0f} us ({sinfo['grid']} workgroups, {sinfo['stages']} stages)")
    for b in bufs:
        b.free()
    return {"workload": f"{nl} layers: q/k/v in one launch -> o -> silu(gate) * up in one launch -> down, then the head "
                        "shards in one launch; each launch reads its producer's output", "launches": launches,
            "step_kernel": {"ms_per_step": round(s_ms, 4), "GB/s": round(step_bytes / (s_ms * 1e-3) / 1e9, 1),
                            "frac_of_peak": round(step_bytes / (s_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                            "stages": sinfo["stages"], "workgroups": sinfo["grid"]},
            "graph_replay": {"ms_per_step": round(g_ms, 4), "GB/s": round(step_bytes / (g_ms * 1e-3) / 1e9, 1)} if g_ms else None,
            "eager": {"ms_per_step": round(eager_ms, 4), "GB/s": round(step_bytes / (eager_ms * 1e-3) / 1e9, 1)}}


def measure_gemm(steps, N=512):
    """prompt GEMM on the Llama-3.1-8B FFN shapes: N bf16 tokens ~ N(0, 1), whole p8x_mul_mat calls timed; class-3
    tensors, and ffn_down with the released models' class mix (the every-class kernel)"""
    out = {}
    rng = np.random.default_rng(3)
    for name, rows, K, cp in (("ffn_up 4096->14336", 14336, 4096, CLASS_C3), ("ffn_down 14336->4096", 4096, 14336, CLASS_C3),
                              ("ffn_down 14336->4096, b4 class mix", 4096, 14336, CLASS_B4["ffn_down"])):
        t = p8x.Tensor(p8x.synth_random(rows + K, rows, K, class_p=cp, nd=8), rows, K)
        u = rng.standard_normal((N, K)).astype(np.float32).view(np.uint32).astype(np.uint64)
        xb = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        xd = p8x.DeviceBuffer.from_numpy(xb)
        yd = p8x.DeviceBuffer(4 * N * rows)
        stream = p8x.Stream()
        for _ in range(20):
            t.mul_mat_dev(xd, p8x.BF16, N, yd, stream=stream)
        stream.sync()
        ev = [(p8x.Event(), p8x.Event()) for _ in range(steps)]
        for a, b in ev:
            a.record(stream)
            t.mul_mat_dev(xd, p8x.BF16, N, yd, stream=stream)
            b.record(stream)
        stream.sync()
        ms = float(np.median([a.elapsed_ms(b) for a, b in ev]))
        tflops = 2.0 * rows * K * N / (ms * 1e-3) / 1e12
        out[name] = {"us_per_call": round(ms * 1e3, 1), "TFLOP/s": round(tflops, 1),
                     "frac_of_fp16_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "tokens": N}
        t.release()
    log("prompt GEMM:", json.dumps(out))
    return out


def measured_traffic(step_bytes, layers, mix):
    """HBM bytes per GEMV launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this workload
    (counter KiB scaled by what the same counters read for a device copy of known size); None if absent or
    taken on another workload."""
    path = os.path.join(ROOT, "profiles", "k_gemv_wave_llama8b_stream.json")
    try:
        with open(path) as f:
            prof = json.load(f)
    except (OSError, ValueError):
        return None, None
    if prof.get("stream_bytes_per_step") != step_bytes or prof.get("layers") != layers or prof.get("class_mix") != mix:
        return None, None
    return int(prof["traffic_bytes_per_launch"]), "profiles/k_gemv_wave_llama8b_stream.json"


def measure_dequant(steps, copies=20):
    """dequantize-to-fp16 (original rows, Hadamard applied) of one Llama FFN weight, 14336 x 4096: a write-bound
    kernel; bytes = packed stream read + fp16 output written. The calls rotate over 20 device copies of the tensor
    (303 MB, more than the 256 MB MALL) and two output buffers, so every call reads its packed weights from HBM."""
    rows, K = 14336, 4096
    slot = p8x.synth_random(99, rows, K, nd=8)
    ts = [p8x.Tensor(slot, rows, K) for _ in range(copies)]
    outs = [p8x.DeviceBuffer(2 * rows * K) for _ in range(2)]
    stream = p8x.Stream()
    for i in range(40):
        ts[i % copies].dequantize_dev(p8x.F16, outs[i % 2], stream=stream)
    stream.sync()
    ev = [(p8x.Event(), p8x.Event()) for _ in range(steps)]
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        ts[i % copies].dequantize_dev(p8x.F16, outs[i % 2], stream=stream)
        b.record(stream)
    stream.sync()
    ms = float(np.median([a.elapsed_ms(b) for a, b in ev]))
    nbytes = ts[0].stream_bytes + 2 * rows * K
    res = {"tensor": f"{rows} x {K} -> fp16, {copies} copies in rotation", "us_per_call": round(ms * 1e3, 1),
           "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "frac_of_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "bytes": int(nbytes)}
    for t in ts:
        t.release()
    for o in outs:
        o.free()
    stream.release()
    log("dequantize to fp16:", json.dumps(res))
    return res


def measure_grouped(tensors, xs, ybufs, stream, steps, warmup):
    """One grouped launch (activation prep + fused decode-GEMV + finishing) over every linear per step. A change of
    load sets off a power-management transient: the first few steps run fast, the next few dozen up to 60% slower,
    then the step time settles (measured per step on MI355X). The grouped launch therefore runs until its step time is
    stable (settle steps, reported), then the warmup steps, then K timed steps back to back (the step time), then the
    same K steps again with each fused decode + GEMV launch carrying a pair of HIP events that the runtime records at
    that kernel's own start and end (hipExtLaunchKernel): the kernel's duration, the interval rocprofv3's kernel trace
    reports. The events put about 11 us of queue work around the kernel, so the step time is timed without them.
    Returns the batch object (still live) and (settle steps, ms per step, ms per step with events, kernel ms, wall s)."""
    batch = p8x.GemvBatch(tensors, [xs[t.K] for t in tensors], ybufs)
    settle_steps, prev = 0, None
    while settle_steps < 400:
        a, b = p8x.Event(), p8x.Event()
        a.record(stream)
        for _ in range(10):
            batch.run(stream)
        b.record(stream)
        settle_steps += 10
        cur = a.elapsed_ms(b)
        if settle_steps >= 60 and prev is not None and abs(cur - prev) <= 0.02 * prev:
            break
        prev = cur
    for _ in range(warmup):
        batch.run(stream)
    stream.sync()
    e0, e1 = p8x.Event(), p8x.Event()
    e0.record(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        batch.run(stream)
    e1.record(stream)
    stream.sync()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_ms(e1) / steps
    ev = [(p8x.Event(), p8x.Event()) for _ in range(steps)]
    e2, e3 = p8x.Event(), p8x.Event()
    e2.record(stream)
    for s_ in range(steps):
        for stage in range(batch.stages):
            batch.run_stage(stage, stream, events=ev[s_] if stage == 1 else None)
    e3.record(stream)
    stream.sync()
    ms_per_step_events = e2.elapsed_ms(e3) / steps
    gemv_ms = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    return batch, settle_steps, ms_per_step, ms_per_step_events, gemv_ms, wall


def measure_b4_mix(args, stream):
    """The same grouped launch over the stack with the released models' class mix (attn_v class 6; ffn_down 78.1%
    class 3, 12.5% class 4, 9.4% class 2; the rest class 3): the kernels for several class sets."""
    tensors, kinds, _ = build_stack(args.layers, "b4", 0)
    step_bytes = sum(t.stream_bytes for t in tensors)
    rng = np.random.default_rng(0)
    xs = {K: p8x.DeviceBuffer.from_numpy(rng.standard_normal(K).astype(np.float32)) for K in sorted({t.K for t in tensors})}
    ybufs = [p8x.DeviceBuffer(4 * t.rows) for t in tensors]
    batch, settle, ms, ms_ev, gemv_ms, _ = measure_grouped(tensors, xs, ybufs, stream, args.steps, args.warmup)
    batch.release()
    for t in tensors:
        t.release()
    for b in list(xs.values()) + ybufs:
        b.free()
    gbs = step_bytes / (ms * 1e-3) / 1e9
    kgbs = step_bytes / (gemv_ms * 1e-3) / 1e9
    log(f"b4 mix: {ms * 1e3:.1f} us/step ({gbs:.0f} GB/s), GEMV kernel {gemv_ms * 1e3:.1f} us -> {kgbs:.0f} GB/s")
    return {"workload": "the headline stack with the released models' class mix (attn_v class 6; ffn_down 78.1% c3, "
                        "12.5% c4, 9.4% c2); one grouped launch per step", "stream_bytes_per_step": int(step_bytes),
            "settle_steps": settle, "ms_per_step": round(ms, 4), "GB/s": round(gbs, 1),
            "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "kernel_us": round(gemv_ms * 1e3, 1),
            "kernel_GB/s": round(kgbs, 1), "kernel_frac": round(kgbs / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--mix", choices=("c3", "b4"), default="c3")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--cpu-layers", type=int, default=10, help="Llama layers in the CPU baseline's sample (10: 563 MB)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-per-linear", action="store_true", help="skip the per-linear launch measurement")
    ap.add_argument("--no-dependent", action="store_true", help="skip the dependency-respecting decode step")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prompt GEMM and dequantize measurements")
    ap.add_argument("--no-qwen", action="store_true", help="skip the Qwen3-14B multi-column and Qwen3-4B layer lines")
    ap.add_argument("--no-mix", action="store_true", help="skip the b4 class-mix line")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP graph replays of the per-linear and dependent steps (the one-launch step still runs)")
    ap.add_argument("--gemv-kernel", choices=("auto", "dot4", "mfma"), default="auto",
                    help="the Qwen3-14B column runs' fused kernel from two columns on (default: the batch plan's choice)")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="also run one device-to-device copy of MIB MiB (the HBM-counter calibration kernel under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the GEMV path shards by rows (each GPU streams rows/G of every linear, then one all-gather of y)",
              file=sys.stderr)
        sys.exit(2)
    if p8x.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)

    t_build = time.perf_counter()
    tensors, kinds, host0 = build_stack(args.layers, args.mix, 0 if args.no_cpu else args.cpu_layers)
    log(f"built {len(tensors)} tensors in {time.perf_counter() - t_build:.1f} s")
    step_bytes = sum(t.stream_bytes for t in tensors)
    rng = np.random.default_rng(0)
    xs = {K: p8x.DeviceBuffer.from_numpy(rng.standard_normal(K).astype(np.float32)) for K in sorted({t.K for t in tensors})}
    ybufs = [p8x.DeviceBuffer(4 * t.rows) for t in tensors]
    stream = p8x.Stream()

    # ---- per-linear launches (the drop-in path: one p8x_mul_mat_vec per graph node), the dependency-respecting
    # step, the prompt GEMM and dequantize; reported beside the headline and timed before it
    per_linear = measure_per_linear(tensors, kinds, xs, ybufs, stream, step_bytes, max(3, args.steps // 3),
                                    not args.no_graph) if not args.no_per_linear else None
    dependent = measure_dependent_step(tensors, kinds, stream, max(5, args.steps // 4), not args.no_graph) \
        if not args.no_dependent else None
    gemm = measure_gemm(max(5, args.steps // 2)) if not args.no_gemm else None
    deq = measure_dequant(max(5, args.steps // 2)) if not args.no_gemm else None

    # ---- headline: one grouped launch over every linear per step (measure_grouped)
    batch, settle_steps, ms_per_step, ms_per_step_events, gemv_ms, wall = measure_grouped(tensors, xs, ybufs, stream, args.steps,
                                                                                          args.warmup)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = step_bytes / (gemv_ms * 1e-3) / 1e9
    log(f"stream: settled after {settle_steps} steps; {ms_per_step * 1e3:.1f} us/step, GEMV kernel {gemv_ms * 1e3:.1f} us "
        f"-> {achieved:.0f} GB/s (steps with kernel events {ms_per_step_events * 1e3:.1f} us)")
    b4 = measure_b4_mix(args, stream) if args.mix == "c3" and not args.no_mix else None

    device_bw = None
    if args.copy_calib:
        # also the practical ceilings of a write-only and a read + write stream on this card: the runtime's own fill
        # and device-to-device copy of the same size, median of 5 (events around each synchronous call)
        n = args.copy_calib << 20
        src, dst = p8x.DeviceBuffer(n), p8x.DeviceBuffer(n)
        src.fill(1)
        p8x.synchronize()
        dst.copy_from(src)
        p8x.synchronize()
        e0, e1 = p8x.Event(), p8x.Event()

        def timed(fn):
            ts = []
            for _ in range(5):
                e0.record(None)
                fn()
                e1.record(None)
                p8x.synchronize()
                ts.append(e0.elapsed_ms(e1))
            return float(np.median(ts))
        fill_ms, copy_ms = timed(lambda: src.fill(7)), timed(lambda: dst.copy_from(src))
        device_bw = {"bytes": n, "fill_TB/s": round(n / (fill_ms * 1e-3) / 1e12, 3),
                     "copy_TB/s (read + write)": round(2 * n / (copy_ms * 1e-3) / 1e12, 3)}
        log("device fill / copy:", json.dumps(device_bw))
        e0.release(); e1.release()
        src.free(); dst.free()
        log(f"copy calibration: {n} bytes device to device")

    qwen14b = qwen4b = quant4096 = None
    if not args.no_qwen:
        batch.release()
        for t in tensors:
            t.release()
        kern = {"auto": p8x.GEMV_KERNEL_AUTO, "dot4": p8x.GEMV_KERNEL_DOT4, "mfma": p8x.GEMV_KERNEL_MFMA}[args.gemv_kernel]
        qwen14b = measure_qwen14b_columns(stream, max(10, args.steps // 4), kernel=kern)
        qwen4b = measure_qwen4b_layer(stream, max(10, args.steps // 4))
        quant4096 = measure_quantized_4096(stream, max(10, args.steps // 10))
    cpu = cpu_baseline(host0, args.cpu_seconds) if not args.no_cpu and host0 else None
    traffic, traffic_src = measured_traffic(int(step_bytes), args.layers, args.mix)
    out = {
        "metric": "bs=1 dequant-GEMV HBM GB/s (% of peak), Llama-3.1-8B linear shapes",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic (random-valid class-3 codes, N(0,1) activations)",
        "config": {"workload": "llama3.1-8b linear stack, batch 1: 32 x (q,k,v,o,gate,up,down) + lm_head as 4 x 32064 rows, "
                               "streamed by one grouped launch per step",
                   "layers": args.layers, "class_mix": args.mix, "linears": len(tensors), "launches_per_step": batch.stages,
                   "settle_steps": settle_steps,
                   "stream_bytes_per_step": int(step_bytes), "frac_of_peak": round(value / HBM_PEAK_GBS, 4),
                   "activations": "q8 per 128 columns (k_vr_qx_real semantics)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": "k_gemv_wave<class 3> (fused decode + GEMV, grouped launch)", "launches": args.steps,
                     "bytes_per_launch": int(step_bytes),
                     "timing": "kernel-attached HIP events on K further steps right after the K timed steps "
                               f"({ms_per_step_events:.4f} ms per step with the events)"},
        "cpu_baseline": cpu,
        "per_linear_launches": per_linear,
        "dependent_step": dependent,
        "prompt_gemm": gemm,
        "dequantize_f16": deq,
        "qwen3_14b_columns": qwen14b,
        "qwen3_4b_layer": qwen4b,
        "quantized_4096": quant4096,
        "b4_mix": b4,
        "device_bandwidth": device_bw,
        "host_wall_s": round(wall, 3),
    }
    # every handle released here, while the runtime (and a profiler's tool attached to it) is still up; nothing is
    # left for interpreter shutdown
    batch.release()
    for t in tensors:
        t.release()
    for b in list(xs.values()) + ybufs:
        b.free()
    stream.release()
    p8x.synchronize()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
