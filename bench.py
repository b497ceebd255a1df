"""Benchmark: Qwen2.5-1.5B-architecture bf16 decode on one MI355X (the headline workload).

A step is one decode step of the full 28-layer model (random-init bf16 weights
N(0, 0.02), tied embeddings) at batch 1 over static KV caches of length 2048,
run through ``DAGExecutor`` + the HIP backend, with the greedy next token computed
on the device and fed back as the next step's ``input_ids`` (no host sync inside
the timed region). Timed steps walk cache positions 1984..1984+K-1 (a 64-step
window ending at the cache length for K=64); every run (warmup, timed, parity)
starts from the same first token at position 1984, and each step writes its
cache row before reading it, so every run sees the caches a cold run would.

Printed JSON line: tok/s (whole job), ms/step, a ``roofline`` object for the
dominant kernel (algorithmic bytes per launch over its average launch time,
measured with HIP events on the launch stream), the step-level fraction of HBM
peak, the rate with host-side per-step inputs, and a ``cpu_baseline`` measured on
this host's cores with the CPU fallback (DAGExecutor over an all-CPU plan, ATen
bf16) over the same 64-step greedy loop, with a teacher-forced top-1 comparison
of the two paths.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pytorch-apple_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "Qwen2.5-1.5B-arch bf16 decode tok/s @ctx2048; achieved HBM GB/s vs peak"
PUBLISHED_TOKS = 30.0   # reference CUDA path, RTX 3090 Ti, cache position 2048 (docs/benchmarks.md:98)


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def step_bytes(cfg, valid_len: int) -> int:
    """Algorithmic HBM bytes of one decode step at KV valid length ``valid_len``."""
    h, i, L, kvh, d, v = cfg.hidden, cfg.intermediate, cfg.layers, cfg.kv_heads, cfg.head_dim, cfg.vocab
    per_layer = 2 * (h * cfg.heads * d + 2 * h * kvh * d + (cfg.heads * d + 2 * kvh * d) + cfg.heads * d * h
                     + 3 * h * i + 2 * h)
    weights = L * per_layer + 2 * h + 2 * v * h + 2 * h      # layers, final norm, lm_head (tied, read once), 1 emb row
    kv_read = L * 2 * kvh * d * 2 * valid_len
    kv_write = L * 2 * kvh * d * 2
    logits = 2 * v
    return weights + kv_read + kv_write + logits


def gemv_launch_bytes(step) -> int:
    """Algorithmic HBM bytes of one fused GEMV launch: weights (+bias), activations in, results out."""
    p = step.params
    nw = p.get("weights", 1)
    resid = p.get("epilogue") == "resid"
    return 2 * (nw * p["N"] * p["K"] + p["M"] * p["K"] + p["M"] * (p["N"] if nw == 1 else p["N"])
                + (p["M"] * p["N"] if resid else 0) + (nw * p["N"] if p.get("has_bias") else 0))


def time_kernel_subset(ex, indices, repeats, stream) -> float:
    """Average ms per launch of ``ex``'s launch records ``indices``, timed with HIP events on ``stream``."""
    from hip_runtime import _shim

    lib = _shim.lib()
    sub = (_shim.LaunchRec * len(indices))(*[ex._recs[i] for i in indices])
    e0, e1 = C.c_void_p(), C.c_void_p()
    _shim.check(lib.hs_event_create(C.byref(e0)))
    _shim.check(lib.hs_event_create(C.byref(e1)))
    _shim.check(lib.hs_replay(sub, len(indices), stream))     # warm
    _shim.check(lib.hs_event_record(e0, stream))
    for _ in range(repeats):
        _shim.check(lib.hs_replay(sub, len(indices), stream))
    _shim.check(lib.hs_event_record(e1, stream))
    _shim.check(lib.hs_event_sync(e1))
    ms = C.c_float()
    _shim.check(lib.hs_event_elapsed_ms(e0, e1, C.byref(ms)))
    lib.hs_event_destroy(e0)
    lib.hs_event_destroy(e1)
    return ms.value / (repeats * len(indices))


def time_graph_reps(ex, reps: int, stream) -> float:
    """Device ms per step: ``reps`` copies of the step's launch list captured into one HIP
    graph and launched once between two HIP events, so no host work sits between steps."""
    from hip_runtime import _shim

    lib = _shim.lib()
    n = len(ex._recs)
    recs = (_shim.LaunchRec * (n * reps))(*[ex._recs[i] for _ in range(reps) for i in range(n)])
    cs, g = C.c_void_p(), C.c_void_p()
    _shim.check(lib.hs_stream_create(C.byref(cs)))
    _shim.check(lib.hs_graph_capture(recs, n * reps, cs, C.byref(g)))
    e0, e1 = C.c_void_p(), C.c_void_p()
    _shim.check(lib.hs_event_create(C.byref(e0)))
    _shim.check(lib.hs_event_create(C.byref(e1)))
    _shim.check(lib.hs_graph_launch(g, stream))      # warm
    _shim.check(lib.hs_event_record(e0, stream))
    _shim.check(lib.hs_graph_launch(g, stream))
    _shim.check(lib.hs_event_record(e1, stream))
    _shim.check(lib.hs_event_sync(e1))
    ms = C.c_float()
    _shim.check(lib.hs_event_elapsed_ms(e0, e1, C.byref(ms)))
    for e in (e0, e1):
        lib.hs_event_destroy(e)
    lib.hs_graph_destroy(g)
    lib.hs_stream_destroy(cs)
    return ms.value / reps


def time_in_step(ex, indices, replays, stream) -> float:
    """Average ms of the launches ``indices`` inside full replays of the step's launch list:
    every launch of the step runs in order, and HIP events on ``stream`` bracket each selected
    launch, so the kernel is timed with the caches and neighbours it has in a real step."""
    from hip_runtime import _shim

    lib = _shim.lib()
    recs = ex._recs
    sel = set(indices)
    n = len(recs)
    evs = [C.c_void_p() for _ in range(2 * len(indices))]
    for e in evs:
        _shim.check(lib.hs_event_create(C.byref(e)))
    total = 0.0
    for _ in range(replays):
        j, k = 0, 0
        while j < n:
            if j in sel:
                _shim.check(lib.hs_event_record(evs[2 * k], stream))
                one = (_shim.LaunchRec * 1)(recs[j])
                _shim.check(lib.hs_replay(one, 1, stream))
                _shim.check(lib.hs_event_record(evs[2 * k + 1], stream))
                j, k = j + 1, k + 1
                continue
            e = j
            while e < n and e not in sel:
                e += 1
            chunk = (_shim.LaunchRec * (e - j))(*recs[j:e])
            _shim.check(lib.hs_replay(chunk, e - j, stream))
            j = e
        _shim.check(lib.hs_event_sync(evs[-1]))
        ms = C.c_float()
        for k in range(len(indices)):
            _shim.check(lib.hs_event_elapsed_ms(evs[2 * k], evs[2 * k + 1], C.byref(ms)))
            total += ms.value
    for e in evs:
        lib.hs_event_destroy(e)
    return total / (replays * len(indices))


def _cpu_decode_loop(ex, ir, x, n_steps, times=None, tokens=None, logits=None, feed=None):
    """Greedy decode steps on a CPU-plan DAGExecutor from the state ``x`` (host arrays) at its
    ``cache_position``. ``feed``: the input token of each step after the first (teacher forcing);
    without it each step reads the previous step's argmax. Every step writes its cache row before
    reading it, so re-running positions from the same first token reproduces a cold run exactly."""
    import numpy as np
    import torch

    from irgen.workloads import decode_mask, to_host

    kv_in = [g["name"] for g in ir["graph_inputs"][4:]]
    kv_out = [o["name"] for o in ir["graph_outputs"][1:-1]]
    start = int(np.asarray(x["cache_position"]).reshape(-1)[0])
    S = x["attention_mask"].shape[-1]
    lname = ir["graph_outputs"][0]["name"]
    mdt = torch.float32 if np.asarray(x["attention_mask"]).dtype == np.float32 else torch.bfloat16
    ins = dict(x)
    for s in range(n_steps):
        pos = start + s
        ins["attention_mask"] = to_host(decode_mask(S, pos).to(mdt))
        ins["position_ids"] = np.array([[pos]], np.int64)
        ins["cache_position"] = np.array([pos], np.int64)
        if feed is not None and s > 0:
            ins["input_ids"] = np.array([[feed[s - 1]]], np.int64)
        t0 = time.perf_counter()
        out = ex.execute(ins)
        if times is not None:
            times.append(time.perf_counter() - t0)
        ins["input_ids"] = out["next_token"]
        if tokens is not None:
            tokens.append(int(np.asarray(out["next_token"]).reshape(-1)[0]))
        if logits is not None:
            lg = np.asarray(out[lname])
            logits.append(torch.from_numpy(lg.view(np.int16)).view(torch.bfloat16).float().reshape(-1).numpy()
                          if lg.dtype == np.uint16 else lg.astype(np.float32).reshape(-1))
        for i, o in zip(kv_in, kv_out):
            ins[i] = out[o]


def cpu_baseline(ir, weights_dev, inputs_dev, cfg, steps: int, warmup: int = 3):
    """CPU fallback (all-CPU plan through DAGExecutor, ATen bf16): ``warmup`` untimed steps, then
    ``steps`` timed greedy decode steps from the same starting state. Returns the baseline record,
    the greedy tokens and the logits (float32) of the timed steps."""
    import torch

    from irgen.workloads import to_host
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    w = {k: v.detach().cpu() for k, v in weights_dev.items()}
    x = {k: to_host(v.detach().cpu()) for k, v in inputs_dev.items()}
    ex = DAGExecutor(partition(ir, lambda *_: False), None)
    ex.load_weights(w)
    start = int(x["cache_position"][0])
    _cpu_decode_loop(ex, ir, x, warmup)
    times, tokens, logits = [], [], []
    _cpu_decode_loop(ex, ir, x, steps, times, tokens, logits)
    med = statistics.median(times)
    total = sum(times)
    rec = {"value": round(steps / total, 4), "unit": "tok/s", "cores": n, "kind": "port",
           "sample": f"the same greedy loop: {steps} decode steps of the full 28-layer model at positions "
                     f"{start}..{start + steps - 1} after {warmup} untimed warmup steps, DAGExecutor with an "
                     f"all-CPU plan (ATen bf16, {n} threads); {total:.1f} s total, median step "
                     f"{med * 1e3:.1f} ms"}
    return rec, tokens, logits


def fp32_teacher_forced(cfg, weights_dev, inputs_dev, feed, steps: int):
    """The same decode graph evaluated in float32 on the CPU (plain ATen fp32: weights, caches and
    mask upcast from the bf16 values), teacher-forced with ``feed``. Returns the logits of each
    step: the reference point both bf16 paths are graded against."""
    import dataclasses

    import torch

    from irgen.qwen import build_decode_ir
    from irgen.workloads import to_host
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    S = inputs_dev["attention_mask"].shape[-1]
    ir32 = build_decode_ir(S, dataclasses.replace(cfg, dtype="float32"), argmax=True)
    w = {k: (v.detach().cpu().float() if v.dtype == torch.bfloat16 else v.detach().cpu())
         for k, v in weights_dev.items()}
    x = {k: to_host(v.detach().cpu().float() if v.dtype == torch.bfloat16 else v.detach().cpu())
         for k, v in inputs_dev.items()}
    ex = DAGExecutor(partition(ir32, lambda *_: False), None)
    ex.load_weights(w)
    logits: list = []
    _cpu_decode_loop(ex, ir32, x, steps, logits=logits, feed=feed)
    return logits


def bf16_ulp(v: float) -> float:
    """Spacing of bf16 values (8 significant bits) at magnitude ``v``."""
    import math

    return 2.0 ** (math.floor(math.log2(max(abs(v), 1e-30))) - 7)


def parity_vs_fp32(hip_rec, cpu_tokens, cpu_logits, f32_logits, tie_ulps: int = 4) -> dict:
    """Grades both bf16 paths against the float32 evaluation of the same teacher-forced steps.

    Per step: each path's largest logit difference from fp32 (relative to fp32's largest
    |logit|) and whether its top-1 token is fp32's. A step is a near tie when fp32's own two
    best logits are within ``tie_ulps`` bf16 ulps of the largest logit: a fixed window set by
    the storage precision, not by either path's error. Raw agreement counts are reported
    beside the near-tie counts."""
    import numpy as np

    n = len(f32_logits)
    rec = {"steps": n, "tie_window": f"fp32 top-2 gap <= {tie_ulps} bf16 ulps of the largest logit"}
    ties = []
    for t in f32_logits:
        top2 = np.partition(t, -2)[-2:]
        ties.append(float(top2[1] - top2[0]) <= tie_ulps * bf16_ulp(float(np.abs(t).max())))
    for name, toks, lgs in (("hip", [g for g, _ in hip_rec], [gl for _, gl in hip_rec]),
                            ("cpu", cpu_tokens, cpu_logits)):
        agree = [int(tk == int(np.argmax(t))) for tk, t in zip(toks, f32_logits)]
        err = [float(np.abs(lg - t).max() / np.abs(t).max()) for lg, t in zip(lgs, f32_logits)]
        rec[f"{name}_vs_fp32"] = {
            "top1_agree": sum(agree),
            "misses": n - sum(agree),
            "misses_at_near_ties": sum(1 for a, tie in zip(agree, ties) if not a and tie),
            "logits_max_rel_err": round(max(err), 4),
            "logits_mean_rel_err": round(float(np.mean(err)), 4)}
    rec["near_tie_steps"] = sum(ties)
    return rec


def run_copy_probe(device_index: int, stream, mib: int = 512, repeats: int = 3) -> float:
    """Launch the library's plain copy kernel (``k_copy16``, the contiguous form of the copy
    lowering) over ``mib`` MiB of bf16, ``repeats`` times.

    Its known traffic (``mib`` MiB read, ``mib`` MiB written per launch) calibrates the
    FETCH_SIZE / WRITE_SIZE counters that give the ``traffic`` figure. Returns the average
    launch time in ms."""
    import torch

    from hip_runtime import _shim
    from hip_runtime.hip_executor import module_cache
    from hip_runtime.kernels import STRUCTS

    n = mib * (1 << 20) // 2
    src = torch.ones(n, dtype=torch.bfloat16, device=f"cuda:{device_index}")
    dst = torch.empty_like(src)
    a = STRUCTS["CopyArgs"]()
    a.dst, a.src, a.n, a.ndim = dst.data_ptr(), src.data_ptr(), n * 2 // 16, 1   # n: 16-byte chunks
    a.sdtype = a.ddtype = 2
    mods = module_cache(device_index)
    mods.ensure_builtin("basic")
    fn = mods.function("basic", "k_copy16")
    lib = _shim.lib()
    e0, e1 = C.c_void_p(), C.c_void_p()
    _shim.check(lib.hs_event_create(C.byref(e0)))
    _shim.check(lib.hs_event_create(C.byref(e1)))
    _shim.check(lib.hs_event_record(e0, stream))
    for _ in range(repeats):
        _shim.check(lib.hs_launch(fn, 8192, 1, 1, 256, 1, 1, 0, stream, C.byref(a), C.sizeof(a)), "k_copy16")
    _shim.check(lib.hs_event_record(e1, stream))
    _shim.check(lib.hs_event_sync(e1))
    ms = C.c_float()
    _shim.check(lib.hs_event_elapsed_ms(e0, e1, C.byref(ms)))
    lib.hs_event_destroy(e0)
    lib.hs_event_destroy(e1)
    if not torch.equal(dst, src):
        raise RuntimeError("copy probe produced wrong data")
    return ms.value / repeats


TRAFFIC_GLOB = os.path.join(ROOT, "profiles", "*_hbm_traffic.md")


STAMP_NAMES = ("A weights in", "A x in", "A q/k/v published", "B q/k/v in", "B partial published",
               "C partials in", "C attention row published", "D o_proj rows landed", "D attention row in",
               "D x1 published", "E register rows issued", "E x1 in", "E h published", "F weights issued",
               "F h in", "F x published")


def decode_stamps(hexec, ex, state, L: int, steps: int = 6) -> dict:
    """Per-part timeline of the persistent decode step from its progress stamps (decode.hip
    DEC_STAMP: thread 0 of each workgroup records the 100 MHz real-time counter at fixed points of
    each part). Runs ``steps`` steps without a graph (the stamp buffer is an argument the captured
    graphs do not carry) and reads the last. Per stamp: the median over the workgroups that record
    it, in µs after the layer's first workgroup has its input row, averaged over layers 2..L-3
    (and the minimum, median and maximum over those workgroups, averaged the same way)."""
    import numpy as np
    import torch

    (st,) = hexec.program.steps
    nwg, H, nsplit = int(st.grid[0]), int(st.args["H"]), int(st.args["nsplit"])
    NB = (int(st.args["KVH"]) if st.params.get("kv_major") else H) * nsplit
    tr = torch.zeros(nwg * (L * 16 + 8), dtype=torch.int64, device=hexec.device)
    s = hexec._structs[0]
    s.trace = tr.data_ptr()
    use_graph, hexec.use_graph = hexec.use_graph, False
    try:
        for _ in range(steps):
            ex.execute(state)
        torch.cuda.synchronize()
    finally:
        s.trace = None
        hexec.use_graph = use_graph
    t = tr.cpu().numpy().reshape(nwg, L * 16 + 8).astype(np.float64) * 0.01   # 10 ns ticks -> µs
    t -= t[:, L * 16 + 7].min()
    b = np.arange(nwg)
    att, comb = b < NB, (b >= NB) & (b < NB + H)
    if st.params.get("slot_combine"):   # the attention workgroups run the combine
        comb = att
    who = {3: att, 4: att, 5: comb, 6: comb, 7: ~att, 8: ~att, 9: ~att}
    layers = range(2, L - 2)
    med, spread = {}, {}
    for k, name in enumerate(STAMP_NAMES):
        vals = []
        for l in layers:
            v = t[:, l * 16 + k] - t[:, l * 16 + 1].min()
            vals.append(np.percentile(v[who.get(k, np.ones(nwg, bool))], [0, 50, 100]))
        m = np.mean(vals, axis=0)
        med[name] = round(float(m[1]), 2)
        spread[name] = [round(float(x), 2) for x in m]
    period = float(np.mean([t[:, (l + 1) * 16 + 1].min() - t[:, l * 16 + 1].min() for l in layers]))
    g_in, g_done = t[:, L * 16 + 1], t[:, L * 16 + 2]
    return {"layers_averaged": f"2..{L - 3}", "per_part_median_us": med,
            "per_part_min_median_max_us": spread, "layer_period_us": round(period, 2),
            "first_layer_input_us": round(float(t[:, 1].min()), 2),
            "lm_head_us": {"median": round(float(np.median(g_done - g_in.min())), 2),
                           "last": round(float(g_done.max() - g_in.min()), 2)},
            "kernel_us": round(float(t[0, L * 16 + 3]), 2)}


def measured_traffic(kernel: str, workload: str | None = None) -> int | None:
    """HBM bytes per launch of ``kernel`` from the committed FETCH_SIZE / WRITE_SIZE summaries
    (lines ``traffic_bytes_per_launch <kernel> <bytes>``, or ``... <bytes> <workload>`` for a
    figure measured on one workload's shapes), or None when none has an entry."""
    import glob

    for path in sorted(glob.glob(TRAFFIC_GLOB)):
        for line in open(path):
            parts = line.strip().strip("`").split()
            if (len(parts) in (3, 4) and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel
                    and (parts[3] if len(parts) == 4 else None) == workload):
                return int(parts[2])
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default: decode 32, since the GPU's clocks ramp over its first "
                         "~10 ms of work and with 8 the first timed steps ran ~2%% slower; prefill 2, mlp / "
                         "attention 20, generate 5, resnet50 3)")
    ap.add_argument("--max-cache-len", type=int, default=2048)
    ap.add_argument("--start-pos", type=int, default=1984)
    ap.add_argument("--cpu-steps", type=int, default=64)
    ap.add_argument("--parity-seed2-steps", type=int, default=32,
                    help="decode: steps of the fp32-graded parity pass on a second seed (0: none)")
    ap.add_argument("--cpu-warmup", type=int, default=3)
    ap.add_argument("--kernel-repeats", type=int, default=10,
                    help="replays per kernel family / per step in the per-kernel timing")
    ap.add_argument("--copy-probe-mib", type=int, default=512,
                    help="size of the k_copy calibration launches run after timing (0: skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--stamps", action="store_true",
                    help="decode: add the persistent step's per-part timeline (its progress stamps) to the line")
    ap.add_argument("--no-fp32-parity", action="store_true",
                    help="skip grading the parity pass against a float32 evaluation of the same steps")
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--workload", choices=("decode", "prefill", "resnet50", "generate", "mlp", "attention"),
                    default="decode",
                    help="decode: the headline (cfg3); prefill: 512-token prefill (cfg4); resnet50: batch-32 "
                         "ResNet-50 inference (cfg5); the last two report MFMA utilisation; generate: HF "
                         "Qwen2 exported to IR, padded prefill then greedy decode (TTFT and tok/s); mlp: the "
                         "RMSNorm + gated MLP + residual subgraph (cfg1) at --tokens; attention: one decode "
                         "attention block over a 1025-entry cache (cfg2); the last two report HBM GB/s")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--prefill-tokens", type=int, default=512)
    ap.add_argument("--tokens", type=int, default=1, help="cfg1 rows (1, 16 or 128)")
    args = ap.parse_args()
    if args.workload == "prefill" and args.gpus == 1:
        return main_prefill(args)
    if args.workload == "resnet50" and args.gpus == 1:
        return main_resnet(args)
    if args.workload == "generate" and args.gpus == 1:
        return main_generate(args)
    if args.workload in ("mlp", "attention") and args.gpus == 1:
        return main_block(args)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 (sharding across "
                                   "GPUs is a design note, not implemented)"}))
        return 2

    import torch

    from hip_compiler import compile_subgraph, is_hip_op_supported
    from hip_runtime import HIPBackend
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, decode_mask, make_weights, to_host
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    if args.warmup is None:
        args.warmup = 32
    cfg = QwenConfig(layers=args.layers)
    S, start = args.max_cache_len, args.start_pos
    if start + max(args.steps, args.warmup) > S:
        raise SystemExit("start-pos + steps exceeds the cache length")
    dev = torch.device("cuda", 0)
    log("building IR and compiling")
    t0 = time.time()
    ir = build_decode_ir(S, cfg, argmax=True)
    backend = HIPBackend(0)
    ex = DAGExecutor(partition(ir, is_hip_op_supported), backend, compile_fn=compile_subgraph)
    compile_s = time.time() - t0
    log(f"compiled in {compile_s:.2f}s; generating weights on the device")
    weights = make_weights(ir, cfg, device="cuda")
    x0 = decode_inputs(S, start, cfg, device="cuda")
    ex.load_weights(weights)
    (program,) = ex.npu_programs.values()
    (hexec,) = ex._npu_executors.values()
    log(f"program: {len(program.steps)} launches, arena {program.arena_bytes / 1e6:.1f} MB")

    kv_in = [g["name"] for g in ir["graph_inputs"][4:]]
    kv_out = [o["name"] for o in ir["graph_outputs"][1:-1]]
    # the positions the runs below visit (not the whole cache: at 32k positions that would be 2 GB
    # of masks)
    window = range(start, min(S, start + max(args.steps, args.warmup, args.cpu_steps) + 1))
    masks = [decode_mask(S, p).to(dev) for p in window]
    pos_ids = [torch.tensor([[p]], dtype=torch.int64, device=dev) for p in window]
    cpos = [torch.tensor([p], dtype=torch.int64, device=dev) for p in window]
    from hip_runtime import HIPBuffer

    state = {k: backend.allocate_buffer(v) for k, v in x0.items()}
    first_token = state["input_ids"]
    mask_t, pos_t, cpos_t = (state[k].native_handle for k in ("attention_mask", "position_ids", "cache_position"))
    advance = backend.decode_advance(state["attention_mask"], state["position_ids"], state["cache_position"])
    # the persistent step moves its own position inputs after each step (no second launch per step)
    folded = hexec.fold_advance(advance)

    host_steps = None

    lname = ir["graph_outputs"][0]["name"]

    def reset():
        # the first step's inputs in place; every later step's come from the advance folded
        # into the step (or k_decode_advance, one launch on the same stream after each step),
        # so the executor's pointers stay fixed and its captured graph is relaunched as-is
        mask_t.copy_(masks[0])
        pos_t.copy_(pos_ids[0])
        cpos_t.copy_(cpos[0])

    def run(n_steps, host=False, feed=None, record=None, fresh=True):
        # every run starts from the same first token at position `start`; each step writes its
        # cache row before reading it, so every run repeats the cold run exactly.
        # feed: per-step host input_ids (teacher forcing); record: list that gets (token, logits);
        # fresh: reset the position inputs first (the timed run has them reset before its clock)
        st = dict(state)
        st["input_ids"] = first_token
        if not host and fresh:
            reset()
        for s in range(n_steps):
            if feed is not None and s > 0:
                st["input_ids"] = feed[s]
            if host:
                # host-side per-step inputs (numpy), uploaded by DAGExecutor every step
                st.update(host_steps[s])
            out = ex.execute(st)
            if not host and not folded and s < n_steps - 1:   # the next step's inputs
                advance()
            st["input_ids"] = out["next_token"]
            if record is not None:
                record.append((int(out["next_token"].native_handle.reshape(-1)[0].item()),
                               out[lname].native_handle.float().reshape(-1).cpu().numpy()))
            for i, o in zip(kv_in, kv_out):
                st[i] = out[o]
        return st

    log(f"warmup {args.warmup} steps")
    run(args.warmup)
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    reset()   # (the run's input set-up, outside the timed steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(args.steps, fresh=False)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    advance.check()   # no step moved past the cache end
    hexec.check()     # no persistent step timed out waiting for data (its tokens would be invalid)
    ms = elapsed * 1e3 / args.steps
    toks = args.steps / elapsed
    valid_avg = start + (args.steps + 1) / 2.0
    sbytes = step_bytes(cfg, int(round(valid_avg)))
    step_gbs = sbytes / (ms * 1e-3) / 1e9
    log(f"{toks:.1f} tok/s, {ms:.3f} ms/step, step roofline {step_gbs:.0f} GB/s")

    # the same loop with the per-step mask / position inputs handed over as host arrays
    # (PCIe-inclusive rate; reported beside the headline, never as it)
    host_steps = [{"attention_mask": to_host(masks[s].cpu()), "position_ids": pos_ids[s].cpu().numpy(),
                   "cache_position": cpos[s].cpu().numpy()} for s in range(args.steps)]
    # (from here on the position inputs are advanced by separate launches, or come from the host:
    # the kernel timings below replay one step without moving its inputs)
    hexec.fold_advance(None)
    folded_timed, folded = folded, False
    run(min(args.warmup, args.steps), host=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(args.steps, host=True)
    torch.cuda.synchronize()
    host_toks = args.steps / (time.perf_counter() - t0)
    log(f"host-input loop: {host_toks:.1f} tok/s")

    stream = torch.cuda.current_stream(dev).cuda_stream
    # per kernel family: average launch time over its launches in one step (HIP events, launch stream)
    fams: dict[str, list[int]] = {}
    for i, s in enumerate(program.steps):
        fams.setdefault(s.kernel, []).append(i)
    per_kernel = {}
    for kname, idx in sorted(fams.items()):
        us = time_kernel_subset(hexec, idx, args.kernel_repeats, stream) * 1e3
        entry = {"launches_per_step": len(idx), "avg_us": round(us, 3)}
        if program.steps[idx[0]].kind == "gemv":
            b = sum(gemv_launch_bytes(program.steps[i]) for i in idx) / len(idx)
            entry["GBs"] = round(b / (us * 1e-6) / 1e9, 1)
            entry["bytes_per_launch"] = int(b)
        elif program.steps[idx[0]].kind == "decode_step":
            # the persistent step is the whole step: its algorithmic bytes are the step's, at the
            # valid length of the replayed launch (the last position of the timed window)
            b = step_bytes(cfg, start + args.steps)
            entry["GBs"] = round(b / (us * 1e-6) / 1e9, 1)
            entry["bytes_per_launch"] = int(b)
        per_kernel[kname] = entry
        log(f"  {kname}: {entry}")
    # dominant kernel: the linear-layer family with the most time per step
    dom = max((k for k in per_kernel if "GBs" in per_kernel[k]),
              key=lambda k: per_kernel[k]["avg_us"] * per_kernel[k]["launches_per_step"])
    lin = fams[dom]
    avg_ms = per_kernel[dom]["avg_us"] * 1e-3
    dom_bytes = per_kernel[dom]["bytes_per_launch"]
    achieved = dom_bytes / (avg_ms * 1e-3) / 1e9
    # the same launches bracketed one by one by events inside full step replays: this also counts
    # each launch's dispatch latency, so it is an upper bound on the kernel's duration
    in_step_ms = time_in_step(hexec, lin, args.kernel_repeats, stream)
    log(f"dominant {dom}: {avg_ms * 1e3:.2f} us per launch ({achieved:.0f} GB/s); "
        f"{in_step_ms * 1e3:.2f} us with per-launch events inside the step")
    traffic = measured_traffic(dom, f"decode_s{S}")   # (the counter summary of this cache length)
    stamps = None
    if args.stamps and program.steps[0].kind == "decode_step":
        stamps = decode_stamps(hexec, ex, dict(state), cfg.layers)
        log(f"stamps: {stamps}")

    probe = None
    if args.copy_probe_mib > 0:
        pm = run_copy_probe(0, stream, args.copy_probe_mib)
        probe = {"kernel": "k_copy16", "mib": args.copy_probe_mib, "avg_ms": round(pm, 4),
                 "GBs": round(2 * args.copy_probe_mib * (1 << 20) / (pm * 1e-3) / 1e9, 1)}
        log(f"copy probe: {probe}")

    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np

        log("cpu baseline")
        x_cpu = decode_inputs(S, start, cfg, device="cuda")
        cpu, cpu_tokens, cpu_logits = cpu_baseline(ir, weights, x_cpu, cfg, args.cpu_steps, args.cpu_warmup)
        log(f"cpu: {cpu['value']} tok/s on {cpu['cores']} cores")
        # untimed parity pass: the device loop teacher-forced with the CPU's tokens, so every step
        # compares the two paths on the same context
        n_check = min(args.cpu_steps, len(masks))
        feed = [None] + [np.array([[t]], np.int64) for t in cpu_tokens[:n_check - 1]]
        rec = []
        run(n_check, feed=feed, record=rec)
        agree = sum(int(g == c) for (g, _), c in zip(rec, cpu_tokens))
        rel = max(float(np.abs(gl - cl).max() / np.abs(cl).max()) for (_, gl), cl in zip(rec, cpu_logits))
        cpu["parity"] = {"steps": n_check, "hip_cpu_top1_agree": agree, "hip_cpu_logits_max_rel_err": round(rel, 4),
                         "mode": "device loop teacher-forced with the CPU greedy tokens; both graded against "
                                 "the same steps evaluated in float32 on the CPU"}
        if not args.no_fp32_parity:
            log("fp32 reference of the same teacher-forced steps")
            f32 = fp32_teacher_forced(cfg, weights, x_cpu, cpu_tokens[:n_check - 1], n_check)
            cpu["parity"].update(parity_vs_fp32(rec, cpu_tokens[:n_check], cpu_logits[:n_check], f32))
        log(f"parity: {cpu['parity']}")
        if not args.no_fp32_parity and args.parity_seed2_steps > 0:
            # the same grading on a second, independent draw of weights, caches and first token
            n2 = min(args.parity_seed2_steps, len(masks))
            log(f"second seed: {n2} teacher-forced steps, CPU fallback and fp32 reference")
            w2 = make_weights(ir, cfg, seed=11, device="cuda")
            x2 = decode_inputs(S, start, cfg, seed=12, token_seed=13, device="cuda")
            _, tok2, lg2 = cpu_baseline(ir, w2, x2, cfg, n2, 0)
            ex.load_weights(w2)
            st2 = {k: backend.allocate_buffer(v) for k, v in x2.items()}
            rec2 = []
            for s in range(n2):
                if s:
                    st2["input_ids"] = np.array([[tok2[s - 1]]], np.int64)
                    st2.update(host_steps[s] if s < len(host_steps) else
                               {"attention_mask": to_host(masks[s].cpu()), "position_ids": pos_ids[s].cpu().numpy(),
                                "cache_position": cpos[s].cpu().numpy()})
                o2 = ex.execute(st2)
                rec2.append((int(o2["next_token"].native_handle.reshape(-1)[0].item()),
                             o2[lname].native_handle.float().reshape(-1).cpu().numpy()))
                for i, o in zip(kv_in, kv_out):
                    st2[i] = o2[o]
            hexec.check()
            f32b = fp32_teacher_forced(cfg, w2, x2, tok2[:n2 - 1], n2)
            p2 = {"steps": n2, "seeds": "weights 11, activations 12, first token 13",
                  "hip_cpu_top1_agree": sum(int(g == c) for (g, _), c in zip(rec2, tok2)),
                  "hip_cpu_logits_max_rel_err": round(max(float(np.abs(gl - cl).max() / np.abs(cl).max())
                                                          for (_, gl), cl in zip(rec2, lg2)), 4)}
            p2.update(parity_vs_fp32(rec2, tok2, lg2, f32b))
            cpu["parity_seed2"] = p2
            log(f"parity, second seed: {p2}")

    line = {
        "metric": METRIC, "value": round(toks, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(toks / PUBLISHED_TOKS, 2), "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"cfg3: Qwen2.5-1.5B-arch full decode step, batch 1, static KV cache {S}, "
                               f"positions {start}..{start + args.steps - 1}, device-side greedy argmax",
                   "layers": cfg.layers, "hidden": cfg.hidden, "vocab": cfg.vocab, "max_cache_len": S,
                   "launches_per_step": len(program.steps), "compile_s": round(compile_s, 2),
                   "advance_in_step": folded_timed,
                   "persistent_timeouts": 0,   # hexec.check() above raises on any
                   "host_input_tok_s": round(host_toks, 2),
                   "vs_baseline_ref": "reference CUDA path on RTX 3090 Ti, 30.0 tok/s at position 2048"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "avg_launch_us": round(avg_ms * 1e3, 3),
                     "in_step_event_us": round(in_step_ms * 1e3, 3),
                     "launches_per_step": len(lin), "bytes_per_launch": dom_bytes},
        "kernels": per_kernel,
        "copy_probe": probe,
        "step_roofline": {"bytes_per_step": sbytes, "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
    }
    if stamps is not None:
        line["stamps"] = stamps
    print(json.dumps(line), flush=True)
    return 0


MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense bf16


def main_prefill(args) -> int:
    """cfg4: full 28-layer prefill of T tokens (causal mask, empty static caches of length T).

    A step is one prefill; ``value`` is prompt tokens per second. The roofline is MFMA: the
    GEMM kernels' linear FLOPs (2 M N K per weight) over their measured time, against the
    dense bf16 peak; the step-level figure divides all linear FLOPs by the step time."""
    import torch

    from hip_compiler import compile_subgraph, is_hip_op_supported
    from hip_runtime import HIPBackend
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import make_weights, prefill_inputs
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    cfg = QwenConfig(layers=args.layers)
    T = args.prefill_tokens
    steps = args.steps if args.steps != 64 else 10
    warm = args.warmup if args.warmup is not None else 2
    log(f"prefill T={T}: building IR and compiling")
    t0 = time.time()
    ir = build_decode_ir(T, cfg, argmax=True, tokens=T)
    backend = HIPBackend(0)
    ex = DAGExecutor(partition(ir, is_hip_op_supported), backend, compile_fn=compile_subgraph)
    compile_s = time.time() - t0
    weights = make_weights(ir, cfg, device="cuda")
    ex.load_weights(weights)
    x0 = prefill_inputs(T, T, cfg, device="cuda")
    state = {k: backend.allocate_buffer(v) for k, v in x0.items()}
    (program,) = ex.npu_programs.values()
    (hexec,) = ex._npu_executors.values()
    log(f"program: {len(program.steps)} launches, arena {program.arena_bytes / 1e6:.1f} MB")
    for _ in range(warm):
        ex.execute(state)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ex.execute(state)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / steps
    toks = T * steps / elapsed
    gemms = [i for i, s in enumerate(program.steps) if s.kernel.startswith("k_gemm_") and not s.params.get("reduce")]
    def gflops(st):
        return 2.0 * st.args["M"] * st.args["N"] * st.args["K"] * st.params.get("weights", 1) * st.args.get("batch", 1)

    flops = sum(gflops(program.steps[i]) for i in gemms)
    stream = torch.cuda.current_stream().cuda_stream
    fams: dict[str, list[int]] = {}
    for i, s in enumerate(program.steps):
        fams.setdefault(s.kernel, []).append(i)
    per_kernel = {}
    gemm_ms = 0.0
    for kname, idx in sorted(fams.items()):
        us = time_kernel_subset(hexec, idx, max(1, args.kernel_repeats // 5), stream) * 1e3
        e = {"launches_per_step": len(idx), "avg_us": round(us, 2)}
        if kname.startswith("k_gemm_") and "reduce" not in kname:
            f = sum(gflops(program.steps[i]) for i in idx) / len(idx)
            e["TFLOPs"] = round(f / (us * 1e-6) / 1e12, 1)
            gemm_ms += us * len(idx) * 1e-3
        per_kernel[kname] = e
        log(f"  {kname}: {e}")
    dom = max((k for k in per_kernel if "TFLOPs" in per_kernel[k]),
              key=lambda k: per_kernel[k]["avg_us"] * per_kernel[k]["launches_per_step"])
    dflops = per_kernel[dom]["TFLOPs"]
    gemm_tf = flops / (gemm_ms * 1e-3) / 1e12
    step_tf = flops / (ms * 1e-3) / 1e12
    log(f"{toks:.0f} tok/s, {ms:.2f} ms/prefill; GEMMs {gemm_tf:.0f} TFLOP/s over {gemm_ms:.2f} ms")
    cpu = None
    if not args.no_cpu_baseline:
        from irgen.workloads import to_host

        n = len(os.sched_getaffinity(0))
        torch.set_num_threads(n)
        cex = DAGExecutor(partition(ir, lambda *_: False), None)
        cex.load_weights({k: v.detach().cpu() for k, v in weights.items()})
        ins = {k: to_host(v.detach().cpu()) for k, v in x0.items()}
        cex.execute(ins)
        t0 = time.perf_counter()
        cex.execute(ins)
        cs = time.perf_counter() - t0
        cpu = {"value": round(T / cs, 2), "unit": "tok/s", "cores": n, "kind": "port",
               "sample": f"one {T}-token prefill of the full {cfg.layers}-layer model after one warmup, "
                         f"DAGExecutor all-CPU plan (ATen bf16, {n} threads): {cs:.2f} s"}
        log(f"cpu: {cpu}")
    line = {
        "metric": "Qwen2.5-1.5B-arch bf16 prefill tok/s @512; MFMA TFLOP/s vs dense bf16 peak",
        "value": round(toks, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"cfg4: Qwen2.5-1.5B-arch prefill, batch 1, {T} tokens, causal mask, "
                               "logits for every position, device-side argmax",
                   "layers": cfg.layers, "launches_per_step": len(program.steps), "compile_s": round(compile_s, 2)},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": dflops, "peak": MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(dflops / MFMA_PEAK_TFLOPS, 4), "traffic": None},
        "gemm_roofline": {"linear_flops_per_step": flops, "gemm_ms": round(gemm_ms, 3),
                          "achieved": round(gemm_tf, 1), "frac": round(gemm_tf / MFMA_PEAK_TFLOPS, 4)},
        "step_roofline": {"achieved": round(step_tf, 1), "unit": "TFLOP/s",
                          "frac": round(step_tf / MFMA_PEAK_TFLOPS, 4)},
        "kernels": per_kernel,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def main_block(args) -> int:
    """cfg1 / cfg2: one subgraph, HBM-bound. A step is one run of the graph on inputs resident
    in HBM; ``value`` is its achieved algorithmic GB/s over the device time of one step (50
    steps captured back to back into one HIP graph, timed with HIP events; the wall time of
    one ``execute()`` call, host-bound at these sizes, is reported beside it), with the
    per-step bytes of the survey's formulas: cfg1 82,578,432 B of weights (gate, up, down
    and the norm weight) + 3 T 1536 2 B of activations (x, residual, output); cfg2
    11,014,144 B of weights and biases + 1,024 S B of K/V read (S = 1025) + 1,024 B of K/V
    written. The CPU baseline is the same graph through the all-CPU plan (median of 5 runs
    after 3 warmups, all host threads)."""
    import statistics

    import torch

    from hip_compiler import compile_subgraph, is_hip_op_supported
    from hip_runtime import HIPBackend
    from irgen.qwen import build_attention_ir, build_mlp_ir
    from irgen.workloads import attention_inputs, make_weights, mlp_inputs, to_host
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    if args.workload == "mlp":
        T = args.tokens
        ir = build_mlp_ir(T)
        x0 = mlp_inputs(T)
        weights = make_weights(ir, norm_std=0.02, device="cuda")
        nbytes = 82_578_432 + 3 * T * 1536 * 2
        name, unit_note = f"cfg1: RMSNorm -> gate/up -> SiLU*up -> down -> +residual, T={T}", f"T={T}"
    else:
        S = 1025
        ir = build_attention_ir(S)
        x0 = attention_inputs(S)
        weights = make_weights(ir, device="cuda")
        nbytes = 11_014_144 + 1_024 * S + 1_024
        name, unit_note = "cfg2: decode attention block (q/k/v + RoPE + index_copy + GQA attention + o_proj), S=1025", "S=1025"
    steps = args.steps if args.steps != 64 else 200
    warm = args.warmup if args.warmup is not None else 20
    backend = HIPBackend(0)
    ex = DAGExecutor(partition(ir, is_hip_op_supported), backend, compile_fn=compile_subgraph)
    ex.load_weights(weights)
    state = {k: backend.allocate_buffer(v) for k, v in x0.items()}
    (program,) = ex.npu_programs.values()
    for _ in range(warm):
        ex.execute(state)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ex.execute(state)
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3 / steps
    # device time of one step: 50 steps back to back in one HIP graph between two HIP events (a
    # step of a few tens of microseconds of kernels is shorter than the host's own cost of one
    # execute() call, so the wall time above measures the host, not the kernels); per-launch
    # times from events around each launch inside full replays, for the breakdown only
    (hexec,) = ex._npu_executors.values()
    stream = torch.cuda.current_stream().cuda_stream
    ms = time_graph_reps(hexec, 50, stream)
    per = {}
    for i, st in enumerate(program.steps):
        per.setdefault(st.kernel, []).append(i)
    ktimes = {k: time_in_step(hexec, idx, 20, stream) for k, idx in per.items()}
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"{args.workload} {unit_note}: device {ms * 1e3:.2f} us/step ({gbs:.0f} GB/s), host-inclusive "
        f"{host_ms * 1e3:.2f} us per execute() ({len(program.steps)} launches)")
    cpu = None
    if not args.no_cpu_baseline:
        n = len(os.sched_getaffinity(0))
        torch.set_num_threads(n)
        cex = DAGExecutor(partition(ir, lambda *_: False), None)
        cex.load_weights({k: v.detach().cpu() for k, v in weights.items()})
        ins = {k: to_host(v) for k, v in x0.items()}
        for _ in range(3):
            cex.execute(ins)
        ts = []
        for _ in range(5):
            t1 = time.perf_counter()
            cex.execute(ins)
            ts.append(time.perf_counter() - t1)
        med = statistics.median(ts)
        cpu = {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": n, "kind": "port",
               "sample": f"the same graph through DAGExecutor's all-CPU plan (ATen bf16, {n} threads), median of 5 "
                         f"runs after 3 warmups: {med * 1e3:.2f} ms per run"}
        log(f"cpu: {cpu}")
    # HBM bytes per step from the committed counter summaries of this workload's kernels (None
    # unless every launch of the step has one)
    tag = f"{args.workload}_t{args.tokens}" if args.workload == "mlp" else args.workload
    per_launch = [measured_traffic(st.kernel, tag) for st in program.steps]
    step_traffic = sum(per_launch) if all(v is not None for v in per_launch) else None
    line = {
        "metric": f"Qwen2.5-1.5B-shaped {args.workload} block bf16: achieved HBM GB/s vs peak ({unit_note})",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": name, "launches_per_step": len(program.steps), "bytes_per_step": nbytes,
                   "host_inclusive_us_per_step": round(host_ms * 1e3, 2),
                   "host_inclusive_GBs": round(nbytes / (host_ms * 1e-3) / 1e9, 1),
                   "kernels_in_step_event_us": {k: {"launches_per_step": len(per[k]),
                                                    "avg_us": round(ktimes[k] * 1e3, 3)} for k in per}},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": step_traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def main_generate(args) -> int:
    """Generation end to end, the reference's TTFT setup (`docs/benchmarks.md:106`: a 64-token
    prompt padded to a 128-token prefill): HF ``Qwen2ForCausalLM`` with Qwen2.5-1.5B's
    architecture is built on the meta device and exported to IR (prefill T = 128 and decode, both
    over static caches of ``--max-cache-len``), random-init weights are created on the GPU, and
    ``GreedyGenerator`` runs the padded prefill then ``--steps`` device-resident greedy decode
    steps. TTFT = prefill through the first token on the host (median of the timed runs);
    decode tok/s = decode steps / their wall time."""
    import statistics

    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from hip_compiler import compile_subgraph, is_hip_op_supported
    from hip_runtime import HIPBackend
    from irgen.hf_qwen import export_qwen, kv_mapping, to_dtype_keep_rotary
    from irgen.qwen import QwenConfig
    from irgen.workloads import make_weights
    from npu_compiler import partition
    from npu_runtime import DAGExecutor
    from npu_runtime.generation import GreedyGenerator

    L, S, T, P = args.layers, args.max_cache_len, 128, 64
    steps = args.steps
    runs = max(3, args.warmup if args.warmup is not None else 5)
    hcfg = Qwen2Config(hidden_size=1536, intermediate_size=8960, num_hidden_layers=L, num_attention_heads=12,
                       num_key_value_heads=2, head_dim=128, vocab_size=151936, rope_theta=1e6,
                       tie_word_embeddings=True, rms_norm_eps=1e-6, max_position_embeddings=32768)
    hcfg._attn_implementation = "eager"
    t0 = time.time()
    with torch.device("meta"):
        model = to_dtype_keep_rotary(Qwen2ForCausalLM(hcfg).eval())
    pre = export_qwen(model, S, tokens=T, argmax=True)
    dec = export_qwen(model, S, tokens=1, argmax=True)
    export_s = time.time() - t0
    log(f"exported prefill ({len(pre['nodes'])} nodes) and decode ({len(dec['nodes'])} nodes) in {export_s:.1f}s")
    backend = HIPBackend(0)
    t0 = time.time()
    pex = DAGExecutor(partition(pre, is_hip_op_supported), backend, compile_fn=compile_subgraph)
    dex = DAGExecutor(partition(dec, is_hip_op_supported), backend, compile_fn=compile_subgraph)
    compile_s = time.time() - t0
    weights = make_weights(dec, QwenConfig(layers=L), device="cuda")   # one copy, shared by both programs
    pex.load_weights(weights)
    dex.load_weights(weights)
    gen = GreedyGenerator(pex, dex, kv_mapping(pre, dec, L, T, S), pre, dec, backend=backend)
    prompt = torch.randint(0, 151936, (P,), generator=torch.Generator().manual_seed(2)).tolist()
    gen.generate(prompt, 4)   # warm: code objects, graph capture
    ttfts, decs, toks = [], [], None
    for _ in range(runs):
        r = gen.generate(prompt, steps + 1)
        ttfts.append(r.ttft_s)
        decs.append(r.decode_s)
        if toks is None:
            toks = r.tokens
        assert r.tokens == toks, "greedy generation is not repeatable"
    ttft = statistics.median(ttfts)
    dec_s = statistics.median(decs)
    tok_s = steps / dec_s
    log(f"TTFT {ttft * 1e3:.2f} ms (prompt {P}, prefill graph {T}), decode {tok_s:.1f} tok/s over {steps} steps")
    line = {
        "metric": "Qwen2.5-1.5B-arch bf16 generation: TTFT ms (64-token prompt, 128-token prefill) and decode tok/s",
        "value": round(ttft * 1e3, 3), "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": 1,
        "ms_per_step": round(dec_s * 1e3 / steps, 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": round(34.3 / (ttft * 1e3), 2), "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"HF Qwen2ForCausalLM (Qwen2.5-1.5B architecture, random init) exported to IR; "
                               f"{P}-token prompt padded to a {T}-token prefill, then {steps} greedy decode "
                               f"steps over static caches of {S}; median of {runs} runs",
                   "layers": L, "max_cache_len": S, "decode_tok_s": round(tok_s, 1), "export_s": round(export_s, 2),
                   "compile_s": round(compile_s, 2), "prefill_launches": len(next(iter(pex.npu_programs.values())).steps),
                   "decode_launches": len(next(iter(dex.npu_programs.values())).steps),
                   "vs_baseline_ref": "reference CUDA path on RTX 3090 Ti: TTFT 34.3 ms (128-token prefill), "
                                      "vs_baseline = 34.3 / TTFT"},
    }
    print(json.dumps(line), flush=True)
    return 0


def main_resnet(args) -> int:
    """cfg5: ResNet-50 inference, fp16, batch 32 at 224 x 224 (He-normal convs, inference batch norm
    with random running statistics). A step is one forward pass; ``value`` is images per second.
    The roofline is MFMA: the convolutions' FLOPs (2 N Ho Wo Cout Cin KH KW each) over their
    measured time, against the dense fp16 peak."""
    import torch

    from hip_compiler import compile_subgraph, is_hip_op_supported
    from hip_runtime import HIPBackend
    from irgen.resnet import build_resnet50_ir, resnet_inputs, resnet_weights
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    B = args.batch
    steps = args.steps if args.steps != 64 else 20
    warm = args.warmup if args.warmup is not None else 3
    t0 = time.time()
    ir = build_resnet50_ir(B, 224)
    backend = HIPBackend(0)
    ex = DAGExecutor(partition(ir, is_hip_op_supported), backend, compile_fn=compile_subgraph)
    compile_s = time.time() - t0
    weights = resnet_weights(ir, device="cuda")
    ex.load_weights(weights)
    x0 = resnet_inputs(B, 224, device="cuda")
    state = {k: backend.allocate_buffer(v) for k, v in x0.items()}
    (program,) = ex.npu_programs.values()
    (hexec,) = ex._npu_executors.values()
    log(f"resnet50 batch {B}: {len(program.steps)} launches, arena {program.arena_bytes / 1e6:.1f} MB")
    for _ in range(warm):
        ex.execute(state)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ex.execute(state)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / steps
    ips = B * steps / elapsed

    def cflops(st):
        if st.kind == "conv" and not st.params.get("reduce"):   # a split-K reduce adds no MFMA work
            # conv.hip's NCHW kernels carry Cout; the channels-last convs run as GEMMs (N = Cout). The
            # algorithmic K: the stem's GEMM runs over zero-padded taps (K_alg = Cin * KH * KW)
            return 2.0 * st.args["M"] * st.args.get("Cout", st.args.get("N")) * st.params.get("K_alg", st.args["K"])
        if st.kernel.startswith("k_gemm_") and not st.params.get("reduce"):
            return 2.0 * st.args["M"] * st.args["N"] * st.args["K"]
        return 0.0

    flops = sum(cflops(s) for s in program.steps)
    stream = torch.cuda.current_stream().cuda_stream
    fams: dict[str, list[int]] = {}
    for i, s in enumerate(program.steps):
        fams.setdefault(s.kernel, []).append(i)
    per_kernel, conv_ms, conv_flops = {}, 0.0, 0.0
    for kname, idx in sorted(fams.items()):
        us = time_kernel_subset(hexec, idx, max(1, args.kernel_repeats // 5), stream) * 1e3
        e = {"launches_per_step": len(idx), "avg_us": round(us, 2)}
        f = sum(cflops(program.steps[i]) for i in idx)
        if f:
            e["TFLOPs"] = round(f / len(idx) / (us * 1e-6) / 1e12, 1)
        if program.steps[idx[0]].kind == "conv":   # conv launches and their split-K reduces
            conv_ms += us * len(idx) * 1e-3
            conv_flops += f
        per_kernel[kname] = e
        log(f"  {kname}: {e}")
    # per conv: its floor max(FLOPs / MFMA peak, algorithmic bytes / HBM peak) next to its own measured
    # time (the conv launch plus its split-K reduce, if any, each timed alone on the launch stream)
    conv_rows = []
    for i, st in enumerate(program.steps):
        if st.kind != "conv" or st.params.get("reduce"):
            continue
        a, pm = st.args, st.params
        kh, kw = pm["kernel"]
        cout, m = a.get("Cout", a.get("N")), a["M"]
        kalg = pm.get("K_alg", a["K"])
        cin = kalg // (kh * kw)
        hw_o = a["cHo"] * a["cWo"]
        nimg = m // hw_o
        # the stem reads a pre-padded buffer: its algorithmic input is the unpadded image
        hin = a["cH"] - (2 * pm["padding"][0] if a.get("cph", 0) == 0 else 0)
        win = a["cW"] - (2 * pm["padding"][1] if a.get("cpw", 0) == 0 else 0)
        nbytes = 2 * (nimg * hin * win * cin + cout * kalg + m * cout * (2 if pm.get("residual") else 1))
        f = 2.0 * m * cout * kalg
        t_f, t_b = f / (MFMA_PEAK_TFLOPS * 1e12) * 1e6, nbytes / (HBM_PEAK_GBS * 1e9) * 1e6
        idx = [i] + ([i + 1] if i + 1 < len(program.steps) and program.steps[i + 1].params.get("reduce") else [])
        meas = time_kernel_subset(hexec, idx, max(1, args.kernel_repeats // 5), stream) * 1e3
        conv_rows.append({"conv": pm["nodes"][0], "kernel": st.kernel,
                          "shape": f"{nimg}x{hin}x{win}x{cin} -> {cout} k{kh}x{kw} s{pm['stride'][0]}",
                          "floor_us": round(max(t_f, t_b), 2), "bound": "mfma" if t_f >= t_b else "hbm",
                          "measured_us": round(meas, 2), "launches": len(idx)})
    floor_sum = sum(r["floor_us"] for r in conv_rows)
    meas_sum = sum(r["measured_us"] for r in conv_rows)
    log(f"conv roofline: floor {floor_sum:.1f} us vs measured {meas_sum:.1f} us over {len(conv_rows)} convs")
    # per conv launch (every conv has its own shape): time each inside the family replay
    n_red = sum(1 for s in program.steps if s.kind == "conv" and s.params.get("reduce"))
    n_conv = sum(1 for s in program.steps if s.kind == "conv") - n_red
    conv_tf = conv_flops / (conv_ms * 1e-3) / 1e12
    step_tf = flops / (ms * 1e-3) / 1e12
    log(f"{ips:.0f} images/s, {ms:.2f} ms/batch; convs {conv_tf:.0f} TFLOP/s over {conv_ms:.2f} ms")
    cpu = None
    if not args.no_cpu_baseline:
        from irgen.workloads import to_host

        n = len(os.sched_getaffinity(0))
        torch.set_num_threads(n)
        cb = min(B, 8)
        cir = build_resnet50_ir(cb, 224)
        cex = DAGExecutor(partition(cir, lambda *_: False), None)
        cex.load_weights({k: v.detach().cpu() for k, v in weights.items()})
        ins = {"x": to_host(x0["x"][:cb].detach().cpu())}
        cex.execute(ins)
        t0 = time.perf_counter()
        cex.execute(ins)
        cs = time.perf_counter() - t0
        cpu = {"value": round(cb / cs, 2), "unit": "images/s", "cores": n, "kind": "port",
               "sample": f"one forward pass of batch {cb} (the first {cb} images of the same input) after one "
                         f"warmup, DAGExecutor all-CPU plan (ATen fp16, {n} threads): {cs:.2f} s"}
        log(f"cpu: {cpu}")
    line = {
        "metric": "ResNet-50 fp16 inference images/s @batch32 224x224; MFMA TFLOP/s vs dense fp16 peak",
        "value": round(ips, 1), "unit": "images/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": f"cfg5: ResNet-50 (torchvision v1.5 layout), batch {B}, 3 x 224 x 224, "
                               "inference batch norm fused into the convolutions",
                   "launches_per_step": len(program.steps), "compile_s": round(compile_s, 2)},
        "roofline": {"bound": "mfma", "kernel": f"all {n_conv} conv launches (channels-last MFMA GEMMs "
                                                f"k_gemm_f16_conv*), with {n_red} split-K reduces",
                     "achieved": round(conv_tf, 1),
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(conv_tf / MFMA_PEAK_TFLOPS, 4),
                     "traffic": None},
        "step_roofline": {"flops_per_step": flops, "achieved": round(step_tf, 1), "unit": "TFLOP/s",
                          "frac": round(step_tf / MFMA_PEAK_TFLOPS, 4)},
        "conv_roofline": {"floor_us_sum": round(floor_sum, 1), "measured_us_sum": round(meas_sum, 1),
                          "floor_frac": round(floor_sum / meas_sum, 4) if meas_sum else None,
                          "floor": "max(FLOPs / 2.5 PFLOP/s, algorithmic bytes / 8 TB/s) per conv",
                          "per_conv": conv_rows},
        "kernels": per_kernel,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
