"""Benchmark: Qwen2.5-1.5B-architecture bf16 decode on one MI355X (BASELINE cfg3).

A step is one decode step of the full 28-layer model (random-init bf16 weights
N(0, 0.02), tied embeddings) at batch 1 over static KV caches of length 2048,
run through ``DAGExecutor`` + the HIP backend, with the greedy next token computed
on the device and fed back as the next step's ``input_ids`` (no host sync inside
the timed region). Timed steps walk cache positions 1984..1984+K-1 (the
BASELINE's 64-step window for K=64); warmup steps run over the same positions
first, so the timed steps see exactly the caches a cold run would.

Printed JSON line: tok/s (whole job), ms/step, a ``roofline`` object for the
dominant kernel (the streaming linear kernel: algorithmic bytes per launch over
its average launch time, measured here with HIP events on the launch stream),
the step-level fraction of HBM peak, and a ``cpu_baseline`` measured on this
host's cores with the CPU fallback (DAGExecutor over an all-CPU plan, ATen bf16)
on a bounded sample of the same workload.
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
PUBLISHED_TOKS = 30.0   # reference CUDA path, RTX 3090 Ti, position 2048 (docs/benchmarks.md:98)


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


def cpu_baseline(ir, weights_dev, inputs_dev, cfg, steps: int) -> dict:
    """CPU fallback (all-CPU plan through DAGExecutor, ATen bf16) on ``steps`` decode steps."""
    import numpy as np
    import torch

    from irgen.workloads import decode_mask, to_host
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    w = {k: v.detach().cpu() for k, v in weights_dev.items()}
    x = {k: v.detach().cpu() for k, v in inputs_dev.items()}
    ex = DAGExecutor(partition(ir, lambda *_: False), None)
    ex.load_weights(w)
    ins = {k: to_host(v) for k, v in x.items()}
    times = []
    start = int(ins["cache_position"][0])
    for s in range(steps + 1):
        pos = start + s
        ins["attention_mask"] = to_host(decode_mask(ins["attention_mask"].shape[-1], pos))
        ins["position_ids"] = np.array([[pos]], np.int64)
        ins["cache_position"] = np.array([pos], np.int64)
        t0 = time.perf_counter()
        out = ex.execute(ins)
        times.append(time.perf_counter() - t0)
        ins["input_ids"] = out["next_token"]
        for i, o in zip([g["name"] for g in ir["graph_inputs"][4:]], [o["name"] for o in ir["graph_outputs"][1:-1]]):
            ins[i] = out[o]
    med = statistics.median(times[1:])
    return {"value": round(1.0 / med, 4), "unit": "tok/s", "cores": n, "kind": "port",
            "sample": f"{steps} decode steps (after 1 warmup) of the full 28-layer model at positions "
                      f"{start}..{start + steps}, DAGExecutor all-CPU plan (ATen bf16), median step "
                      f"{med * 1e3:.1f} ms"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--max-cache-len", type=int, default=2048)
    ap.add_argument("--start-pos", type=int, default=1984)
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layers", type=int, default=28)
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU; --gpus must be 1 (multi-GPU sharding is "
                                   "described in DESIGN.md, not implemented)"}))
        return 2

    import torch

    from hip_compiler import compile_subgraph, is_hip_op_supported
    from hip_runtime import HIPBackend
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, decode_mask, make_weights
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

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
    masks = [decode_mask(S, p).to(dev) for p in range(start, start + max(args.steps, args.warmup))]
    pos_ids = [torch.tensor([[p]], dtype=torch.int64, device=dev) for p in range(start, S)]
    cpos = [torch.tensor([p], dtype=torch.int64, device=dev) for p in range(start, S)]
    from hip_runtime import HIPBuffer

    state = {k: backend.allocate_buffer(v) for k, v in x0.items()}
    mask_t, pos_t, cpos_t = (state[k].native_handle for k in ("attention_mask", "position_ids", "cache_position"))

    def run(n_steps):
        st = state
        for s in range(n_steps):
            # per-step inputs are refreshed in place (device copies on the launch stream), so the
            # executor's pointers stay fixed and its captured graph is relaunched as-is
            mask_t.copy_(masks[s])
            pos_t.copy_(pos_ids[s])
            cpos_t.copy_(cpos[s])
            out = ex.execute(st)
            st["input_ids"] = out["next_token"]
            for i, o in zip(kv_in, kv_out):
                st[i] = out[o]
        return st

    log(f"warmup {args.warmup} steps")
    run(args.warmup)
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    run(args.steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / args.steps
    toks = args.steps / elapsed
    valid_avg = start + (args.steps + 1) / 2.0
    sbytes = step_bytes(cfg, int(round(valid_avg)))
    step_gbs = sbytes / (ms * 1e-3) / 1e9
    log(f"{toks:.1f} tok/s, {ms:.3f} ms/step, step roofline {step_gbs:.0f} GB/s")

    # dominant kernel: the streaming linear kernel (most algorithmic bytes per step)
    stream = torch.cuda.current_stream(dev).cuda_stream
    # per kernel family: average launch time over its launches in one step (HIP events, launch stream)
    fams: dict[str, list[int]] = {}
    for i, s in enumerate(program.steps):
        fams.setdefault(s.kernel, []).append(i)
    per_kernel = {}
    for kname, idx in sorted(fams.items()):
        us = time_kernel_subset(hexec, idx, 10, stream) * 1e3
        entry = {"launches_per_step": len(idx), "avg_us": round(us, 3)}
        if program.steps[idx[0]].kind == "gemv":
            b = sum(gemv_launch_bytes(program.steps[i]) for i in idx) / len(idx)
            entry["GBs"] = round(b / (us * 1e-6) / 1e9, 1)
            entry["bytes_per_launch"] = int(b)
        per_kernel[kname] = entry
        log(f"  {kname}: {entry}")
    dom = max((k for k in per_kernel if "GBs" in per_kernel[k]),
              key=lambda k: per_kernel[k]["avg_us"] * per_kernel[k]["launches_per_step"])
    avg_ms = per_kernel[dom]["avg_us"] * 1e-3
    achieved = per_kernel[dom]["GBs"]
    lin = fams[dom]
    lin_bytes = per_kernel[dom]["bytes_per_launch"] * len(lin)

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
        x_cpu = decode_inputs(S, start, cfg, device="cuda")
        cpu = cpu_baseline(ir, weights, x_cpu, cfg, args.cpu_steps)
        log(f"cpu: {cpu['value']} tok/s on {cpu['cores']} cores")

    line = {
        "metric": METRIC, "value": round(toks, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(toks / PUBLISHED_TOKS, 2), "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cfg3: Qwen2.5-1.5B-arch full decode step, batch 1, static KV cache 2048, "
                               f"positions {start}..{start + args.steps - 1}, device-side greedy argmax",
                   "layers": cfg.layers, "hidden": cfg.hidden, "vocab": cfg.vocab, "max_cache_len": S,
                   "launches_per_step": len(program.steps), "compile_s": round(compile_s, 2),
                   "vs_baseline_ref": "reference CUDA path on RTX 3090 Ti, 30.0 tok/s at position 2048"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None, "avg_launch_us": round(avg_ms * 1e3, 3),
                     "launches_per_step": len(lin), "bytes_per_launch": lin_bytes // len(lin)},
        "kernels": per_kernel,
        "step_roofline": {"bytes_per_step": sbytes, "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
