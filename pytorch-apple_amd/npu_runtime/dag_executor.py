"""DAG executor: runs a PartitionPlan over a device backend plus the CPU fallback.

Same constructor, methods and data flow as the reference
(`npu_runtime/dag_executor.py:32-407`):

* ``__init__(plan, backend, compile_fn)`` calls ``compile_fn(sub_ir_dict)`` once
  per device partition and ``backend.create_executor(program)`` on the result;
* ``load_weights(weights)`` uploads each device partition's weights once and
  builds cached CPU executors for CPU partitions;
* ``execute(inputs, weights=None)`` walks the plan: device partitions receive
  DeviceBuffers (numpy inputs are written into pre-allocated input buffers), CPU
  partitions receive numpy arrays, ``TransferOp``s download/upload across the
  boundary, and graph outputs are returned as-is (DeviceBuffer or numpy).

Two defects of the reference's generic (non-Metal) path are not reproduced:
weights and pre-allocated inputs keep the dtype the program declares instead of
being forced to float16 (`dag_executor.py:114-115`, `127-128`, `145-146`), so
bfloat16 stays bfloat16 and int64 token ids stay exact.
"""

from __future__ import annotations

from typing import Any, Callable

import numpy as np

from npu_compiler.partitioner import Partition, PartitionPlan, TransferOp
from npu_runtime.backend import Backend, DeviceBuffer
from npu_runtime.cpu_fallback import build_cpu_executor, execute_cpu_partition, execute_cpu_partition_cached

_HOST_CARRIER = {"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16,
                 "int64": np.int64, "int32": np.int32, "float64": np.float64, "bool": np.bool_,
                 "uint8": np.uint8, "int8": np.int8}


def host_dtype(ir_dtype: str) -> np.dtype:
    """numpy carrier for an IR dtype string (bf16 travels as uint16 bits)."""
    return np.dtype(_HOST_CARRIER.get(ir_dtype, np.float32))


def _default_compile(sub_ir: dict):
    import npu_compiler

    return npu_compiler.compile(sub_ir)


class DAGExecutor:
    def __init__(self, plan: PartitionPlan, backend: Backend, compile_fn: Callable[[dict], Any] | None = None):
        self.plan = plan
        self.backend = backend
        self._compile_fn = compile_fn or _default_compile
        self.npu_programs: dict[int, Any] = {}
        self._npu_executors: dict[int, Any] = {}
        self._npu_weight_cache: dict[int, dict[str, DeviceBuffer]] = {}
        self._cpu_weights: dict | None = None
        self._cpu_irs: dict[int, Any] = {}
        self._cpu_executors: dict[int, Any] = {}
        self._npu_input_buffers: dict[int, dict[str, DeviceBuffer]] = {}
        self._output_names = [o["name"] for o in plan.original_ir.get("graph_outputs", [])]
        self._weight_name_mapping = plan.original_ir.get("weight_name_mapping")
        self._cpu_needed_inputs: dict[int, set[str]] = {}
        self._dispatch_table: list[tuple[str, Any, Any, Any]] = []

        for step in plan.steps:
            if isinstance(step, TransferOp):
                self._dispatch_table.append(("transfer", step, None, None))
                continue
            if step.target == "npu":
                program = self._compile_fn(_build_sub_ir_dict(step, plan.original_ir))
                self.npu_programs[step.partition_id] = program
                ex = backend.create_executor(program)
                self._npu_executors[step.partition_id] = ex
                self._dispatch_table.append(("npu", step, program, ex))
            else:
                reads = {i["name"] for n in step.nodes for i in n.get("inputs", [])}
                made = {o["name"] for n in step.nodes for o in n.get("outputs", [])}
                self._cpu_needed_inputs[step.partition_id] = reads - made
                self._dispatch_table.append(("cpu", step, None, None))

    # -- weights ---------------------------------------------------------------------------

    def _init_npu_input_buffers(self) -> None:
        for pid, program in self.npu_programs.items():
            bufs: dict[str, DeviceBuffer] = {}
            for spec in program.input_specs:
                bufs[spec.name] = self.backend.allocate_zeros(
                    tuple(spec.shape), dtype=host_dtype(spec.dtype),
                    alloc_shape=tuple(spec.alloc_shape) if spec.alloc_shape else None)
            self._npu_input_buffers[pid] = bufs

    def _load_weights_for_backend(self, weights: dict, program: Any) -> dict[str, DeviceBuffer]:
        reverse = {sd: ph for ph, sd in getattr(program, "weight_name_mapping", {}).items()}
        out: dict[str, DeviceBuffer] = {}
        for spec in program.weight_specs:
            sd_key = spec.name
            ph = reverse.get(sd_key, sd_key)
            if sd_key in weights:
                arr = weights[sd_key]
            elif ph in weights:
                arr = weights[ph]
            else:
                continue
            out[ph] = self.backend.allocate_buffer(arr, spec=spec)
        return out

    @property
    def npu_executors(self) -> dict:
        """The backend executor of each device partition (partition id -> executor), read-only."""
        return dict(self._npu_executors)

    def load_weights(self, weights: dict) -> None:
        self._cpu_weights = weights
        self._npu_weight_cache.clear()
        for pid, program in self.npu_programs.items():
            self._npu_weight_cache[pid] = self._load_weights_for_backend(weights, program)
        self._cpu_irs.clear()
        self._cpu_executors.clear()
        for step in self.plan.steps:
            if isinstance(step, Partition) and step.target == "cpu":
                sub, ex, _ = build_cpu_executor(step.nodes, weights, self._weight_name_mapping)
                self._cpu_irs[step.partition_id] = sub
                self._cpu_executors[step.partition_id] = ex
        if not self._npu_input_buffers:
            self._init_npu_input_buffers()

    # -- execution ---------------------------------------------------------------------------

    def execute(self, inputs: dict, weights: dict | None = None) -> dict:
        if weights is not None and not self._npu_weight_cache and not self._cpu_executors:
            self.load_weights(weights)
        elif weights is not None:
            self._cpu_weights = weights
        cpu_weights = self._cpu_weights or weights or {}

        pool: dict[str, Any] = dict(inputs)
        for kind, step, program, executor in self._dispatch_table:
            if kind == "transfer":
                self._execute_transfer(step, pool)
            elif kind == "npu":
                self._execute_npu_partition(step, pool, self._npu_weight_cache.get(step.partition_id, {}),
                                            program, executor)
            else:
                self._execute_cpu_partition(step, pool, cpu_weights)
        return {name: pool[name] for name in self._output_names}

    def _execute_npu_partition(self, partition: Partition, pool: dict, npu_weights: dict,
                               program: Any, executor: Any) -> None:
        pre = self._npu_input_buffers.get(partition.partition_id)
        dev_inputs: dict[str, DeviceBuffer] = {}
        for spec in program.input_specs:
            val = pool.get(spec.name)
            if val is None:
                continue
            if isinstance(val, np.ndarray):
                if pre and spec.name in pre:
                    pre[spec.name].write_from_numpy(val, spec=spec)
                    dev_inputs[spec.name] = pre[spec.name]
                else:
                    dev_inputs[spec.name] = self.backend.allocate_buffer(val, alloc_shape=spec.alloc_shape, spec=spec)
            else:
                dev_inputs[spec.name] = val
        pool.update(executor.run(dev_inputs, npu_weights))

    def _execute_cpu_partition(self, partition: Partition, pool: dict, weights: dict) -> None:
        pid = partition.partition_id
        needed = self._cpu_needed_inputs.get(pid) or set(pool.keys())
        cpu_pool: dict[str, np.ndarray] = {}
        for name in needed:
            val = pool.get(name)
            if val is None:
                continue
            cpu_pool[name] = val if isinstance(val, np.ndarray) else val.to_numpy(dtype=val.dtype)
        if pid in self._cpu_executors:
            res = execute_cpu_partition_cached(self._cpu_irs[pid], self._cpu_executors[pid], cpu_pool)
        else:
            res = execute_cpu_partition(partition.nodes, cpu_pool, weights, self._weight_name_mapping)
        pool.update(res)

    def _execute_transfer(self, op: TransferOp, pool: dict) -> None:
        for name in op.tensor_names:
            val = pool.get(name)
            if val is None:
                raise RuntimeError(
                    f"Transfer op expected tensor '{name}' but it was not found in pool. "
                    f"Available: {sorted(pool.keys())[:20]}")
            if op.direction == "to_cpu":
                if not isinstance(val, np.ndarray):
                    pool[name] = val.to_numpy(dtype=val.dtype)
            elif isinstance(val, np.ndarray):
                pool[name] = self.backend.allocate_buffer(val)


def _build_sub_ir_dict(part: Partition, original_ir: dict) -> dict:
    """IR dict of one device partition (`dag_executor.py:332-407`).

    External inputs that are weights (by placeholder mapping or by state-dict key)
    become ``weights``; the rest become ``graph_inputs``, followed by every original
    graph input the partition does not produce. Outputs are the produced tensors
    that are graph outputs or read by another partition, sorted by name.
    """
    produced = {o["name"] for n in part.nodes for o in n.get("outputs", [])}
    ext: dict[str, dict] = {}
    for n in part.nodes:
        for i in n.get("inputs", []):
            if i["name"] not in produced and i["name"] not in ext:
                ext[i["name"]] = i
    wmap = original_ir.get("weight_name_mapping", {})
    wkeys = {w["name"] for w in original_ir.get("weights", [])}
    gi, ws, wnm = [], [], {}
    for name, meta in ext.items():
        rec = {"name": name, "shape": meta["shape"], "dtype": meta.get("dtype", "float32")}
        if name in wmap:
            ws.append({**rec, "name": wmap[name]})
            wnm[name] = wmap[name]
        elif name in wkeys:
            ws.append(rec)
        else:
            gi.append(rec)
    have = {g["name"] for g in gi}
    for g in original_ir.get("graph_inputs", []):
        if g["name"] not in have and g["name"] not in produced:
            gi.append({"name": g["name"], "shape": g["shape"], "dtype": g.get("dtype", "float32")})
    wanted = {o["name"] for o in original_ir.get("graph_outputs", [])} | set(part.output_names)
    outs_by_name = {o["name"]: o for n in part.nodes for o in n.get("outputs", [])}
    go = [{"name": o["name"], "shape": o["shape"], "dtype": o.get("dtype", "float32"),
           "producer_node": o.get("producer_node"), "producer_output_idx": o.get("producer_output_idx", 0)}
          for nm, o in sorted(outs_by_name.items()) if nm in wanted]
    return {
        "model_name": original_ir.get("model_name", "sub_partition"),
        "graph_inputs": gi, "graph_outputs": go, "weights": ws, "weight_name_mapping": wnm,
        "nodes": part.nodes, "constants": original_ir.get("constants", {}),
    }
