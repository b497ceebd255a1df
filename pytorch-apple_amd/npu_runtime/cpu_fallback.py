"""CPU fallback for IR partitions the device does not run.

Same API as the reference (`npu_runtime/cpu_fallback.py:32-194`):
``execute_cpu_partition``, ``build_cpu_executor`` and
``execute_cpu_partition_cached``. Tensors cross the boundary as numpy arrays;
bfloat16 crosses as ``uint16`` bit patterns (the reference uses ``ml_dtypes``,
absent here, and already accepts ``uint16`` on the way in, `cpu_fallback.py:178-181`).
Every tensor produced by the partition is returned, as in the reference
(`cpu_fallback.py:102`). Execution goes through ``ATenExecutor``, this build's
restatement of the schema-based ATen interpreter the reference imports from
``torch_ir``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from npu_runtime.aten_executor import ATenExecutor


@dataclass
class CPUPartitionIR:
    nodes: list[dict]
    graph_inputs: list[dict]
    graph_outputs: list[dict]
    weights: list[dict]
    weight_name_mapping: dict[str, str]


def _external_inputs(nodes: list[dict]) -> dict[str, dict]:
    produced = {o["name"] for n in nodes for o in n.get("outputs", [])}
    ext: dict[str, dict] = {}
    for n in nodes:
        for i in n.get("inputs", []):
            if i["name"] not in produced and i["name"] not in ext:
                ext[i["name"]] = i
    return ext


def _build_sub_ir(nodes, weights, weight_name_mapping) -> CPUPartitionIR:
    weight_names = set(weights.keys()) | set((weight_name_mapping or {}).keys())
    gi, ws = [], []
    for name, meta in _external_inputs(nodes).items():
        (ws if name in weight_names else gi).append(meta)
    outs = [o for n in nodes for o in n.get("outputs", [])]
    wn = {w["name"] for w in ws}
    wnm = {k: v for k, v in (weight_name_mapping or {}).items() if k in wn}
    return CPUPartitionIR(nodes=nodes, graph_inputs=gi, graph_outputs=outs, weights=ws,
                          weight_name_mapping=wnm)


def _torch_weights(sub: CPUPartitionIR, weights, weight_name_mapping) -> dict[str, torch.Tensor]:
    out: dict[str, torch.Tensor] = {}
    for w in sub.weights:
        name = w["name"]
        if name in weights:
            out[name] = numpy_to_torch(weights[name], w.get("dtype"))
        elif weight_name_mapping and weight_name_mapping.get(name) in weights:
            out[name] = numpy_to_torch(weights[weight_name_mapping[name]], w.get("dtype"))
    return out


def build_cpu_executor(partition_nodes: list[dict], weights: dict, weight_name_mapping: dict | None = None):
    """Build a reusable executor: returns ``(sub_ir, executor, torch_weights)``."""
    sub = _build_sub_ir(partition_nodes, weights, weight_name_mapping)
    tw = _torch_weights(sub, weights, weight_name_mapping)
    ex = ATenExecutor(partition_nodes, [g["name"] for g in sub.graph_inputs],
                      [o["name"] for o in sub.graph_outputs], tw)
    return sub, ex, tw


def execute_cpu_partition_cached(sub_ir: CPUPartitionIR, executor: ATenExecutor,
                                 tensor_pool: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
    ins = tuple(numpy_to_torch(tensor_pool[g["name"]], g.get("dtype")) for g in sub_ir.graph_inputs)
    res = executor.execute(ins)
    return {o["name"]: torch_to_numpy(t) for o, t in zip(sub_ir.graph_outputs, res)}


def execute_cpu_partition(partition_nodes: list[dict], tensor_pool: dict[str, np.ndarray],
                          weights: dict, weight_name_mapping: dict | None = None) -> dict[str, np.ndarray]:
    sub, ex, _ = build_cpu_executor(partition_nodes, weights, weight_name_mapping)
    return execute_cpu_partition_cached(sub, ex, tensor_pool)


def numpy_to_torch(arr, dtype: str | None = None) -> torch.Tensor:
    """numpy → CPU tensor; ``uint16`` (or a declared ``bfloat16``) is read as bf16 bits."""
    if isinstance(arr, torch.Tensor):
        return arr.detach().cpu()
    arr = np.asarray(arr)
    if arr.dtype == np.uint16 or (dtype == "bfloat16" and arr.dtype.itemsize == 2 and arr.dtype.kind in "ui"):
        return torch.from_numpy(arr.view(np.uint16).copy()).view(torch.bfloat16)
    if dtype == "bfloat16" and arr.dtype == np.float32:
        return torch.from_numpy(arr.copy()).to(torch.bfloat16)
    return torch.from_numpy(arr.copy())


def torch_to_numpy(t: torch.Tensor) -> np.ndarray:
    """CPU/GPU tensor → numpy; bf16 comes back as ``uint16`` bits."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.uint16).numpy().copy()
    return t.numpy().copy()
