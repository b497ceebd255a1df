"""Build IR dicts in the reference's schema by tracing ATen ops on meta tensors.

The reference obtains IR from ``torch_ir.extract_ir`` (absent here). This builder
emits the same schema (`npu_compiler/ir_reader.py:46-94`): every ``op()`` call
appends one node whose output shape/dtype come from running the very same ATen
overload on ``meta`` tensors through ``npu_runtime.aten_executor.run_node``, so the
declared dtypes follow ATen's promotion rules exactly as the CPU fallback will
compute them.
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass

import torch

from npu_runtime.aten_executor import run_node

_DTYPE_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16",
                torch.int64: "int64", torch.int32: "int32", torch.bool: "bool", torch.float64: "float64",
                torch.uint8: "uint8", torch.int8: "int8"}
_TORCH = {v: k for k, v in _DTYPE_NAMES.items()}


@dataclass
class T:
    """A traced tensor: IR name plus a meta tensor carrying shape and dtype."""

    name: str
    meta: torch.Tensor

    @property
    def shape(self) -> list[int]:
        return list(self.meta.shape)

    @property
    def dtype(self) -> str:
        return _DTYPE_NAMES[self.meta.dtype]

    def spec(self) -> dict:
        return {"name": self.name, "shape": self.shape, "dtype": self.dtype}


class IRBuilder:
    def __init__(self, model_name: str):
        self.model_name = model_name
        self.nodes: list[dict] = []
        self.graph_inputs: list[dict] = []
        self.graph_outputs: list[dict] = []
        self.weights: list[dict] = []
        self.weight_name_mapping: dict[str, str] = {}
        self._env: dict[str, torch.Tensor] = {}
        self._counts: Counter = Counter()
        self._weights_by_key: dict[str, T] = {}

    def _fresh(self, base: str) -> str:
        k = self._counts[base]
        self._counts[base] += 1
        return base if k == 0 else f"{base}_{k}"

    def input(self, name: str, shape, dtype: str) -> T:
        t = T(name, torch.empty(list(shape), dtype=_TORCH[dtype], device="meta"))
        self.graph_inputs.append(t.spec())
        self._env[name] = t.meta
        return t

    def weight(self, sd_key: str, shape, dtype: str, buffer: bool = False) -> T:
        """A parameter (placeholder ``p_*``) or buffer (``b_*``) mapped to ``sd_key``."""
        if sd_key in self._weights_by_key:
            return self._weights_by_key[sd_key]
        ph = ("b_" if buffer else "p_") + sd_key.replace(".", "_")
        t = T(ph, torch.empty(list(shape), dtype=_TORCH[dtype], device="meta"))
        self.weights.append({"name": sd_key, "shape": list(shape), "dtype": dtype})
        self.weight_name_mapping[ph] = sd_key
        self._env[ph] = t.meta
        self._weights_by_key[sd_key] = t
        return t

    def op(self, op_type: str, inputs: list[T], attrs: dict | None = None, n_out: int = 1,
           base: str | None = None, out_dtype: str | None = None):
        if base is None:
            base = op_type.split(".")[1] if op_type.startswith("aten.") else op_type
            base = base.lstrip("_")
        name = self._fresh(base)
        outs = [{"name": name if n_out == 1 else f"{name}_out{i}", "shape": [], "dtype": out_dtype or "float32",
                 "producer_node": name, "producer_output_idx": i} for i in range(n_out)]
        node = {"name": name, "op_type": op_type, "inputs": [t.spec() for t in inputs],
                "outputs": outs, "attrs": dict(attrs or {})}
        run_node(node, self._env)
        res = []
        for o in outs:
            m = self._env[o["name"]]
            o["shape"] = list(m.shape)
            o["dtype"] = _DTYPE_NAMES[m.dtype]
            res.append(T(o["name"], m))
        self.nodes.append(node)
        return res[0] if n_out == 1 else tuple(res)

    def getitem(self, multi: tuple[T, ...], index: int) -> T:
        name = self._fresh("getitem")
        src = multi[index]
        node = {"name": name, "op_type": "<built-in function getitem>", "inputs": [t.spec() for t in multi],
                "outputs": [{"name": name, "shape": src.shape, "dtype": src.dtype, "producer_node": name,
                             "producer_output_idx": 0}], "attrs": {"index": index}}
        self.nodes.append(node)
        self._env[name] = src.meta
        return T(name, src.meta)

    def output(self, *ts: T) -> None:
        for t in ts:
            self.graph_outputs.append(t.spec())

    def to_dict(self) -> dict:
        return {
            "model_name": self.model_name, "graph_inputs": self.graph_inputs,
            "graph_outputs": self.graph_outputs, "weights": self.weights,
            "weight_name_mapping": self.weight_name_mapping, "nodes": self.nodes, "constants": {},
        }
