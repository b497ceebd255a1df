"""Schema-driven ATen interpreter for IR partitions on the host CPU.

The reference runs CPU partitions through ``torch_ir.IRExecutor`` from the
third-party package ``pytorch-ir`` 0.2.2 (pinned in the reference's
``uv.lock:1575-1584``; not vendored and not installed here). Its documented
contract (`docs/partitioning.md:56`, `npu_runtime/cpu_fallback.py:32-72`) is a
"schema-based ATen fallback": every IR node is executed by calling
``torch.ops.aten.<op>.<overload>`` on CPU tensors, with tensor arguments taken
from ``node.inputs`` in schema order and every other argument taken from
``node.attrs`` by schema name. This module restates that contract:

* Tensor-typed schema arguments consume ``inputs`` in order, unless ``attrs``
  names them (the IR's "scalar binary" form: one input plus ``attrs.other``);
* ``Tensor[]`` arguments consume every remaining input;
* other arguments come from ``attrs`` (dtype strings such as ``"float32"`` or
  ``"torch.float32"`` are mapped to ``torch.dtype``; device, layout and
  memory-format values are host-neutralised), falling back to the schema default,
  or, for a missing ``size``/``shape``, to the node's declared output shape;
* three non-ATen node kinds have fixed meanings: ``<built-in function getitem>``
  selects ``inputs[attrs.index]``; ``wrap_with_set_grad_enabled`` is the rotary
  embedding of HF ``Qwen2RotaryEmbedding.forward`` (fp32 ``inv_freq @ position``,
  ``cat(freqs, freqs)``, ``cos``/``sin`` times ``attention_scaling``, cast to the
  declared output dtype); ``aten._assert_tensor_metadata.default`` does nothing.
"""

from __future__ import annotations

from typing import Any

import torch

TORCH_DTYPES: dict[str, torch.dtype] = {
    "float32": torch.float32, "float": torch.float32, "float16": torch.float16, "half": torch.float16,
    "bfloat16": torch.bfloat16, "float64": torch.float64, "double": torch.float64,
    "int64": torch.int64, "long": torch.int64, "int32": torch.int32, "int": torch.int32,
    "int16": torch.int16, "int8": torch.int8, "uint8": torch.uint8, "bool": torch.bool,
}


def parse_dtype(v: Any) -> torch.dtype | None:
    if v is None or isinstance(v, torch.dtype):
        return v
    s = str(v)
    if s.startswith("torch."):
        s = s[len("torch."):]
    if s not in TORCH_DTYPES:
        raise ValueError(f"unknown dtype attr {v!r}")
    return TORCH_DTYPES[s]


_OP_CACHE: dict[str, Any] = {}


def resolve_aten(op_type: str):
    op = _OP_CACHE.get(op_type)
    if op is not None:
        return op
    parts = op_type.split(".")
    if len(parts) != 3 or parts[0] != "aten":
        raise NotImplementedError(f"not an ATen op: {op_type}")
    op = getattr(getattr(torch.ops.aten, parts[1]), parts[2])
    _OP_CACHE[op_type] = op
    return op


def _is_tensor_type(t: str) -> bool:
    return t in ("Tensor", "Optional[Tensor]")


def _is_tensor_list(t: str) -> bool:
    return t in ("List[Tensor]", "List[Optional[Tensor]]")


def bind_arguments(op, node: dict, tensors: list) -> tuple[list, dict]:
    """Bind IR inputs/attrs to ``op``'s schema; returns (args, kwargs)."""
    attrs = node.get("attrs", {}) or {}
    outs = node.get("outputs", [])
    args: list = []
    kwargs: dict = {}
    pending = list(tensors)
    for a in op._schema.arguments:
        t = str(a.type)
        if _is_tensor_list(t):
            val: Any = pending
            pending = []
        elif _is_tensor_type(t):
            if a.name in attrs:
                val = attrs[a.name]
            elif pending:
                val = pending.pop(0)
            elif a.has_default_value():
                val = a.default_value
            else:
                raise ValueError(f"{node['name']}: missing tensor argument {a.name}")
        elif a.name in attrs:
            val = attrs[a.name]
            if a.name == "dtype":
                val = parse_dtype(val)
            elif a.name in ("device",):
                val = torch.device("cpu")
            elif a.name in ("layout", "memory_format") and isinstance(val, str):
                val = None
        elif a.name in ("size", "shape") and outs:
            val = list(outs[0]["shape"])
        elif a.name == "dtype" and not a.has_default_value() and outs:
            val = parse_dtype(outs[0].get("dtype", "float32"))
        elif a.has_default_value():
            if a.kwarg_only:
                continue
            val = a.default_value
        else:
            raise ValueError(f"{node['name']}: missing argument {a.name} for {node['op_type']}")
        if a.kwarg_only:
            kwargs[a.name] = val
        else:
            args.append(val)
    if node["op_type"] == "aten.full.default" and "dtype" not in kwargs and outs:
        kwargs["dtype"] = parse_dtype(outs[0].get("dtype", "float32"))
    return args, kwargs


def rotary_cos_sin(inv_freq: torch.Tensor, position_ids: torch.Tensor, out_dtype: torch.dtype,
                   attention_scaling: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """HF ``Qwen2RotaryEmbedding.forward`` (transformers ``modeling_qwen2.py:91-102``)."""
    pos = position_ids.reshape(1, -1) if position_ids.dim() == 1 else position_ids
    inv = inv_freq[None, :, None].float().expand(pos.shape[0], -1, 1)
    freqs = (inv @ pos[:, None, :].float()).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos() * attention_scaling
    sin = emb.sin() * attention_scaling
    return cos.to(out_dtype), sin.to(out_dtype)


def run_node(node: dict, env: dict[str, torch.Tensor]) -> None:
    """Execute one IR node, reading tensors from and writing results to ``env``."""
    op_type = node["op_type"]
    ins = [env[i["name"]] for i in node.get("inputs", [])]
    outs = node.get("outputs", [])
    if op_type == "aten._assert_tensor_metadata.default":
        return
    if op_type == "<built-in function getitem>":
        idx = int(node.get("attrs", {}).get("index", 0))
        src = ins[idx] if idx < len(ins) else ins[0]
        if isinstance(src, (tuple, list)):
            src = src[idx]
        env[outs[0]["name"]] = src
        return
    if op_type == "wrap_with_set_grad_enabled":
        scaling = float(node.get("attrs", {}).get("attention_scaling", 1.0))
        dt = parse_dtype(outs[0].get("dtype", "float32"))
        cos, sin = rotary_cos_sin(ins[0], ins[1], dt, scaling)
        env[outs[0]["name"]] = cos
        if len(outs) > 1:
            env[outs[1]["name"]] = sin
        return
    op = resolve_aten(op_type)
    args, kwargs = bind_arguments(op, node, ins)
    res = op(*args, **kwargs)
    if isinstance(res, (tuple, list)):
        for spec, val in zip(outs, res):
            env[spec["name"]] = val
    elif outs:
        env[outs[0]["name"]] = res


class ATenExecutor:
    """Runs a fixed node list on CPU tensors; the counterpart of ``torch_ir.IRExecutor``."""

    def __init__(self, nodes: list[dict], input_names: list[str], output_names: list[str],
                 weights: dict[str, torch.Tensor]):
        self.nodes = nodes
        self.input_names = input_names
        self.output_names = output_names
        self.weights = weights

    def execute(self, inputs: tuple[torch.Tensor, ...]) -> list[torch.Tensor]:
        env: dict[str, Any] = dict(self.weights)
        env.update(zip(self.input_names, inputs))
        with torch.no_grad():
            for node in self.nodes:
                run_node(node, env)
        return [env[n] for n in self.output_names]
