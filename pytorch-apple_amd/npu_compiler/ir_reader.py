"""IR JSON model: tensor specs, op nodes and the graph container.

Same schema and loader API as the reference (`npu_compiler/ir_reader.py:9-94`):
a graph is ``{model_name, graph_inputs[], graph_outputs[], weights[],
weight_name_mapping{}, nodes[], constants{}}``; a tensor is
``{name, shape, dtype, alloc_shape?, transform_steps?, producer_node?,
producer_output_idx?}``; a node is ``{name, op_type, inputs[], outputs[], attrs{}}``.
Tensor arguments of an ATen op sit in ``inputs`` in schema order, the other
arguments in ``attrs`` under their schema names.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field


@dataclass
class TensorSpec:
    name: str
    shape: list[int]
    dtype: str = "float32"
    alloc_shape: list[int] | None = None
    transform_steps: list[dict] | None = None
    producer_node: str | None = None
    producer_output_idx: int = 0


@dataclass
class OpNode:
    name: str
    op_type: str
    inputs: list[TensorSpec]
    outputs: list[TensorSpec]
    attrs: dict = field(default_factory=dict)


@dataclass
class IRGraph:
    model_name: str
    graph_inputs: list[TensorSpec]
    graph_outputs: list[TensorSpec]
    weights: list[TensorSpec]
    weight_name_mapping: dict[str, str]
    nodes: list[OpNode]
    constants: dict = field(default_factory=dict)

    def get_node_by_name(self, name: str) -> OpNode | None:
        return next((n for n in self.nodes if n.name == name), None)


def _spec(d: dict) -> TensorSpec:
    return TensorSpec(
        name=d["name"],
        shape=list(d["shape"]),
        dtype=d.get("dtype", "float32"),
        alloc_shape=d.get("alloc_shape"),
        transform_steps=d.get("transform_steps"),
        producer_node=d.get("producer_node"),
        producer_output_idx=d.get("producer_output_idx", 0),
    )


def _node(d: dict) -> OpNode:
    return OpNode(
        name=d["name"],
        op_type=d["op_type"],
        inputs=[_spec(t) for t in d["inputs"]],
        outputs=[_spec(t) for t in d["outputs"]],
        attrs=dict(d.get("attrs", {})),
    )


def load_ir_from_dict(data: dict) -> IRGraph:
    """Build an IRGraph from an in-memory IR dict (`ir_reader.py:84-94`)."""
    return IRGraph(
        model_name=data.get("model_name", "unknown"),
        graph_inputs=[_spec(t) for t in data["graph_inputs"]],
        graph_outputs=[_spec(t) for t in data["graph_outputs"]],
        weights=[_spec(t) for t in data["weights"]],
        weight_name_mapping=dict(data.get("weight_name_mapping", {})),
        nodes=[_node(n) for n in data["nodes"]],
        constants=dict(data.get("constants", {})),
    )


def load_ir(path: str) -> IRGraph:
    """Load an IR JSON file (`ir_reader.py:68-81`)."""
    with open(path) as f:
        return load_ir_from_dict(json.load(f))
