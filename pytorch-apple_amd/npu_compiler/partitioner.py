"""Graph partitioner: split an IR graph into device and CPU segments.

Same API and result structure as the reference (`npu_compiler/partitioner.py:15-143`):

* every node is tagged ``"npu"`` when ``is_supported_fn(op_type, attrs)`` is true,
  else ``"cpu"``; nodes are assumed to be in topological order already;
* maximal runs of equally tagged consecutive nodes form ``Partition``s, numbered
  from 0 in order;
* a partition's ``input_names`` are the (sorted) tensors its nodes read but do
  not produce; its ``output_names`` are the (sorted) tensors it produces that a
  later-or-earlier *other* partition reads, plus the graph outputs it produces;
* before each partition whose target differs from its predecessor's, a
  ``TransferOp`` moves the (sorted) inputs that some *preceding* partition
  produced, towards the new target; no transfer is emitted when that set is empty.

The device target keeps the reference's name ``"npu"`` so that callers written
against the reference keep working; here it means the MI355X.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Literal

Target = Literal["npu", "cpu"]


@dataclass
class Partition:
    partition_id: int
    target: Target
    nodes: list[dict]
    input_names: list[str] = field(default_factory=list)
    output_names: list[str] = field(default_factory=list)


@dataclass
class TransferOp:
    tensor_names: list[str]
    direction: Literal["to_cpu", "to_npu"]


@dataclass
class PartitionPlan:
    steps: list[Partition | TransferOp]
    original_ir: dict


def _group_runs(nodes: list[dict], is_supported_fn) -> list[Partition]:
    parts: list[Partition] = []
    for node in nodes:
        tgt: Target = "npu" if is_supported_fn(node["op_type"], node.get("attrs")) else "cpu"
        if parts and parts[-1].target == tgt:
            parts[-1].nodes.append(node)
        else:
            parts.append(Partition(partition_id=len(parts), target=tgt, nodes=[node]))
    return parts


def partition(ir_dict: dict, is_supported_fn: Callable[[str, dict | None], bool]) -> PartitionPlan:
    """Partition ``ir_dict`` by ``is_supported_fn`` (`partitioner.py:42-88`)."""
    nodes = ir_dict.get("nodes", [])
    if not nodes:
        return PartitionPlan(steps=[], original_ir=ir_dict)

    parts = _group_runs(nodes, is_supported_fn)

    owner: dict[str, int] = {}
    made: list[set[str]] = []
    for p in parts:
        names = {o["name"] for n in p.nodes for o in n.get("outputs", [])}
        made.append(names)
        for nm in names:
            owner[nm] = p.partition_id

    graph_outs = {o["name"] for o in ir_dict.get("graph_outputs", [])}
    exported: list[set[str]] = [set() for _ in parts]
    for p in parts:
        reads = {i["name"] for n in p.nodes for i in n.get("inputs", [])}
        p.input_names = sorted(reads - made[p.partition_id])
        for nm in p.input_names:
            src = owner.get(nm)
            if src is not None and src != p.partition_id:
                exported[src].add(nm)
    for p in parts:
        p.output_names = sorted(exported[p.partition_id] | (made[p.partition_id] & graph_outs))

    steps: list[Partition | TransferOp] = []
    earlier: set[str] = set()
    for i, p in enumerate(parts):
        if i > 0 and parts[i - 1].target != p.target:
            crossing = sorted(nm for nm in p.input_names if nm in earlier)
            if crossing:
                steps.append(TransferOp(tensor_names=crossing,
                                        direction="to_cpu" if p.target == "cpu" else "to_npu"))
        steps.append(p)
        earlier |= made[p.partition_id]
    return PartitionPlan(steps=steps, original_ir=ir_dict)
