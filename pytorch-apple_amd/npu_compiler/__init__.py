"""IR model and partitioner shared by every backend.

``compile`` is the default ``compile_fn`` of ``DAGExecutor`` when none is given;
in the reference it is the Metal compiler. Here the only device compiler is the
HIP one, so the default is ``hip_compiler.compile_subgraph``.
"""

from npu_compiler.ir_reader import IRGraph, OpNode, TensorSpec, load_ir, load_ir_from_dict
from npu_compiler.partitioner import Partition, PartitionPlan, TransferOp, partition


def compile(ir_dict: dict):  # noqa: A001 - name kept from the reference API
    from hip_compiler import compile_subgraph

    return compile_subgraph(ir_dict)


__all__ = [
    "IRGraph", "OpNode", "TensorSpec", "load_ir", "load_ir_from_dict",
    "Partition", "PartitionPlan", "TransferOp", "partition", "compile",
]
