"""Partition structure KATs (cases of the reference's tests/test_partitioner.py:34-203)."""

from npu_compiler.partitioner import Partition, TransferOp, partition


def node(name, op, ins, outs):
    return {"name": name, "op_type": op,
            "inputs": [{"name": n, "shape": [1, 64], "dtype": "float32"} for n in ins],
            "outputs": [{"name": n, "shape": [1, 64], "dtype": "float32", "producer_node": name,
                         "producer_output_idx": i} for i, n in enumerate(outs)], "attrs": {}}


def ir_of(nodes, gi=("x",), go=None):
    go = go if go is not None else [o["name"] for o in nodes[-1]["outputs"]] if nodes else []
    return {"model_name": "t", "graph_inputs": [{"name": n, "shape": [1, 64], "dtype": "float32"} for n in gi],
            "graph_outputs": [{"name": n, "shape": [1, 64], "dtype": "float32"} for n in go],
            "weights": [], "weight_name_mapping": {}, "nodes": nodes}


def only(ops):
    return lambda op, _a=None: op in ops


def test_all_supported_single_partition():
    plan = partition(ir_of([node("conv", "aten.conv2d.default", ["x"], ["c"]),
                            node("relu", "aten.relu.default", ["c"], ["r"])]), lambda *_: True)
    assert len(plan.steps) == 1 and plan.steps[0].target == "npu" and len(plan.steps[0].nodes) == 2


def test_empty_graph():
    assert partition(ir_of([], go=[]), lambda *_: True).steps == []


def test_all_unsupported_single_cpu_partition():
    plan = partition(ir_of([node("g", "aten.gelu.default", ["x"], ["a"]),
                            node("t", "aten.tanh.default", ["a"], ["b"])]), lambda *_: False)
    assert len(plan.steps) == 1 and plan.steps[0].target == "cpu"


def test_npu_cpu_npu_split():
    nodes = [node("conv", "aten.conv2d.default", ["x"], ["conv_out"]),
             node("relu", "aten.relu.default", ["conv_out"], ["relu_out"]),
             node("gelu", "aten.gelu.default", ["relu_out"], ["gelu_out"]),
             node("linear", "aten.linear.default", ["gelu_out"], ["linear_out"])]
    plan = partition(ir_of(nodes), only({"aten.conv2d.default", "aten.relu.default", "aten.linear.default"}))
    parts = [s for s in plan.steps if isinstance(s, Partition)]
    xfers = [s for s in plan.steps if isinstance(s, TransferOp)]
    assert [p.target for p in parts] == ["npu", "cpu", "npu"]
    assert [len(p.nodes) for p in parts] == [2, 1, 1]
    assert [t.direction for t in xfers] == ["to_cpu", "to_npu"]
    assert [type(s).__name__ for s in plan.steps] == ["Partition", "TransferOp", "Partition", "TransferOp",
                                                       "Partition"]


def test_transfer_tensor_names_and_boundary_io():
    nodes = [node("conv", "aten.conv2d.default", ["x"], ["conv_out"]),
             node("gelu", "aten.gelu.default", ["conv_out"], ["gelu_out"]),
             node("relu", "aten.relu.default", ["gelu_out"], ["relu_out"])]
    plan = partition(ir_of(nodes), only({"aten.conv2d.default", "aten.relu.default"}))
    xfers = [s for s in plan.steps if isinstance(s, TransferOp)]
    parts = [s for s in plan.steps if isinstance(s, Partition)]
    assert xfers[0].tensor_names == ["conv_out"] and xfers[0].direction == "to_cpu"
    assert xfers[1].tensor_names == ["gelu_out"] and xfers[1].direction == "to_npu"
    assert parts[0].output_names == ["conv_out"]
    assert parts[1].input_names == ["conv_out"] and parts[1].output_names == ["gelu_out"]
    assert parts[2].output_names == ["relu_out"]
    assert parts[0].input_names == ["x"]


def test_consecutive_unsupported_grouped():
    nodes = [node("conv", "aten.conv2d.default", ["x"], ["a"]), node("gelu", "aten.gelu.default", ["a"], ["b"]),
             node("tanh", "aten.tanh.default", ["b"], ["c"]), node("relu", "aten.relu.default", ["c"], ["d"])]
    parts = [s for s in partition(ir_of(nodes), only({"aten.conv2d.default", "aten.relu.default"})).steps
             if isinstance(s, Partition)]
    assert len(parts) == 3 and parts[1].target == "cpu" and len(parts[1].nodes) == 2


def test_skip_connection_crosses_two_boundaries():
    # x -> conv -> gelu(cpu) -> add(conv_out, gelu_out) on npu: conv_out is exported by p0 and read by p2
    nodes = [node("conv", "aten.conv2d.default", ["x"], ["c"]), node("gelu", "aten.gelu.default", ["c"], ["g"]),
             node("add", "aten.add.Tensor", ["c", "g"], ["o"])]
    plan = partition(ir_of(nodes), only({"aten.conv2d.default", "aten.add.Tensor"}))
    parts = [s for s in plan.steps if isinstance(s, Partition)]
    xfers = [s for s in plan.steps if isinstance(s, TransferOp)]
    assert parts[0].output_names == ["c"]
    assert parts[2].input_names == ["c", "g"]
    assert xfers[1].tensor_names == ["c", "g"]


def test_supported_fn_receives_attrs():
    seen = []
    n = node("m", "aten.mean.dim", ["x"], ["y"])
    n["attrs"] = {"dim": [1]}
    partition(ir_of([n]), lambda op, attrs=None: seen.append((op, attrs)) or True)
    assert seen == [("aten.mean.dim", {"dim": [1]})]
