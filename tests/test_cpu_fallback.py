"""CPU fallback and DAG executor on all-CPU plans (cases of the reference's
tests/test_cpu_fallback.py:14-173 and the CS4 flow of tests/test_dag_executor.py)."""

import numpy as np
import pytest
import torch

from npu_compiler import partition
from npu_runtime import DAGExecutor
from npu_runtime.cpu_fallback import execute_cpu_partition, numpy_to_torch, torch_to_numpy


def spec(name, shape, dtype="float32"):
    return {"name": name, "shape": list(shape), "dtype": dtype}


def nd(name, op, ins, outs, attrs=None):
    return {"name": name, "op_type": op, "inputs": ins, "outputs": outs, "attrs": attrs or {}}


def test_bf16_roundtrip_bitexact():
    t = torch.randn(257, dtype=torch.float32).to(torch.bfloat16)
    a = torch_to_numpy(t)
    assert a.dtype == np.uint16
    assert torch.equal(numpy_to_torch(a), t)


def test_fp32_roundtrip():
    a = np.random.default_rng(0).standard_normal((3, 5)).astype(np.float32)
    assert np.array_equal(torch_to_numpy(numpy_to_torch(a)), a)


def test_add_two_plus_three():
    n = nd("add", "aten.add.Tensor", [spec("a", [1]), spec("b", [1])], [spec("c", [1])])
    out = execute_cpu_partition([n], {"a": np.array([2.0], np.float32), "b": np.array([3.0], np.float32)}, {})
    assert out["c"].tolist() == [5.0]


def test_relu_and_neg_relu_chain():
    x = np.array([-1.0, 0.0, 2.5, -3.0], np.float32)
    n1 = nd("neg", "aten.neg.default", [spec("x", [4])], [spec("n", [4])])
    n2 = nd("relu", "aten.relu.default", [spec("n", [4])], [spec("r", [4])])
    out = execute_cpu_partition([n1, n2], {"x": x}, {})
    assert out["n"].tolist() == [1.0, -0.0, -2.5, 3.0]
    assert out["r"].tolist() == [1.0, 0.0, 0.0, 3.0]


def test_mul_by_one_element_tensor_and_scalar_attr():
    n1 = nd("mul", "aten.mul.Tensor", [spec("x", [4]), spec("s", [1])], [spec("y", [4])])
    n2 = nd("mul2", "aten.mul.Tensor", [spec("y", [4])], [spec("z", [4])], {"other": 0.5})
    out = execute_cpu_partition([n1, n2], {"x": np.arange(4, dtype=np.float32), "s": np.array([3.0], np.float32)}, {})
    assert out["y"].tolist() == [0.0, 3.0, 6.0, 9.0]
    assert out["z"].tolist() == [0.0, 1.5, 3.0, 4.5]


def test_weights_resolved_through_mapping():
    n = nd("lin", "aten.linear.default", [spec("x", [1, 4]), spec("p_w", [2, 4])], [spec("y", [1, 2])])
    w = np.arange(8, dtype=np.float32).reshape(2, 4)
    out = execute_cpu_partition([n], {"x": np.ones((1, 4), np.float32)}, {"lin.weight": w}, {"p_w": "lin.weight"})
    assert out["y"].tolist() == [[6.0, 22.0]]


def test_index_copy_kv_update_cpu():
    n = nd("ic", "aten.index_copy.default",
           [spec("cache", [1, 2, 8, 4]), spec("pos", [1], "int64"), spec("src", [1, 2, 1, 4])],
           [spec("out", [1, 2, 8, 4])], {"dim": 2})
    cache = np.random.default_rng(1).standard_normal((1, 2, 8, 4)).astype(np.float32)
    src = np.full((1, 2, 1, 4), 7.0, np.float32)
    out = execute_cpu_partition([n], {"cache": cache, "pos": np.array([5]), "src": src}, {})["out"]
    exp = cache.copy()
    exp[:, :, 5] = 7.0
    assert np.array_equal(out, exp)


def test_dag_executor_all_cpu_mlp_matches_torch():
    from irgen.qwen import QwenConfig, build_mlp_ir
    from irgen.workloads import make_weights, mlp_inputs, to_host

    cfg = QwenConfig(hidden=64, intermediate=128)
    ir = build_mlp_ir(4, cfg)
    w = make_weights(ir, cfg, norm_std=0.02)
    x = mlp_inputs(4, cfg)["x"]
    ex = DAGExecutor(partition(ir, lambda *_: False), backend=None)
    ex.load_weights({k: to_host(v) for k, v in w.items()})
    got = ex.execute({"x": to_host(x)})
    (name,) = got
    # the same model written directly in torch (bf16 on CPU)
    h = x.float()
    n = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    y = w["post_attention_layernorm.weight"] * n
    g = torch.nn.functional.silu(y @ w["mlp.gate_proj.weight"].T) * (y @ w["mlp.up_proj.weight"].T)
    ref = x + g @ w["mlp.down_proj.weight"].T
    assert np.array_equal(got[name], to_host(ref))


def test_transfer_missing_tensor_raises():
    from npu_compiler.partitioner import PartitionPlan, TransferOp

    ex = DAGExecutor(PartitionPlan(steps=[TransferOp(["nope"], "to_cpu")], original_ir={"graph_outputs": []}), None)
    with pytest.raises(RuntimeError, match="nope"):
        ex.execute({})
