"""Pins the oracle's remaining op rules (oracle/numpy_ref.py ``_unary``, ``_bin`` and the
structural ops) one op at a time, the way the reference's fusion tests pin its chains
(tests/test_cuda_fusion.py:31-59: relu/neg/add/mul/silu against numpy closed forms).

Every case evaluates a one-op IR graph with the oracle and with ATen (the CPU
fallback's engine) on asymmetric inputs, and checks a closed form for the op's
meaning. The inputs are chosen so that a plausible mistake fails: swapped operands
of ``sub``/``div`` (a != b), an inverse permutation (dims not self-inverse), the
wrong ``select`` axis (non-square input), ``addmm``'s beta/alpha exchanged
(beta != alpha), a dropped rounding to bf16 (outputs compared bit for bit).
"""

import numpy as np
import pytest
import torch

from oracle import numpy_ref as R


def _graph(op, shapes, attrs=None, dtype="bfloat16", out_dtype=None):
    from irgen.builder import IRBuilder

    b = IRBuilder("one_op")
    ins = [b.input(f"x{i}", s, dtype) for i, s in enumerate(shapes)]
    y = b.op(op, ins, attrs or {}, out_dtype=out_dtype)
    b.output(y)
    return b.to_dict()


def _inputs(shapes, dtype, seed, positive=False):
    from irgen.workloads import to_host

    g = torch.Generator().manual_seed(seed)
    out = {}
    for i, s in enumerate(shapes):
        t = torch.randn(*s, generator=g) * 2
        if positive:
            t = t.abs() + 0.1
        out[f"x{i}"] = to_host(t.to(getattr(torch, dtype)))
    return out


def _aten(ir, inputs):
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    ex = DAGExecutor(partition(ir, lambda *_: False), None)
    ex.load_weights({})
    return ex.execute(inputs)


def _f(a):
    a = np.asarray(a)
    return R.bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float64)


UNARY = {
    "aten.relu.default": lambda x: np.maximum(x, 0),
    "aten.exp.default": np.exp,
    "aten.sigmoid.default": lambda x: 1 / (1 + np.exp(-x)),
    "aten.tanh.default": np.tanh,
    "aten.sqrt.default": np.sqrt,
    "aten.abs.default": np.abs,
    "aten.reciprocal.default": lambda x: 1 / x,
}


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("op", sorted(UNARY))
def test_unary_rule_equals_aten_and_closed_form(op, dtype):
    shapes = [(3, 257)]
    ir = _graph(op, shapes, dtype=dtype)
    x = _inputs(shapes, dtype, seed=len(op), positive=op == "aten.sqrt.default")
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name])
    assert ours.dtype == aten.dtype and ours.shape == aten.shape
    # bf16: bit for bit with ATen except where the two fp32 libm results straddle a bf16 rounding
    # boundary; fp32: numpy's and ATen's vectorised libm differ in the last ulp (rtol 1e-6 below)
    if dtype == "bfloat16":
        assert (ours == aten).mean() >= 0.995
    np.testing.assert_allclose(_f(ours), _f(aten), rtol=1e-6 if dtype == "float32" else 8e-3, atol=1e-30)
    closed = UNARY[op](_f(x["x0"]))
    np.testing.assert_allclose(_f(ours), closed, rtol=8e-3 if dtype == "bfloat16" else 1e-5)


def test_relu_of_negative_is_zero_and_nan_propagates():
    ir = _graph("aten.relu.default", [(4,)], dtype="float32")
    out = R.run_ir(ir, {"x0": np.array([-3.0, -0.0, 2.5, np.nan], np.float32)}, {})[ir["graph_outputs"][0]["name"]]
    assert out[0] == 0 and out[2] == 2.5 and np.isnan(out[3])


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("op,alpha", [("aten.sub.Tensor", 1.0), ("aten.sub.Tensor", 0.5), ("aten.div.Tensor", None)])
def test_binary_rule_equals_aten_and_closed_form(op, alpha, dtype):
    shapes = [(5, 64), (5, 64)]
    attrs = {} if alpha is None else {"alpha": alpha}
    ir = _graph(op, shapes, attrs, dtype=dtype)
    x = _inputs(shapes, dtype, seed=7)
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name])
    assert np.array_equal(ours, aten)
    a, b = _f(x["x0"]), _f(x["x1"])
    closed = a - (alpha or 1.0) * b if op == "aten.sub.Tensor" else a / b
    np.testing.assert_allclose(_f(ours), closed, rtol=8e-3 if dtype == "bfloat16" else 1e-6)
    # the swapped operands give a different answer on these inputs (the check can fail)
    swapped = b - (alpha or 1.0) * a if op == "aten.sub.Tensor" else b / a
    assert not np.allclose(_f(ours), swapped, rtol=1e-2)


@pytest.mark.parametrize("beta,alpha", [(1.0, 1.0), (0.5, 2.0)])
def test_addmm_rule_equals_aten_and_closed_form(beta, alpha):
    shapes = [(6,), (4, 16), (16, 6)]
    ir = _graph("aten.addmm.default", shapes, {"beta": beta, "alpha": alpha}, dtype="float32")
    x = _inputs(shapes, "float32", seed=3)
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name])
    np.testing.assert_allclose(ours, aten, rtol=1e-5, atol=1e-5)
    closed = beta * x["x0"].astype(np.float64) + alpha * (x["x1"].astype(np.float64) @ x["x2"].astype(np.float64))
    np.testing.assert_allclose(ours, closed, rtol=1e-5, atol=1e-5)
    if beta != alpha:   # beta and alpha exchanged would fail
        wrong = alpha * x["x0"] + beta * (x["x1"] @ x["x2"])
        assert not np.allclose(ours, wrong, rtol=1e-3)


@pytest.mark.parametrize("dtype,fill", [("bfloat16", 0.1), ("float32", -2.5), ("int64", 7)])
def test_full_rule_equals_aten(dtype, fill):
    from irgen.builder import IRBuilder

    b = IRBuilder("full")
    y = b.op("aten.full.default", [], {"size": [3, 5], "fill_value": fill,
                                       "dtype": getattr(torch, dtype)})
    b.output(y)
    ir = b.to_dict()
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, {}, {})[name], np.asarray(_aten(ir, {})[name])
    assert ours.shape == (3, 5) and np.array_equal(ours, aten)
    expect = fill if dtype == "int64" else float(torch.tensor(fill, dtype=getattr(torch, dtype)).float())
    assert np.all(_f(ours) == expect)


@pytest.mark.parametrize("dim,index", [(0, 1), (1, 2), (2, -1)])
def test_select_rule_equals_aten_and_indexing(dim, index):
    shapes = [(2, 3, 4)]
    ir = _graph("aten.select.int", shapes, {"dim": dim, "index": index})
    x = _inputs(shapes, "bfloat16", seed=11)
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name])
    assert np.array_equal(np.ascontiguousarray(ours), aten)
    sl = [slice(None)] * 3
    sl[dim] = index
    assert np.array_equal(ours, x["x0"][tuple(sl)])


@pytest.mark.parametrize("dims", [[2, 0, 1], [1, 2, 0], [0, 2, 1]])
def test_permute_rule_equals_aten_and_element_map(dims):
    shapes = [(2, 3, 4)]
    ir = _graph("aten.permute.default", shapes, {"dims": dims})
    x = _inputs(shapes, "bfloat16", seed=13)
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name])
    assert ours.shape == tuple(np.array([2, 3, 4])[dims]) and np.array_equal(np.ascontiguousarray(ours), aten)
    src = x["x0"]
    for idx in np.ndindex(*ours.shape):   # out[i_0, i_1, i_2] = in[i at position dims^-1]
        s = [0, 0, 0]
        for k, d in enumerate(dims):
            s[d] = idx[k]
        assert ours[idx] == src[tuple(s)]


def test_t_rule_equals_aten_and_transpose():
    shapes = [(3, 5)]
    ir = _graph("aten.t.default", shapes)
    x = _inputs(shapes, "bfloat16", seed=17)
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name])
    assert ours.shape == (5, 3) and np.array_equal(np.ascontiguousarray(ours), aten)
    assert all(ours[j, i] == x["x0"][i, j] for i in range(3) for j in range(5))


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("op", ["aten.maximum.default", "aten.minimum.default"])
def test_maximum_minimum_rule_equals_aten_with_nan(op, dtype):
    """torch.maximum / minimum propagate a NaN from either operand (unlike fmax / fmin)."""
    shapes = [(4, 32), (4, 32)]
    ir = _graph(op, shapes, dtype=dtype)
    x = _inputs(shapes, dtype, seed=19)
    nan = np.float32(np.nan) if dtype == "float32" else R.f32_to_bf16_bits(np.array([np.nan], np.float32))[0]
    x["x0"][1, 2] = nan
    x["x1"][2, 3] = nan
    name = ir["graph_outputs"][0]["name"]
    ours, aten = R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name])
    fo, fa = _f(ours), _f(aten)
    assert np.isnan(fo[1, 2]) and np.isnan(fo[2, 3])
    assert np.array_equal(np.isnan(fo), np.isnan(fa)) and np.array_equal(fo[~np.isnan(fo)], fa[~np.isnan(fa)])
    closed = (np.maximum if op == "aten.maximum.default" else np.minimum)(_f(x["x0"]), _f(x["x1"]))
    assert np.array_equal(fo[~np.isnan(fo)], closed[~np.isnan(closed)])


def test_planted_operand_swap_in_sub_is_caught(monkeypatch):
    """A sub rule that computes b - a must break the ATen agreement."""
    shapes = [(5, 64), (5, 64)]
    ir = _graph("aten.sub.Tensor", shapes)
    x = _inputs(shapes, "bfloat16", seed=7)
    orig = R._bin

    def swapped(op, a, b, out_dtype, alpha=1.0):
        return orig(op, b, a, out_dtype, alpha) if op == "sub" else orig(op, a, b, out_dtype, alpha)

    monkeypatch.setattr(R, "_bin", swapped)
    name = ir["graph_outputs"][0]["name"]
    assert not np.array_equal(R.run_ir(ir, x, {})[name], np.asarray(_aten(ir, x)[name]))
