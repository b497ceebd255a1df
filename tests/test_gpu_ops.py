"""The rest of the device op surface, one op at a time, against the CPU fallback (ATen) and
the numpy oracle: generated elementwise chains for every unary and binary op the codegen
table holds, ``aten.full``, NCHW max-pool, standalone batch norm, ``addmm`` and the
``select`` / ``permute`` / ``t`` views materialised by the copy kernel.

Reference counterparts: the fused-chain closed forms of tests/test_cuda_fusion.py:31-59
(chains emitted by cuda_compiler/cuda_codegen.py:47-142) and the special kernels of
cuda_compiler/cuda_templates.py:304-348 (pools, fill), 432-456 (batch norm).
Tolerances: bf16/fp16 outputs within 2e-2 of the output's largest magnitude (the north-star
bound) and, where both sides round the same fp32 value, bit for bit on almost every element;
fills and views bit-exact.
"""

import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


def _f(a):
    from oracle.numpy_ref import bf16_bits_to_f32

    a = np.asarray(a)
    return bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float64)


def _close(got, ref, rtol=2e-2):
    g, r = _f(got), _f(ref)
    assert g.shape == r.shape, (g.shape, r.shape)
    scale = max(float(np.abs(r[np.isfinite(r)]).max(initial=0.0)), 1e-6)
    fin = np.isfinite(r)
    assert np.array_equal(np.isnan(g), np.isnan(r))
    assert np.array_equal(g[np.isinf(r)], r[np.isinf(r)])
    err = float(np.abs(g[fin] - r[fin]).max(initial=0.0))
    assert err <= rtol * scale, f"max abs err {err} vs scale {scale}"


def _run(ir, inputs, backend, weights=None):
    from hip_compiler import compile_subgraph, is_hip_op_supported
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    print(f"[case] {ir['model_name']}", flush=True)
    plan = partition(ir, is_hip_op_supported)
    ex = DAGExecutor(plan, backend, compile_fn=compile_subgraph)
    ex.load_weights(weights or {})
    got = {k: v if isinstance(v, np.ndarray) else v.to_numpy() for k, v in ex.execute(inputs).items()}
    cpu = DAGExecutor(partition(ir, lambda *_: False), None)
    cpu.load_weights(weights or {})
    ref = cpu.execute(inputs)
    from npu_compiler.partitioner import Partition

    parts = [s for s in ex.plan.steps if isinstance(s, Partition)]
    assert parts and all(s.target == "npu" for s in parts)
    kernels = [st.kernel for p in ex.npu_programs.values() for st in p.steps]
    return got, ref, kernels


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


UNARY = ["aten.relu.default", "aten.exp.default", "aten.sigmoid.default", "aten.tanh.default", "aten.sqrt.default",
         "aten.abs.default", "aten.reciprocal.default", "aten.neg.default", "aten.silu.default", "aten.rsqrt.default"]
BINARY = ["aten.sub.Tensor", "aten.div.Tensor", "aten.maximum.default", "aten.minimum.default", "aten.add.Tensor",
          "aten.mul.Tensor"]


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("op", UNARY)
def test_unary_chain_vs_cpu_fallback(backend, op, dtype):
    """op(x0) * x1 + x0: one generated chain of three ops with the op under test first."""
    from irgen.builder import IRBuilder
    from oracle.numpy_ref import run_ir

    shapes = [(33, 65), (33, 65)]
    b = IRBuilder(f"unary_{op}_{dtype}")
    x0, x1 = (b.input(f"x{i}", s, dtype) for i, s in enumerate(shapes))
    y = b.op(op, [x0])
    y = b.op("aten.add.Tensor", [b.op("aten.mul.Tensor", [y, x1]), x0])
    b.output(y)
    ir = b.to_dict()
    x = _inputs(shapes, dtype, seed=len(op), positive=op in ("aten.sqrt.default", "aten.rsqrt.default"))
    got, ref, kernels = _run(ir, x, backend)
    assert any(k.startswith("fused_ew_") for k in kernels)
    (name,) = got
    _close(got[name], ref[name])
    _close(got[name], run_ir(ir, x, {})[name])
    if dtype == "bfloat16":
        assert (np.asarray(got[name]) == np.asarray(ref[name])).mean() >= 0.98


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("op", BINARY)
def test_binary_chain_with_broadcast_vs_cpu_fallback(backend, op, dtype):
    """op(x0, x1[1, N]) then * x0: the second operand broadcast along rows (stride 0). The last
    dimension (96) takes the 8-elements-per-thread form of the generated kernel (16-byte loads of
    x0, one load of x1 per 8 outputs); the unary test's (33, 65) takes the scalar form."""
    from irgen.builder import IRBuilder
    from oracle.numpy_ref import run_ir

    b = IRBuilder(f"binary_{op}_{dtype}")
    x0 = b.input("x0", [17, 96], dtype)
    x1 = b.input("x1", [1, 96], dtype)
    attrs = {"alpha": 0.5} if op == "aten.sub.Tensor" else {}
    y = b.op(op, [x0, x1], attrs)
    y = b.op("aten.mul.Tensor", [y, x0])
    b.output(y)
    ir = b.to_dict()
    x = _inputs([(17, 96), (1, 96)], dtype, seed=len(op) + 1)
    if op in ("aten.maximum.default", "aten.minimum.default"):   # NaN in either operand propagates
        nan = np.array(np.nan, np.float32)
        nanv = nan if dtype == "float32" else np.asarray(torch.tensor(float("nan")).bfloat16().view(torch.uint16))
        x["x0"][3, 5] = nanv
        x["x1"][0, 9] = nanv
    got, ref, kernels = _run(ir, x, backend)
    assert any(k.startswith("fused_ew_") for k in kernels)
    (name,) = got
    _close(got[name], ref[name])
    _close(got[name], run_ir(ir, x, {})[name])
    if dtype == "bfloat16":
        assert (np.asarray(got[name]) == np.asarray(ref[name])).mean() >= 0.98


@pytest.mark.parametrize("dtype,fill", [("bfloat16", 0.1), ("float32", -2.5), ("int64", 7), ("float16", 3.0)])
def test_full_is_bit_exact(backend, dtype, fill):
    from irgen.builder import IRBuilder

    b = IRBuilder(f"full_{dtype}")
    x = b.input("x0", [3, 700], "float32")
    y = b.op("aten.full.default", [], {"size": [3, 700], "fill_value": fill, "dtype": getattr(torch, dtype)})
    b.output(y, b.op("aten.relu.default", [x]))
    ir = b.to_dict()
    xin = _inputs([(3, 700)], "float32", seed=5)
    got, ref, kernels = _run(ir, xin, backend)
    assert "k_fill" in kernels
    name = ir["graph_outputs"][0]["name"]
    assert np.array_equal(np.asarray(got[name]), np.asarray(ref[name]))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("k,s,p", [(3, 2, 1), (2, 2, 0), (3, 1, 1)])
def test_maxpool_nchw_is_bit_exact(backend, dtype, k, s, p):
    """NCHW max-pool on a graph input (the channels-last kernel is taken only after an NHWC conv):
    a max of stored values, so bit-exact with the CPU path, including padded borders."""
    from irgen.builder import IRBuilder

    b = IRBuilder(f"maxpool_{dtype}_{k}{s}{p}")
    x = b.input("x0", [2, 5, 13, 11], dtype)
    y = b.op("aten.max_pool2d.default", [x], {"kernel_size": [k, k], "stride": [s, s], "padding": [p, p]})
    b.output(y)
    ir = b.to_dict()
    xin = _inputs([(2, 5, 13, 11)], dtype, seed=k * 10 + s)
    got, ref, kernels = _run(ir, xin, backend)
    assert "k_maxpool2d" in kernels
    (name,) = got
    assert np.array_equal(np.asarray(got[name]), np.asarray(ref[name]))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_batch_norm_standalone_vs_cpu_fallback(backend, dtype):
    """Inference batch norm with no convolution before it (k_batchnorm), vs ATen and the closed
    form (x - mean) / sqrt(var + eps) * w + b."""
    from irgen.builder import IRBuilder
    from irgen.workloads import to_host

    C = 6
    b = IRBuilder(f"bn_{dtype}")
    x = b.input("x0", [2, C, 7, 5], dtype)
    ps = [b.weight(f"bn.{n}", [C], dtype, buffer=n in ("running_mean", "running_var"))
          for n in ("weight", "bias", "running_mean", "running_var")]
    y = b.op("aten.batch_norm.default", [x, *ps], {"training": False, "momentum": 0.1, "eps": 1e-5,
                                                    "cudnn_enabled": False})
    b.output(y)
    ir = b.to_dict()
    g = torch.Generator().manual_seed(3)
    td = getattr(torch, dtype)
    w = {"bn.weight": 1 + 0.3 * torch.randn(C, generator=g), "bn.bias": 0.2 * torch.randn(C, generator=g),
         "bn.running_mean": 0.1 * torch.randn(C, generator=g), "bn.running_var": 0.5 + torch.rand(C, generator=g)}
    w = {k: to_host(v.to(td)) for k, v in w.items()}
    xin = _inputs([(2, C, 7, 5)], dtype, seed=4)
    got, ref, kernels = _run(ir, xin, backend, w)
    assert "k_batchnorm" in kernels
    (name,) = got
    _close(got[name], ref[name])
    xf = _f(xin["x0"]) if dtype != "float16" else xin["x0"].astype(np.float64)
    pf = {k: (_f(v) if dtype != "float16" else v.astype(np.float64)).reshape(1, C, 1, 1) for k, v in w.items()}
    closed = (xf - pf["bn.running_mean"]) / np.sqrt(pf["bn.running_var"] + 1e-5) * pf["bn.weight"] + pf["bn.bias"]
    gf = _f(got[name]) if dtype != "float16" else np.asarray(got[name]).astype(np.float64)
    _close(gf, closed)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_addmm_vs_cpu_fallback_and_closed_form(backend, dtype):
    from irgen.builder import IRBuilder

    b = IRBuilder(f"addmm_{dtype}")
    bias = b.input("x0", [40], dtype)
    a = b.input("x1", [24, 64], dtype)
    m = b.input("x2", [64, 40], dtype)
    y = b.op("aten.addmm.default", [bias, a, m], {"beta": 0.5, "alpha": 2.0})
    b.output(y)
    ir = b.to_dict()
    xin = _inputs([(40,), (24, 64), (64, 40)], dtype, seed=9)
    got, ref, _ = _run(ir, xin, backend)
    (name,) = got
    _close(got[name], ref[name])
    closed = 0.5 * _f(xin["x0"]) + 2.0 * (_f(xin["x1"]) @ _f(xin["x2"]))
    _close(got[name], closed)


@pytest.mark.parametrize("view", ["select", "permute", "t"])
def test_views_materialised_bit_exact(backend, view):
    """select / permute / t as graph outputs: the copy kernel writes the strided view contiguously."""
    from irgen.builder import IRBuilder

    b = IRBuilder(f"view_{view}")
    if view == "t":
        x = b.input("x0", [37, 53], "bfloat16")
        y = b.op("aten.t.default", [x])
        shape = (37, 53)
    else:
        x = b.input("x0", [3, 29, 41], "bfloat16")
        shape = (3, 29, 41)
        y = (b.op("aten.select.int", [x], {"dim": 1, "index": 7}) if view == "select"
             else b.op("aten.permute.default", [x], {"dims": [2, 0, 1]}))
    b.output(y)
    ir = b.to_dict()
    xin = _inputs([shape], "bfloat16", seed=21)
    got, ref, _ = _run(ir, xin, backend)
    (name,) = got
    assert np.array_equal(np.ascontiguousarray(got[name]), np.ascontiguousarray(ref[name]))


@pytest.mark.parametrize("case", ["bias_r8", "resid_r8", "bias_r16", "silu", "silu_bias", "resid_m24", "silu_m24",
                                  "wide_m33", "wide_m64_bias", "wide_m65", "wide_m128_k2048", "wide_m100_bias",
                                  "wide_m100_mt8"])
def test_skinny_linear_vs_cpu_fallback(backend, case, monkeypatch):
    """The skinny MFMA kernels (16-32 activation rows, gemv.hip k_skinny_*): a linear with bias,
    a linear + residual add, and SiLU(gate) * up over two weights, against the CPU fallback;
    the output tile widths (8 / 16 rows, the short-N variant), one and two 16-row tiles, a
    long K and an N that is not a multiple of the tile. ``wide_*``: SiLU(gate) * up over 33-128
    rows (k_wide_silu_mt4 / _mt8: rows past M repeat the last, N not a multiple of the
    workgroup's 40 pairs nor of 8, biases, a K of 32 stages)."""
    from irgen.builder import IRBuilder
    from irgen.qwen import linear

    M, N, K, kind = {"bias_r8": (16, 1000, 768, "bias"), "resid_r8": (16, 1536, 8960, "resid"),
                     "bias_r16": (16, 4104, 512, "bias"), "silu": (16, 2056, 1536, "silu"),
                     "silu_bias": (16, 1032, 512, "silu_bias"), "resid_m24": (24, 1536, 2048, "resid"),
                     "silu_m24": (24, 2048, 1536, "silu"), "wide_m33": (33, 1004, 1536, "silu"),
                     "wide_m64_bias": (64, 1032, 512, "silu_bias"), "wide_m65": (65, 2056, 1536, "silu"),
                     "wide_m128_k2048": (128, 8960, 2048, "silu"), "wide_m100_bias": (100, 1004, 512, "silu_bias"),
                     "wide_m100_mt8": (100, 2056, 1536, "silu_bias")}[case]
    if case.endswith("_mt8"):   # one 128-row workgroup per group of weight tiles (k_wide_silu_mt8)
        from hip_compiler import subgraph_analyzer
        monkeypatch.setattr(subgraph_analyzer, "WIDE_HALVES", False)
    dt = "bfloat16"
    b = IRBuilder(f"skinny_{case}")
    x = b.input("x0", [M, K], dt)
    w = b.input("x1", [N, K], dt)
    shapes = [(M, K), (N, K)]
    if kind == "bias":
        bias = b.input("x2", [N], dt)
        shapes.append((N,))
        y = linear(b, x, w, bias)
    elif kind == "resid":
        r = b.input("x2", [M, N], dt)
        shapes.append((M, N))
        y = b.op("aten.add.Tensor", [r, linear(b, x, w)])
    else:
        w2 = b.input("x2", [N, K], dt)
        shapes.append((N, K))
        bias = bias2 = None
        if kind == "silu_bias":
            bias, bias2 = b.input("x3", [N], dt), b.input("x4", [N], dt)
            shapes += [(N,), (N,)]
        y = b.op("aten.mul.Tensor", [b.op("aten.silu.default", [linear(b, x, w, bias)]), linear(b, x, w2, bias2)])
    b.output(y)
    ir = b.to_dict()
    xin = _inputs(shapes, dt, seed=21)
    for k in ("x1", "x2", "x3", "x4"):   # weights of a trained scale: sums over K stay O(1)
        if k in xin and xin[k].ndim == 2 and xin[k].shape[1] == K:
            xin[k] = (torch.from_numpy(_f(xin[k]) / np.sqrt(K)).to(torch.bfloat16).view(torch.int16).numpy()
                      .view(np.uint16))
    got, ref, kernels = _run(ir, xin, backend)
    assert any(k.startswith("k_wide_silu_mt" if case.startswith("wide") else "k_skinny_") for k in kernels), kernels
    if case.endswith("_mt8"):
        assert "k_wide_silu_mt8" in kernels, kernels
    (name,) = got
    _close(got[name], ref[name])
