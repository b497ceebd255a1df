"""HIP source generation for fused elementwise chains.

Counterpart of the reference's ``generate_fused_kernel`` (`cuda_compiler/cuda_codegen.py:47-142`),
which emits one ``__half`` CUDA kernel per chain that reads every operand at the
output index (no broadcasting, defect D3). Here a chain is compiled for its exact
operand layouts: each external operand is read through its own strides relative
to the (contiguous) output shape, stride 0 expressing broadcast, so RoPE's
``q * cos[1,1,1,128]`` or a ``[T,1]`` scale need no materialised expand. Values
are carried in fp32 (or int64 for integer results) and rounded to the IR dtype of
every node's output, which are ATen's rounding points on the CPU. Shapes and
strides are baked into the source as constants, so kernels are specialised and
identical layers share one compiled kernel through the source hash.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

from hip_compiler.program import DTYPE_CODE, FLOAT_DTYPES, TView

MAX_CHAIN_INPUTS = 8

_UNARY_F = {
    "aten.relu.default": "(({a}) != ({a}) ? ({a}) : fmaxf(({a}), 0.f))",
    "aten.relu_.default": "(({a}) != ({a}) ? ({a}) : fmaxf(({a}), 0.f))",
    "aten.silu.default": "(({a}) / (1.f + expf(-({a}))))",
    "aten.sigmoid.default": "(1.f / (1.f + expf(-({a}))))",
    "aten.neg.default": "(-({a}))",
    "aten.rsqrt.default": "(1.f / sqrtf({a}))",
    "aten.sqrt.default": "sqrtf({a})",
    "aten.cos.default": "cosf({a})",
    "aten.sin.default": "sinf({a})",
    "aten.exp.default": "expf({a})",
    "aten.tanh.default": "tanhf({a})",
    "aten.abs.default": "fabsf({a})",
    "aten.reciprocal.default": "(1.f / ({a}))",
    "aten.to.dtype": "({a})",
    "aten._to_copy.default": "({a})",
    "aten.clone.default": "({a})",
    "aten.alias.default": "({a})",
}
_UNARY_I = {"aten.neg.default": "(-({a}))", "aten.to.dtype": "({a})", "aten._to_copy.default": "({a})",
            "aten.abs.default": "llabs({a})", "aten.clone.default": "({a})"}
_BINARY = {
    "aten.add.Tensor": "(({a}) + ({alpha}) * ({b}))",
    "aten.add_.Tensor": "(({a}) + ({alpha}) * ({b}))",
    "aten.sub.Tensor": "(({a}) - ({alpha}) * ({b}))",
    "aten.mul.Tensor": "(({a}) * ({b}))",
    "aten.mul_.Tensor": "(({a}) * ({b}))",
    "aten.div.Tensor": "(({a}) / ({b}))",
    # NaN in either operand gives NaN, as torch.maximum / minimum (fmaxf alone would drop it)
    "aten.maximum.default": "(({a}) != ({a}) ? ({a}) : (({b}) != ({b}) ? ({b}) : fmaxf(({a}), ({b}))))",
    "aten.minimum.default": "(({a}) != ({a}) ? ({a}) : (({b}) != ({b}) ? ({b}) : fminf(({a}), ({b}))))",
}
EW_OPS = set(_UNARY_F) | set(_BINARY) | {"aten.pow.Tensor_Scalar"}


@dataclass
class ChainOp:
    op_type: str
    operands: list          # ("ext", k) | ("val", j) | ("scalar", value)
    out_dtype: str
    attrs: dict = field(default_factory=dict)


def _lit(x: float) -> str:
    if x != x:
        return "__builtin_nanf(\"\")"
    if x in (float("inf"), float("-inf")):
        return "INFINITY" if x > 0 else "(-INFINITY)"
    return f"(float)({float(x)!r})"


VEC = 8   # elements per thread on the vector path (16 bytes of a 16-bit dtype)


def vector_ok(ext: list[TView], out_shape: tuple[int, ...], out_dtype: str) -> bool:
    """Whether a chain can run 8 consecutive output elements per thread with 16-byte accesses:
    float operands and result, the last dimension a multiple of 8, and every operand either
    contiguous along it (stride 1, its 8-element groups 16-byte aligned for 16-bit dtypes and
    32-byte aligned for fp32: offset and outer strides multiples of 8) or broadcast along it
    (stride 0: one load serves the 8 elements)."""
    if not out_shape or out_dtype not in FLOAT_DTYPES or out_shape[-1] % VEC:
        return False
    for v in ext:
        if v.dtype not in FLOAT_DTYPES:
            return False
        if not v.shape:
            continue
        st = list(v.strides)
        if st[-1] == 0:
            continue
        if st[-1] != 1 or v.offset % VEC or any(s % VEC for s in st[:-1]):
            return False
    return True


def generate_chain(ops: list[ChainOp], ext: list[TView], out_shape: tuple[int, ...], out_dtype: str) -> tuple[str, str]:
    """Return ``(kernel_name, source)`` computing ``ops`` over ``out_shape``.

    Where ``vector_ok`` holds, thread g computes output elements 8g..8g+7 (one row of the last
    dimension, so they share every outer coordinate): 16-byte loads of each contiguous operand,
    one load of each operand broadcast along the last dimension, the chain evaluated per
    element at the same rounding points, and 16-byte stores (``n`` is then the number of
    8-element groups). Otherwise one element per thread."""
    if len(ext) > MAX_CHAIN_INPUTS:
        raise ValueError("too many chain inputs")
    vec = vector_ok(ext, out_shape, out_dtype)
    nd = max(len(out_shape), 1)
    shape = list(out_shape) if out_shape else [1]
    body: list[str] = []
    # coordinates of element i of the contiguous output
    body.append(f"    long long r_ = i{' * 8' if vec else ''};")
    for d in range(nd - 1, -1, -1):
        if shape[d] == 1:
            body.append(f"    const long long c{d} = 0;")
        elif d == 0:
            body.append(f"    const long long c{d} = r_;")
        else:
            body.append(f"    const long long c{d} = r_ % {shape[d]}LL; r_ /= {shape[d]}LL;")
    for k, v in enumerate(ext):
        strides = list(v.strides) if v.shape else [0]
        pad = nd - len(strides)
        strides = [0] * pad + strides
        terms = [f"c{d} * {strides[d]}LL" for d in range(nd) if strides[d] != 0 and shape[d] != 1]
        off = " + ".join(terms) if terms else "0LL"
        dt = v.dtype
        if vec:
            wide = v.shape and strides[-1] == 1
            fn = "ld8_f" if wide else "ld1x8_f"
            body.append(f"    float e{k}v[8]; {fn}(a.in[{k}], {off}, {DTYPE_CODE[dt]}, e{k}v);")
        elif dt in FLOAT_DTYPES:
            body.append(f"    const float e{k} = ld_f(a.in[{k}], {off}, {DTYPE_CODE[dt]});")
        else:
            body.append(f"    const long long e{k} = ld_i(a.in[{k}], {off}, {DTYPE_CODE[dt]});")
    if vec:
        body.append("    float res_[8];")
        body.append("#pragma unroll")
        body.append("    for (int j_ = 0; j_ < 8; ++j_) {")
        for k in range(len(ext)):
            body.append(f"    const float e{k} = e{k}v[j_];")
    vals: list[tuple[str, str]] = []     # (expr var, dtype)

    def operand(o, want_float: bool) -> str:
        kind, x = o
        if kind == "ext":
            name, dt = f"e{x}", ext[x].dtype
        elif kind == "val":
            name, dt = vals[x]
        else:
            return _lit(x) if want_float else f"(long long)({x!r})"
        if want_float and dt not in FLOAT_DTYPES:
            return f"(float){name}"
        return name

    for j, op in enumerate(ops):
        fl = op.out_dtype in FLOAT_DTYPES
        ctype = "float" if fl else "long long"
        if op.op_type in _BINARY:
            a = operand(op.operands[0], fl)
            b = operand(op.operands[1], fl)
            alpha = op.attrs.get("alpha", 1)
            expr = _BINARY[op.op_type].format(a=a, b=b, alpha=_lit(alpha) if fl else f"{int(alpha)}LL")
            if op.op_type == "aten.div.Tensor" and not fl:
                raise ValueError("integer division is not fused")
        elif op.op_type == "aten.pow.Tensor_Scalar":
            a = operand(op.operands[0], True)
            e = float(op.attrs.get("exponent", 2.0))
            if e == 2.0:
                expr = f"(({a}) * ({a}))"
            elif e == 1.0:
                expr = f"({a})"
            elif e == 0.5:
                expr = f"sqrtf({a})"
            elif e == -1.0:
                expr = f"(1.f / ({a}))"
            else:
                expr = f"powf(({a}), {_lit(e)})"
        else:
            table = _UNARY_F if fl else _UNARY_I
            if op.op_type not in table:
                raise ValueError(f"op {op.op_type} not fusable for dtype {op.out_dtype}")
            expr = table[op.op_type].format(a=operand(op.operands[0], fl))
        if fl and op.out_dtype in ("bfloat16", "float16"):
            expr = f"round_to({expr}, {DTYPE_CODE[op.out_dtype]})"
        body.append(f"    const {ctype} t{j} = {expr};")
        vals.append((f"t{j}", op.out_dtype))
    last, ldt = vals[-1]
    if vec:
        body.append(f"    res_[j_] = {last if ldt in FLOAT_DTYPES else f'(float){last}'};")
        body.append("    }")
        body.append(f"    st8_f(a.out, i * 8, {DTYPE_CODE[out_dtype]}, res_);")
    elif out_dtype in FLOAT_DTYPES:
        src_last = last if ldt in FLOAT_DTYPES else f"(float){last}"
        body.append(f"    st_f(a.out, i, {DTYPE_CODE[out_dtype]}, {src_last});")
    elif out_dtype == "int64":
        body.append(f"    ((long long*)a.out)[i] = (long long)({last});")
    elif out_dtype == "int32":
        body.append(f"    ((int*)a.out)[i] = (int)({last});")
    else:
        body.append(f"    ((unsigned char*)a.out)[i] = (unsigned char)(({last}) != 0);")
    text = "\n".join(body)
    h = hashlib.sha1(text.encode()).hexdigest()[:16]
    name = f"fused_ew_{h}"
    src = (f'#include "common.h"\n'
           f'extern "C" __global__ void __launch_bounds__(256) {name}(const FusedArgs a) {{\n'
           f"  const long long stride_ = (long long)gridDim.x * blockDim.x;\n"
           f"  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride_) {{\n"
           f"{text}\n"
           f"  }}\n}}\n")
    return name, src
