"""Op categories of the HIP subgraph compiler.

Same categories as the reference (`cuda_compiler/op_classify.py:17-79`): ANCHOR
ops (GEMM-shaped, fusion barriers), ELEMENTWISE ops (chained into one generated
kernel), REDUCTION ops (dedicated kernels), SHAPE_ALIAS ops (views, no launch),
SPECIAL ops (hand-written kernels) and NOOPs. One difference: ``aten.to.dtype``
is ELEMENTWISE here because dtypes are kept exact (a bf16→fp32 cast is real work
when the model is bf16), and it degrades to an alias when the dtype is unchanged.
"""

from __future__ import annotations

from enum import Enum, auto

from hip_compiler.codegen import EW_OPS


class OpCategory(Enum):
    ANCHOR_BLAS = auto()
    ELEMENTWISE = auto()
    REDUCTION = auto()
    SHAPE_ALIAS = auto()
    SPECIAL = auto()
    NOOP = auto()


_TABLE: dict[str, OpCategory] = {
    "aten.matmul.default": OpCategory.ANCHOR_BLAS,
    "aten.linear.default": OpCategory.ANCHOR_BLAS,
    "aten.addmm.default": OpCategory.ANCHOR_BLAS,
    "aten.mm.default": OpCategory.ANCHOR_BLAS,
    "aten.bmm.default": OpCategory.ANCHOR_BLAS,
    "aten.conv2d.default": OpCategory.ANCHOR_BLAS,
    "aten.batch_norm.default": OpCategory.REDUCTION,
    "aten.max_pool2d.default": OpCategory.REDUCTION,
    "aten.adaptive_avg_pool2d.default": OpCategory.REDUCTION,
    "aten.softmax.int": OpCategory.REDUCTION,
    "aten._softmax.default": OpCategory.REDUCTION,
    "aten.mean.dim": OpCategory.REDUCTION,
    "aten.argmax.default": OpCategory.REDUCTION,
    "aten.reshape.default": OpCategory.SHAPE_ALIAS,
    "aten.view.default": OpCategory.SHAPE_ALIAS,
    "aten._unsafe_view.default": OpCategory.SHAPE_ALIAS,
    "aten.flatten.using_ints": OpCategory.SHAPE_ALIAS,
    "aten.contiguous.default": OpCategory.SHAPE_ALIAS,
    "aten.unsqueeze.default": OpCategory.SHAPE_ALIAS,
    "aten.squeeze.dim": OpCategory.SHAPE_ALIAS,
    "aten.squeeze.default": OpCategory.SHAPE_ALIAS,
    "aten.alias.default": OpCategory.SHAPE_ALIAS,
    "aten.detach.default": OpCategory.SHAPE_ALIAS,
    "aten.detach_.default": OpCategory.SHAPE_ALIAS,
    "aten.dropout.default": OpCategory.SHAPE_ALIAS,
    "<built-in function getitem>": OpCategory.SHAPE_ALIAS,
    "aten.t.default": OpCategory.SHAPE_ALIAS,
    "aten.expand.default": OpCategory.SHAPE_ALIAS,
    "aten.slice.Tensor": OpCategory.SHAPE_ALIAS,
    "aten.select.int": OpCategory.SHAPE_ALIAS,
    "aten.transpose.int": OpCategory.SHAPE_ALIAS,
    "aten.permute.default": OpCategory.SHAPE_ALIAS,
    "aten.cat.default": OpCategory.SPECIAL,
    "aten.embedding.default": OpCategory.SPECIAL,
    "wrap_with_set_grad_enabled": OpCategory.SPECIAL,
    "aten.index_copy.default": OpCategory.SPECIAL,
    "aten.full.default": OpCategory.SPECIAL,
    "aten._assert_tensor_metadata.default": OpCategory.NOOP,
}
for _op in EW_OPS:
    _TABLE.setdefault(_op, OpCategory.ELEMENTWISE)


def classify_op(op_type: str) -> OpCategory:
    return _TABLE.get(op_type, OpCategory.SPECIAL)
