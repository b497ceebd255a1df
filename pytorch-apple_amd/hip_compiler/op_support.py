"""Which IR ops the MI355X backend runs (the ``partition()`` callback).

Same callback signature as the reference's ``is_cuda_op_supported(op_type, attrs)``
(`cuda_compiler/op_support.py:9-73`, `npu_compiler/partitioner.py:42`). Unlike
the reference, ``attrs`` is consulted where a variant of an op has no device
lowering (e.g. ``mean.dim`` over non-trailing dims), so the partitioner routes
that node to the CPU instead of failing at compile time.
"""

from __future__ import annotations

from hip_compiler.codegen import EW_OPS

_HIP_SUPPORTED_OPS: set[str] = {
    # GEMM-shaped
    "aten.linear.default", "aten.matmul.default", "aten.addmm.default", "aten.mm.default", "aten.bmm.default",
    # convolution networks
    "aten.conv2d.default", "aten.batch_norm.default", "aten.max_pool2d.default",
    "aten.adaptive_avg_pool2d.default",
    # reductions
    "aten.softmax.int", "aten._softmax.default", "aten.mean.dim", "aten.argmax.default",
    # specials
    "aten.embedding.default", "aten.index_copy.default", "aten.full.default", "aten.cat.default",
    "wrap_with_set_grad_enabled",
    # views and no-ops
    "aten.reshape.default", "aten.view.default", "aten._unsafe_view.default", "aten.flatten.using_ints",
    "aten.contiguous.default", "aten.unsqueeze.default", "aten.squeeze.dim", "aten.squeeze.default",
    "aten.alias.default", "aten.detach.default", "aten.detach_.default", "aten.dropout.default",
    "<built-in function getitem>", "aten.t.default", "aten.expand.default", "aten.slice.Tensor",
    "aten.select.int", "aten.transpose.int", "aten.permute.default", "aten._assert_tensor_metadata.default",
} | set(EW_OPS)


def is_hip_op_supported(op_type: str, attrs: dict | None = None) -> bool:
    if op_type not in _HIP_SUPPORTED_OPS:
        return False
    attrs = attrs or {}
    if op_type == "aten.dropout.default" and attrs.get("train", False) and attrs.get("p", 0.0) != 0.0:
        return False
    def pair(v, default):
        v = attrs.get(v, default)
        return [v, v] if isinstance(v, int) else list(v or default)

    if op_type == "aten.conv2d.default":
        return int(attrs.get("groups", 1)) == 1 and pair("dilation", [1, 1]) == [1, 1]
    if op_type == "aten.batch_norm.default":
        return not attrs.get("training", False)
    if op_type == "aten.max_pool2d.default":
        return pair("dilation", [1, 1]) == [1, 1] and not attrs.get("ceil_mode", False)
    if op_type == "aten.adaptive_avg_pool2d.default":
        return pair("output_size", [1, 1]) == [1, 1]
    if op_type == "aten.mean.dim":
        dims = attrs.get("dim", [-1])
        if dims is None:
            return True
        dims = [dims] if isinstance(dims, int) else list(dims)
        return sorted(dims) in ([-1], [-2, -1], [-3, -2, -1]) or all(d >= 0 for d in dims)
    return True


def get_hip_supported_ops() -> frozenset[str]:
    return frozenset(_HIP_SUPPORTED_OPS)
