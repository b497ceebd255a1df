"""Zero-copy view arithmetic for shape ops (reshape, transpose, expand, slice, ...).

The reference turns transpose/slice/expand into CuPy views at dispatch time
(`cuda_runtime/cuda_executor.py:74-87, 596-649`) and reshape-like ops into
``AliasStep`` rebinding (`cuda_compiler/subgraph_analyzer.py:450-603`). Here the
same decisions are made once at compile time: each such op maps its input
``TView`` to an output ``TView`` over the same storage, or returns ``None`` when
no strided view can express the result (a copy is then materialised).
"""

from __future__ import annotations

from hip_compiler.program import TView, contiguous_strides, numel

INT64_MAX = 9223372036854775807


def restride(v: TView, new_shape) -> TView | None:
    """Strides for ``v.reshape(new_shape)`` without a copy (ATen ``computeStride``), or None."""
    new_shape = tuple(int(s) for s in new_shape)
    if numel(new_shape) != v.numel:
        return None
    if v.is_contiguous():
        return v.with_(shape=new_shape, strides=contiguous_strides(new_shape))
    if v.numel == 0:
        return v.with_(shape=new_shape, strides=contiguous_strides(new_shape))
    old_shape, old_strides = list(v.shape), list(v.strides)
    new_strides = [0] * len(new_shape)
    view_d = len(new_shape) - 1
    chunk_base = old_strides[-1] if old_strides else 1
    tensor_numel = 1
    view_numel = 1
    for td in range(len(old_shape) - 1, -1, -1):
        tensor_numel *= old_shape[td]
        if td == 0 or (old_shape[td - 1] != 1 and old_strides[td - 1] != tensor_numel * chunk_base):
            while view_d >= 0 and (view_numel < tensor_numel or new_shape[view_d] == 1):
                new_strides[view_d] = view_numel * chunk_base
                view_numel *= new_shape[view_d]
                view_d -= 1
            if view_numel != tensor_numel:
                return None
            if td > 0:
                chunk_base = old_strides[td - 1]
                tensor_numel = 1
                view_numel = 1
    if view_d != -1:
        return None
    return v.with_(shape=new_shape, strides=tuple(new_strides))


def transpose(v: TView, d0: int, d1: int) -> TView:
    n = len(v.shape)
    d0 %= n
    d1 %= n
    sh, st = list(v.shape), list(v.strides)
    sh[d0], sh[d1] = sh[d1], sh[d0]
    st[d0], st[d1] = st[d1], st[d0]
    return v.with_(shape=tuple(sh), strides=tuple(st))


def permute(v: TView, dims) -> TView:
    n = len(v.shape)
    dims = [d % n for d in dims]
    return v.with_(shape=tuple(v.shape[d] for d in dims), strides=tuple(v.strides[d] for d in dims))


def expand(v: TView, size) -> TView:
    size = [int(s) for s in size]
    pad = len(size) - len(v.shape)
    shape = [1] * pad + list(v.shape)
    strides = [0] * pad + list(v.strides)
    out_sh, out_st = [], []
    for i, s in enumerate(size):
        if s == -1:
            s = shape[i]
        if shape[i] == 1 and s != 1:
            out_st.append(0)
        else:
            out_st.append(strides[i])
        out_sh.append(s)
    return v.with_(shape=tuple(out_sh), strides=tuple(out_st))


def broadcast_to(v: TView, shape) -> TView:
    """Right-aligned broadcast of ``v`` to ``shape`` (numpy/ATen rules)."""
    return expand(v, shape)


def slice_(v: TView, dim: int, start, end, step: int = 1) -> TView:
    n = len(v.shape)
    dim %= n
    size = v.shape[dim]
    start = 0 if start is None else int(start)
    end = size if end is None else int(end)
    if start < 0:
        start += size
    if end < 0:
        end += size
    start = min(max(start, 0), size)
    end = min(max(end, start), size)
    length = (end - start + step - 1) // step
    sh, st = list(v.shape), list(v.strides)
    sh[dim] = length
    off = v.offset + start * st[dim]
    st[dim] = st[dim] * step
    return v.with_(offset=off, shape=tuple(sh), strides=tuple(st))


def select(v: TView, dim: int, index: int) -> TView:
    n = len(v.shape)
    dim %= n
    if index < 0:
        index += v.shape[dim]
    sh, st = list(v.shape), list(v.strides)
    off = v.offset + index * st[dim]
    del sh[dim]
    del st[dim]
    return v.with_(offset=off, shape=tuple(sh), strides=tuple(st))


def squeeze_like(v: TView, out_shape) -> TView | None:
    return restride(v, out_shape)
