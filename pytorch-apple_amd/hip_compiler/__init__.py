"""HIP subgraph compiler for MI355X (gfx950).

Entry point ``compile_subgraph(ir_dict) -> HIPProgram``, the drop-in counterpart
of the reference's ``cuda_compiler.compile_subgraph`` (`cuda_compiler/__init__.py:20-80`)
used as ``DAGExecutor``'s ``compile_fn``. Pipeline: load the IR dict, lower it to
launch steps over strided views (pattern pre-passes, greedy elementwise chains),
collect the generated kernel sources, plan the arena, package the program.

``compute_dtype`` is inferred from the IR (bf16 when any floating tensor is bf16)
instead of defaulting to float16 as in the reference (D1); it is informational —
every tensor keeps its own IR dtype.
"""

from __future__ import annotations

from hip_compiler.buffer_planner import buffer_allocations, plan_arena
from hip_compiler.op_support import get_hip_supported_ops, is_hip_op_supported
from hip_compiler.persistent import enabled as persistent_enabled
from hip_compiler.persistent import fuse_attention_step, fuse_decode_step
from hip_compiler.program import HIPProgram, KernelSource, TView, contiguous_strides
from hip_compiler.subgraph_analyzer import analyze_subgraph
from npu_compiler.ir_reader import IRGraph, load_ir_from_dict


def _infer_compute_dtype(graph: IRGraph) -> str:
    dts = {t.dtype for n in graph.nodes for t in n.outputs} | {t.dtype for t in graph.graph_inputs} | \
          {w.dtype for w in graph.weights}
    for cand in ("bfloat16", "float16"):
        if cand in dts:
            return cand
    return "float32"


def compile_subgraph(ir_dict: dict, compute_dtype: str | None = None, *, inplace_inputs: bool = True,
                     fuse: bool = True, exact_attention: bool = False,
                     fold_attention: bool | None = None, persistent: bool | None = None) -> HIPProgram:
    """Compile one IR dict (a whole graph or one device partition) into a HIPProgram.

    ``inplace_inputs``: let ``index_copy`` update a graph-input cache in place when nothing else
    reads it. ``fuse``: run the pattern pre-passes (off = one generic lowering per op).
    ``exact_attention``: decode attention repeats every CPU rounding point, including the bf16
    rounding of the softmax probabilities (two kernels and a combine-free output pass) instead of
    the default split-S kernel whose combine folds into the following projection.
    ``fold_attention``: combine the split-S partials in the prologue of the projection that reads
    the attention output (True) or in a kernel of their own (False); None = the default.
    ``persistent``: run a whole decoder step as one persistent launch when the fused lowering is
    one (``hip_compiler.persistent``); None = ``HIPRT_PERSISTENT`` (default on).
    """
    return compile_graph(load_ir_from_dict(ir_dict), compute_dtype, inplace_inputs=inplace_inputs, fuse=fuse,
                         exact_attention=exact_attention, fold_attention=fold_attention, persistent=persistent)


def compile_graph(graph: IRGraph, compute_dtype: str | None = None, *, inplace_inputs: bool = True,
                  fuse: bool = True, exact_attention: bool = False, fold_attention: bool | None = None,
                  persistent: bool | None = None) -> HIPProgram:
    low = analyze_subgraph(graph, inplace_inputs=inplace_inputs, fuse=fuse, exact_attention=exact_attention,
                           fold_attention=fold_attention)
    out_views: dict[str, TView] = {}
    for spec in graph.graph_outputs:
        v = low.view(spec.name)
        st = low.storages[v.storage]
        whole = v.is_contiguous() and v.offset == 0 and v.numel * v.itemsize == st.nbytes
        ok = whole and (st.kind == "arena" or (st.kind == "input" and st.name in low.mutated_inputs))
        if not ok or any(o.storage == v.storage for o in out_views.values()):
            dst = low.new_storage(spec.name + ".out", v.shape, v.dtype)
            low.emit_copy(v, dst, [spec.name], [spec.name])
            v = dst
        if tuple(v.shape) != tuple(spec.shape):
            v = v.with_(shape=tuple(spec.shape), strides=contiguous_strides(spec.shape))
        out_views[spec.name] = v
    steps = low.steps
    if fuse and (persistent if persistent is not None else persistent_enabled()):
        steps = fuse_decode_step(low.steps, low.storages) or fuse_attention_step(low.steps, low.storages) or low.steps
    arena_bytes = plan_arena(steps, low.storages, {v.storage for v in out_views.values()})
    by_storage = {}
    for name, v in low.views.items():
        if v.storage not in by_storage and v.offset == 0 and v.is_contiguous():
            by_storage[v.storage] = (v.shape, v.dtype)
    prog = HIPProgram(
        steps=steps,
        buffer_allocations=buffer_allocations(low.storages, by_storage),
        input_specs=list(graph.graph_inputs),
        output_specs=list(graph.graph_outputs),
        weight_specs=list(graph.weights),
        weight_name_mapping=dict(graph.weight_name_mapping),
        kernel_sources=[KernelSource(k, s) for k, s in low.kernel_sources.items()],
        compute_dtype=compute_dtype or _infer_compute_dtype(graph),
        storages=low.storages,
        views=low.views,
        output_views=out_views,
        arena_bytes=arena_bytes,
        stats={"launches": len(steps), "mutated_inputs": sorted(low.mutated_inputs)},
    )
    return prog


__all__ = ["compile_subgraph", "compile_graph", "is_hip_op_supported", "get_hip_supported_ops", "HIPProgram"]
