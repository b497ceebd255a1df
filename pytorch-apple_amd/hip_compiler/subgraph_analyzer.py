"""Subgraph analyzer: IR graph → ordered launch steps over views and arena storages.

Counterpart of the reference's ``analyze_subgraph`` (`cuda_compiler/subgraph_analyzer.py:797-981`).
The algorithm keeps the reference's shape — pattern pre-passes first, then one
walk over the nodes in topological order that classifies each op and greedily
grows elementwise chains — with MI355X-specific choices:

* pattern pre-passes (`patterns.py`) claim RMSNorm chains (reference cs:667-756),
  add+softmax (cs:759-789) and the whole GQA decode-attention chain (the span of
  cs:85-160 plus the scale/mask/softmax steps between the two matmuls);
* shape ops never launch: they map a ``TView`` to a ``TView`` (``views.py``);
* a chain grows while the new elementwise node reads the chain's current tail, the
  tail has exactly one consumer and the output shape is unchanged (the reference's
  rule, cs:984-1013); operands may broadcast (stride 0), fixing defect D3;
* chains are emitted lazily, when something first needs their value, so the step
  list is already in dependency order (the reference re-sorts with Kahn's
  algorithm afterwards, cs:1047-1091);
* an ``index_copy`` whose target is a graph input read by nothing else updates that
  input in place (the reference copies the whole cache every step, defect D7).
"""

from __future__ import annotations

import dataclasses

import math
import os
from dataclasses import dataclass, field

from hip_compiler import views as V
from hip_compiler.codegen import MAX_CHAIN_INPUTS, VEC, ChainOp, generate_chain, vector_ok
from hip_compiler.op_classify import OpCategory, classify_op
from hip_compiler.program import (DTYPE_CODE, ELEM_SIZE, FLOAT_DTYPES, LaunchStep, Ref, Storage, TView,
                                  contiguous_strides, numel)
from npu_compiler.ir_reader import IRGraph, OpNode

HS_BF16, HS_F16 = DTYPE_CODE["bfloat16"], DTYPE_CODE["float16"]


# linears with at least this many activation rows use the MFMA GEMM (weights read once per
# column tile) instead of the streaming GEMV (weights re-read per block of 4 rows)
GEMM_MIN_M = 16
# up to this many activation rows, bf16 linears take the skinny MFMA kernels (gemv.hip
# k_skinny_*: every weight element read once and multiplied with all rows in one 16x16x32 MFMA)
SKINNY_MAX_M = 32
# from this many rows the bf16 linears take the skinny kernels rather than the streaming GEMVs,
# which stream the weights once per 4 rows (cfg1 at T = 2 .. 15: 21-22 us per block against
# 25-80 us)
SKINNY_MIN_M = 2
# the SiLU skinny kernel with the RMSNorm folded in (gemv.hip k_skinny_silu_norm_*): rows of at
# most this many elements (its LDS copy of the 16 normalised rows), and its waves per workgroup
SKINNY_NORM_MAX_K = 2048
SKINNY_NORM_WAVES = 8
# gate/up with the SiLU * up epilogue from SKINNY_MAX_M + 1 to this many rows takes the wide
# streaming kernel (gemv.hip k_wide_silu_mt4 / _mt8: 4 waves per workgroup over WIDE_TA tiles
# of 8 output pairs and every activation row, weights read once); WIDE_TA must match the kernel's
WIDE_MAX_M = int(os.environ.get("HIPRT_WIDE_MAX_M", "128"))
WIDE_TA = 5
# past 64 rows, two 64-row workgroups per group of weight tiles (k_wide_silu_mt4x2) instead of
# one 128-row workgroup (k_wide_silu_mt8)
WIDE_HALVES = os.environ.get("HIPRT_WIDE_HALVES", "1") == "1"
GEMM_TARGET_WGS = 256    # workgroups a GEMM launch should reach (one per CU)
GEMM_MIN_KCHUNK = 256    # smallest K range of one split-K workgroup
GEMM_DMA_MAX_TILES = 1024   # tile grids at least this large keep register staging (gemm_tiling)
CONV_D2_MAX_K = int(os.environ.get("HIPRT_CONV_D2_MAX_K", "1024"))   # convs up to this K: 2-stage staging
CONV_D1_MAX_K = int(os.environ.get("HIPRT_CONV_D1_MAX_K", "64"))   # emit_conv_nhwc: one-stage 64x64 kernels up to this K
CONV_SMALL_TILE_MAX_K = 512   # conv_gemm_tiling: 64 x 64 tiles for K up to this over many tiles
CONV_NFAST = os.environ.get("HIPRT_CONV_NFAST", "1") == "1"   # conv tile order by operand sizes (emit_conv_nhwc)


def gemm_tiling(M: int, N: int, K: int, nw: int = 1) -> tuple[int, int, int, bool]:
    """(BM, BN, split-K, direct-to-LDS) for an M x N x K MFMA GEMM (nw = 2: two weights, BN
    columns of each).

    Rules fitted to sweeps on MI355X at M = 512 (bf16, K step 64, split-K reduce pass
    included). Direct-to-LDS staging (the ``_k64d`` kernels: operands land in LDS several
    K steps ahead without passing through registers) needs K % 64 == 0; it pays wherever the
    tile grid is not large enough to hide the operand latency by itself, i.e. below
    GEMM_DMA_MAX_TILES tiles. Two weights (gate/up with the SiLU-mul epilogue): 64 x 64
    tiles, 52 us against 57 for 128 x 64 without. One weight: the largest tile that still
    gives >= 256 workgroups; long rows (K >= 4096) take 128 x 128 with up to 4 K splits
    (down_proj 512 x 1536 x 8960: 26 us with 4 splits, 32 with 8), or, with fewer than 48 such
    tiles, 64 x 64 with up to 8 (down_proj at M = 128, a 128-token prefill: 17.0 us on 64 x 64
    with 8 splits, 18.2 on 64 x 128 with 8, 19.6 on 128 x 128 with 16, 29.0 with 4); other grids under 256
    tiles split K toward ~384 workgroups (o_proj 512 x 1536 x 1536 on 64 x 64: 9.5 us with
    2 splits, 12.9 unsplit). The lm_head (4,748 tiles of 128 x 128) keeps register staging:
    324 us against 367."""
    dma = K % 64 == 0
    ntiles = lambda bm, bn: ((M + bm - 1) // bm) * ((N + bn - 1) // bn)
    if nw == 2:
        if dma:
            # 128 x 96 tiles (4 x 1 waves) where they still give a full round of workgroups: more
            # MFMA work per operand byte than 64 x 64 (77 against 44 FLOP per staged byte), and a
            # grid that fits one round at two per CU (M = 512, N = 8960: 376)
            return (128, 96, 1, True) if ntiles(128, 96) >= GEMM_TARGET_WGS else (64, 64, 1, True)
        for bm, bn in ((128, 64), (64, 64)):
            if ntiles(bm, bn) >= GEMM_TARGET_WGS:
                return bm, bn, 1, False
        return 64, 64, 1, False
    for bm, bn in ((128, 128), (64, 128), (64, 64)):
        t = ntiles(bm, bn)
        if t >= GEMM_TARGET_WGS:
            return bm, bn, 1, dma and t < GEMM_DMA_MAX_TILES
    if K >= 4096:
        t = ntiles(128, 96)
        if dma and t >= 48:
            # 128 x 96 over 4 x 1 waves, up to 8 K splits toward one round of 512 workgroups (two per
            # CU): down_proj 512 x 1536 x 8960 23.1 us + 5.3 reduce, against 28.6 + 4.6 on 128 x 128
            # with 4 splits (one workgroup per CU)
            return 128, 96, max(1, min(8, 512 // t, K // GEMM_MIN_KCHUNK)), dma
        t = ntiles(128, 128)
        if t >= 48:
            return 128, 128, max(1, min(4, 384 // t, K // GEMM_MIN_KCHUNK)), dma
        t = ntiles(64, 64)
        return 64, 64, max(1, min(8, (384 + t - 1) // t, K // GEMM_MIN_KCHUNK)), dma
    t = ntiles(64, 64)
    return 64, 64, max(1, min((384 + t - 1) // t, K // GEMM_MIN_KCHUNK)), dma


def _is_nhwc(v: TView) -> bool:
    """A 4-d [N, C, H, W] view whose memory is channels-last ([N, H, W, C] contiguous)."""
    if len(v.shape) != 4:
        return False
    _, C, H, W = v.shape
    return tuple(v.strides) == (H * W * C, 1, W * C, C) and C > 1


def conv_gemm_tiling(M: int, N: int, K: int) -> tuple[int, int, int]:
    """(BM, BN, split-K) for a conv as a GEMM over M pixels, N output channels, K = KH*KW*Cin:
    64 x 64 for short K over many tiles (K <= 512, >= 1024 tiles); otherwise the largest tile no
    wider than the channels that still gives >= 256 workgroups; smaller
    grids take 64 x 64 tiles and, for K >= 1024, split K toward ~384 workgroups (fp32
    partials, then the reduce applies the epilogue)."""
    ntiles = lambda bm, bn: ((M + bm - 1) // bm) * ((N + bn - 1) // bn)
    if K <= CONV_SMALL_TILE_MAX_K and ntiles(64, 64) >= 4 * GEMM_TARGET_WGS:
        # short K, many tiles: the time goes to each tile's load latency and store drain, not to
        # MFMA work; 64 x 64 tiles (32 KB of LDS at two stages) let four workgroups share a CU,
        # so one workgroup's loads overlap another's stores
        return 64, 64, 1
    cands = [(bm, bn) for bm, bn in ((128, 128), (128, 64), (64, 128), (64, 64)) if bn <= max(N, 64)]
    for bm, bn in cands:
        if ntiles(bm, bn) >= GEMM_TARGET_WGS:
            return bm, bn, 1
    t = ntiles(64, 64)
    if K >= 1024:
        return 64, 64, max(1, min(8, (384 + t - 1) // t, K // GEMM_MIN_KCHUNK))
    return 64, 64, 1


def grid1d(n: int, block: int = 256, cap: int = 65536) -> tuple[int, int, int]:
    return (max(1, min(cap, (int(n) + block - 1) // block)), 1, 1)


def mean_rows_step(x, out, rows: int, cols: int, x_dtype: str, out_dtype: str, ins, outs) -> LaunchStep:
    """Mean over the last dimension of a [rows, cols] contiguous view: one wave per row when the
    rows are short (k_mean_short, e.g. a 7 x 7 global pool), else one workgroup per row."""
    short = cols <= 64
    return LaunchStep(
        kind="reduction", kernel="k_mean_short" if short else "k_mean_last", module="basic",
        arg_struct="ReduceLastArgs",
        args=dict(x=x, out=out, rows=rows, cols=cols, x_dtype=DTYPE_CODE[x_dtype], out_dtype=DTYPE_CODE[out_dtype]),
        grid=((max(rows, 1) + 3) // 4 if short else max(rows, 1), 1, 1), inputs=ins, outputs=outs,
        params={"rows": rows, "cols": cols})


def apply_alias(node: OpNode, v: TView) -> TView | None:
    """The view a shape op produces from ``v`` (getitem excluded), or None when it needs a copy."""
    op = node.op_type
    out = node.outputs[0]
    a = node.attrs
    if op in ("aten.transpose.int",):
        return V.transpose(v, int(a.get("dim0", 0)), int(a.get("dim1", 1)))
    if op == "aten.t.default":
        return V.transpose(v, 0, 1) if len(v.shape) == 2 else v
    if op == "aten.permute.default":
        return V.permute(v, a.get("dims"))
    if op == "aten.expand.default":
        return V.expand(v, out.shape)
    if op == "aten.slice.Tensor":
        return V.slice_(v, int(a.get("dim", 0)), a.get("start", 0), a.get("end", V.INT64_MAX), int(a.get("step", 1)))
    if op == "aten.select.int":
        return V.select(v, int(a.get("dim", 0)), int(a.get("index", 0)))
    if op in ("aten.alias.default", "aten.detach.default", "aten.detach_.default", "aten.dropout.default"):
        return v
    if op == "aten.contiguous.default":
        return v if v.is_contiguous() else None
    return V.restride(v, out.shape)   # reshape / view / flatten / unsqueeze / squeeze


def skinny_rows(M: int, K: int, dtype: str) -> bool:
    """Rows a linear hands to the skinny MFMA kernels (gemv.hip ``k_skinny_*``: every weight
    element read once and multiplied with up to 16 rows per MFMA) below the MFMA GEMM's range."""
    return SKINNY_MIN_M <= M < GEMM_MIN_M and dtype == "bfloat16" and K % 64 == 0 and K >= 512


@dataclass
class _Chain:
    ops: list[ChainOp] = field(default_factory=list)
    ext: list[TView] = field(default_factory=list)
    ext_names: list[str] = field(default_factory=list)
    node_names: list[str] = field(default_factory=list)
    tail: str = ""
    shape: tuple[int, ...] = ()
    dtype: str = "float32"


_RENAMES = ("aten.alias.default", "aten.detach.default")


def drop_renames(graph: IRGraph) -> IRGraph:
    """``graph`` without ``alias`` / ``detach`` nodes: their readers read the source tensor
    itself. They only rename a value, but a rename between two ops hides one from a
    fusion pattern (transformers 5 places an ``alias`` between the final RMSNorm and the
    lm_head). A node whose output is a graph output stays."""
    outs = {o.name for o in graph.graph_outputs}
    src: dict[str, object] = {}
    nodes = []
    for n in graph.nodes:
        ins = [src.get(t.name, t) for t in n.inputs]
        if n.op_type in _RENAMES and ins and n.outputs[0].name not in outs:
            src[n.outputs[0].name] = ins[0]
            continue
        nodes.append(n if not src else dataclasses.replace(n, inputs=ins))
    return dataclasses.replace(graph, nodes=nodes) if src else graph


class Lowering:
    """Lowers one IR graph; ``steps``, ``storages`` and ``views`` are the result."""

    def __init__(self, graph: IRGraph, inplace_inputs: bool = True, exact_attention: bool = False,
                 fold_attention: bool | None = None):
        graph = drop_renames(graph)
        self.g = graph
        self.inplace_inputs = inplace_inputs
        self.exact_attention = exact_attention
        # fold the split-attention combine into the following projection's prologue (True) or
        # emit it as its own small kernel (False); when not given, HIPRT_FOLD_ATTN decides
        if fold_attention is None:
            fold_attention = os.environ.get("HIPRT_FOLD_ATTN", "1") == "1"
        self.fold_attn_combine = fold_attention
        # convolutions on channels-last activations through the MFMA GEMM (HIPRT_CONV_NHWC=0: NCHW kernels only)
        self.conv_nhwc = os.environ.get("HIPRT_CONV_NHWC", "1") == "1"
        self._conv_zero: Ref | None = None
        # bound conv weights read as (zero-padded) OHWI: (name, OIHW view, destination view,
        # (cin, kh, kw) of the source, (cp, khp, kwp) of the destination)
        self._ohwi: list = []
        self.steps: list[LaunchStep] = []
        self.storages: dict[str, Storage] = {}
        self.views: dict[str, TView] = {}
        self.kernel_sources: dict[str, str] = {}
        self.consumers: dict[str, list[OpNode]] = {}
        self.producer: dict[str, OpNode] = {}
        for n in graph.nodes:
            for t in n.inputs:
                self.consumers.setdefault(t.name, []).append(n)
            for t in n.outputs:
                self.producer[t.name] = n
        self.chains: dict[str, _Chain] = {}
        self.claimed: dict[str, object] = {}     # node name -> pattern emitter (at its last node) or None
        self.lazy: dict[str, object] = {}        # tensor name -> emitter run when the value is first needed
        self.rms_info: dict[str, dict] = {}      # RMSNorm output -> {x, w, eps, n_dtype} (foldable prologue)
        self.attn_info: dict[str, dict] = {}     # split decode attention output -> partials (foldable prologue)
        self.mask_extents: dict[tuple, Ref] = {}  # prefill mask view -> per-query-block open extent
        self.graph_output_names = {o.name for o in graph.graph_outputs}
        self.mutated_inputs: set[str] = set()
        self._uid = 0
        for spec in graph.graph_inputs:
            self._external(spec.name, spec.shape, spec.dtype, "input")
        for ph, sd in graph.weight_name_mapping.items():
            w = next((w for w in graph.weights if w.name == sd), None)
            if w is not None:
                self._external(ph, w.shape, w.dtype, "weight")
        for w in graph.weights:
            if w.name not in self.views:
                self._external(w.name, w.shape, w.dtype, "weight")

    # ------------------------------------------------------------------ storages and views

    def _external(self, name: str, shape, dtype: str, kind: str) -> None:
        shape = tuple(int(s) for s in shape)
        self.storages[name] = Storage(name, kind, numel(shape) * ELEM_SIZE[dtype], dtype)
        self.views[name] = TView(name, 0, shape, contiguous_strides(shape), dtype)

    def new_storage(self, name: str, shape, dtype: str, kind: str = "arena") -> TView:
        shape = tuple(int(s) for s in shape)
        key = name
        while key in self.storages:
            self._uid += 1
            key = f"{name}#{self._uid}"
        self.storages[key] = Storage(key, kind, max(numel(shape) * ELEM_SIZE[dtype], 1), dtype)
        return TView(key, 0, shape, contiguous_strides(shape), dtype)

    def scratch(self, name: str, nbytes: int, persistent: bool = False) -> Ref:
        key = name
        while key in self.storages:
            self._uid += 1
            key = f"{name}#{self._uid}"
        self.storages[key] = Storage(key, "persistent" if persistent else "arena", max(int(nbytes), 4), "uint8",
                                     zero_init=persistent)
        return Ref(key, 0)

    @staticmethod
    def ref(v: TView) -> Ref:
        return Ref(v.storage, v.offset * ELEM_SIZE[v.dtype])

    def view(self, name: str) -> TView:
        if name in self.chains:
            self.flush_chain(name)
        if name in self.lazy:
            self.lazy.pop(name)()
        if name not in self.views:
            raise KeyError(f"tensor {name} has no value (producer not lowered)")
        return self.views[name]

    def contiguous(self, name: str, v: TView | None = None) -> TView:
        """A contiguous view with the value of ``name`` (copying when needed)."""
        v = v or self.view(name)
        if v.is_contiguous():
            return v
        out = self.new_storage(name + ".c", v.shape, v.dtype)
        self.emit_copy(v, out, [name], [name + ".c"])
        return out

    def emit(self, step: LaunchStep) -> None:
        self.steps.append(step)

    def aligned16(self, v: TView, name: str) -> TView:
        """``v`` (contiguous) if it starts on a 16-byte boundary, else a fresh aligned copy of it."""
        if (v.offset * ELEM_SIZE[v.dtype]) % 16 == 0:
            return v
        if name + ".a16" in self.views:
            return self.views[name + ".a16"]
        aligned = self.new_storage(name + ".a16", v.shape, v.dtype)
        self.emit_copy(v, aligned, [name], [name + ".a16"])
        self.views[name + ".a16"] = aligned
        return aligned

    def emit_copy(self, src: TView, dst: TView, ins: list[str], outs: list[str]) -> None:
        nd = len(src.shape)
        if nd > 6:
            raise NotImplementedError("copy of rank > 6")
        shape = list(src.shape) + [1] * (6 - nd)
        ss = list(src.strides) + [0] * (6 - nd)
        ds = list(dst.strides) + [0] * (6 - nd)
        n = src.numel
        nbytes = n * ELEM_SIZE[src.dtype]
        if src.dtype == dst.dtype and src.is_contiguous() and dst.is_contiguous() and nbytes % 16 == 0 and \
                (src.offset * ELEM_SIZE[src.dtype]) % 16 == 0 and (dst.offset * ELEM_SIZE[dst.dtype]) % 16 == 0:
            # a plain byte copy: 16-byte chunks, one contiguous range per workgroup, eight chunks
            # in flight per thread
            chunks = nbytes // 16
            self.emit(LaunchStep(
                kind="copy", kernel="k_copy16", module="basic", arg_struct="CopyArgs",
                args=dict(dst=self.ref(dst), src=self.ref(src), n=chunks, shape=[1] * 6, sstride=[0] * 6,
                          dstride=[0] * 6, ndim=1, sdtype=DTYPE_CODE[src.dtype], ddtype=DTYPE_CODE[dst.dtype]),
                grid=grid1d(-(-chunks // 8), cap=8192), inputs=ins, outputs=outs, params={"total": n}))
            return
        self.emit(LaunchStep(
            kind="copy", kernel="k_copy", module="basic", arg_struct="CopyArgs",
            args=dict(dst=self.ref(dst), src=self.ref(src), n=n, shape=shape, sstride=ss, dstride=ds,
                      ndim=max(nd, 1), sdtype=DTYPE_CODE[src.dtype], ddtype=DTYPE_CODE[dst.dtype]),
            grid=grid1d(n), inputs=ins, outputs=outs, params={"total": n}))

    # ------------------------------------------------------------------ elementwise chains

    def flush_chain(self, tail: str) -> None:
        ch = self.chains.pop(tail)
        out = self.new_storage(tail, ch.shape, ch.dtype)
        name, src = generate_chain(ch.ops, ch.ext, ch.shape, ch.dtype)
        self.kernel_sources[name] = src
        n = numel(ch.shape)
        # the vector form takes 8 elements per thread (its `n` counts 8-element groups)
        nt = n // VEC if vector_ok(ch.ext, ch.shape, ch.dtype) else n
        ptrs = [self.ref(v) for v in ch.ext] + [None] * (MAX_CHAIN_INPUTS - len(ch.ext))
        self.emit(LaunchStep(
            kind="fused", kernel=name, module=name, arg_struct="FusedArgs",
            args=dict(out=self.ref(out), **{"in": ptrs}, n=nt), grid=grid1d(nt),
            inputs=list(ch.ext_names), outputs=[tail],
            params={"total": n, "ops": [o.op_type for o in ch.ops], "nodes": list(ch.node_names)}))
        self.views[tail] = out

    def flush_chains_reading(self, storage: str) -> None:
        for tail in [t for t, ch in self.chains.items() if any(v.storage == storage for v in ch.ext)]:
            if tail in self.chains:
                self.flush_chain(tail)

    def lower_elementwise(self, node: OpNode) -> None:
        out = node.outputs[0]
        shape = tuple(out.shape)
        if node.op_type == "aten.to.dtype" or node.op_type == "aten._to_copy.default":
            src = node.inputs[0]
            if src.dtype == out.dtype and src.name not in self.chains:
                self.views[out.name] = self.view(src.name)
                return
        ext_inputs = [t for t in node.inputs]
        # extend an open chain whose tail this node reads (single consumer, same shape)
        chain = None
        for t in ext_inputs:
            ch = self.chains.get(t.name)
            if ch is not None and len(self.consumers.get(t.name, [])) == 1 and ch.shape == shape:
                new_ext = {x.name for x in ext_inputs if x.name != t.name and x.name not in ch.ext_names}
                if len(ch.ext) + len(new_ext) <= MAX_CHAIN_INPUTS:
                    chain = ch
                    break
        if chain is None:
            chain = _Chain(shape=shape)
        else:
            del self.chains[chain.tail]
        operands = []
        for t in ext_inputs:
            if t.name == chain.tail and chain.ops:
                operands.append(("val", len(chain.ops) - 1))
                continue
            if t.name in chain.ext_names:
                operands.append(("ext", chain.ext_names.index(t.name)))
                continue
            v = self.view(t.name)
            try:
                v = V.broadcast_to(v, shape)
            except Exception as e:  # pragma: no cover - malformed IR
                raise ValueError(f"{node.name}: cannot broadcast {t.name} {v.shape} to {shape}") from e
            chain.ext.append(v)
            chain.ext_names.append(t.name)
            operands.append(("ext", len(chain.ext) - 1))
        attrs = dict(node.attrs)
        if node.op_type in ("aten.add.Tensor", "aten.add_.Tensor", "aten.sub.Tensor", "aten.mul.Tensor",
                            "aten.mul_.Tensor", "aten.div.Tensor") and len(operands) == 1:
            operands.append(("scalar", float(attrs.get("other", 0.0))))
        chain.ops.append(ChainOp(node.op_type, operands, out.dtype, attrs))
        chain.node_names.append(node.name)
        chain.tail = out.name
        chain.dtype = out.dtype
        self.chains[out.name] = chain

    # ------------------------------------------------------------------ generic lowering per op

    def lower_alias(self, node: OpNode) -> None:
        """Views are resolved when first used, so a view nobody reads costs nothing."""
        self.lazy[node.outputs[0].name] = lambda node=node: self._alias_now(node)

    def _alias_now(self, node: OpNode) -> None:
        op = node.op_type
        out = node.outputs[0]
        if op == "<built-in function getitem>":
            idx = int(node.attrs.get("index", 0))
            src = node.inputs[idx] if idx < len(node.inputs) else node.inputs[0]
            self.views[out.name] = self.view(src.name)
            return
        v = self.view(node.inputs[0].name)
        nv = apply_alias(node, v)
        if nv is None:
            nv = V.restride(self.contiguous(node.inputs[0].name, v), out.shape)
        if tuple(nv.shape) != tuple(out.shape):
            raise ValueError(f"{node.name}: view shape {nv.shape} != declared {out.shape}")
        self.views[out.name] = nv

    def lower_linear(self, node: OpNode) -> None:
        x_t, w_t = node.inputs[0], node.inputs[1]
        b_t = node.inputs[2] if len(node.inputs) > 2 else None
        out = node.outputs[0]
        if self.gemv_ok(x_t.name, w_t.name, out.dtype, x_t.dtype) and (b_t is None or b_t.dtype == "bfloat16"):
            self.emit_gemv(x_t.name, w_t.name, b_t.name if b_t else None, out.name, tuple(out.shape),
                           epi="bias", nodes=[node.name])
            return
        self.emit_linear(x_t.name, w_t.name, b_t.name if b_t else None, out.name, tuple(out.shape), out.dtype,
                         resid=None, node_names=[node.name])

    # ------------------------------------------------------------------ fused decode GEMV

    def foldable_norm(self, x_name: str, fused_nodes: set[str]) -> dict | None:
        """RMSNorm parameters when ``x_name`` is a not-yet-emitted RMSNorm read only by ``fused_nodes``."""
        info = self.rms_info.get(x_name)
        if info is None or x_name not in self.lazy:
            return None
        if x_name in self.graph_output_names:
            return None
        if any(n.name not in fused_nodes for n in self.consumers.get(x_name, [])):
            return None
        return info

    def foldable_attn(self, x_name: str, fused_nodes: set[str]) -> dict | None:
        """Split-attention partials when ``x_name`` is a pure, order-preserving view of a decode
        attention output that nothing else reads and that has not been combined yet."""
        if any(n.name not in fused_nodes for n in self.consumers.get(x_name, [])):
            return None
        chain: list[OpNode] = []
        name = x_name
        while name not in self.attn_info:
            prod = self.producer.get(name)
            if (prod is None or classify_op(prod.op_type) != OpCategory.SHAPE_ALIAS
                    or prod.op_type in ("<built-in function getitem>", "aten.expand.default", "aten.slice.Tensor",
                                        "aten.select.int")):
                return None
            if len(self.consumers.get(prod.inputs[0].name, [])) != 1 or prod.inputs[0].name in self.graph_output_names:
                return None
            chain.append(prod)
            name = prod.inputs[0].name
        info = self.attn_info[name]
        if name not in self.lazy or name in self.graph_output_names:
            return None
        shape = tuple(info["shape"])
        v = TView("virtual", 0, shape, contiguous_strides(shape), "bfloat16")
        for node in reversed(chain):
            v = apply_alias(node, v)
            if v is None:
                return None
        if not (v.is_contiguous() and v.offset == 0):
            return None
        return info

    def gemv_ok(self, x_name: str, w_name: str, out_dtype: str, x_dtype: str = "bfloat16") -> bool:
        """Shapes the streaming GEMV kernels take: bf16, K % 8 == 0, contiguous 16-byte aligned weights."""
        w = self.views.get(w_name)
        if w is None or w.dtype != "bfloat16" or out_dtype != "bfloat16" or x_dtype != "bfloat16":
            return False
        if len(w.shape) != 2 or not w.is_contiguous():
            return False
        K = w.shape[1]
        if K % 8 or (w.offset * 2) % 16:
            return False
        info = self.rms_info.get(x_name)
        if info is not None and x_name in self.lazy:
            return info["x_dtype"] == "bfloat16"
        return True

    def emit_gemv(self, x_name: str, w_name: str, b_name: str | None, out_name: str, out_shape, *, epi: str,
                  nodes: list[str], resid: str | None = None, w2: str | None = None, b2: str | None = None,
                  argmax_out=None) -> None:
        """One fused GEMV launch (csrc/kernels/gemv.hip); folds a pending RMSNorm of ``x`` when possible.
        Prefill-shaped calls (M >= GEMM_MIN_M) go to the MFMA GEMM instead."""
        w_view = self.view(w_name)
        n_out = numel(out_shape) // w_view.shape[0] if w_view.shape[0] else 0
        if epi in ("bias", "resid", "silu") and (n_out >= GEMM_MIN_M and w_view.shape[1] % 32 == 0
                                                 or skinny_rows(n_out, w_view.shape[1], "bfloat16")):
            self.emit_gemm(x_name, w_name, b_name, out_name, out_shape, "bfloat16", epi=epi, nodes=nodes,
                           resid=resid, w2=w2, b2=b2)
            return
        norm = self.foldable_norm(x_name, set(nodes))
        attn = None
        w = self.contiguous(w_name)
        K = w.shape[1]
        N = w.shape[0]
        if norm is not None:
            x = self.aligned16(self.contiguous(norm["x"]), norm["x"])
            M = x.numel // K
            mb = 1 if M == 1 else 4
            if K > 3072:   # the normalised rows are staged in LDS: MB x 3072 bf16
                norm = None
        if norm is None and self.fold_attn_combine:
            attn = self.foldable_attn(x_name, set(nodes))
            if attn is not None and (K != attn["H"] * 128 or attn["H"] > 16 or attn["nsplit"] > 16
                                     or epi not in ("bias", "resid")):
                attn = None
        if attn is not None:
            x, M = None, 1
        elif norm is None:
            x = self.aligned16(self.contiguous(x_name), x_name)
            M = x.numel // K
        mb = 1 if M == 1 else 4
        if epi == "argmax":
            rpw = 4 if M == 1 else 2
        elif epi == "silu":
            rpw = 1
        else:
            rpw = 1 if M == 1 else 2
        if mb == 4 and epi == "argmax":
            raise NotImplementedError("argmax epilogue with M > 1")
        pro = "attn" if attn is not None else ("norm" if norm is not None else "")
        kname = {("bias", 1, ""): "k_gemv_bias_r1", ("bias", 1, "norm"): "k_gemv_norm_bias_r1",
                 ("resid", 1, ""): "k_gemv_resid_r1", ("silu", 1, ""): "k_gemv_silu_r1",
                 ("silu", 1, "norm"): "k_gemv_norm_silu_r1", ("argmax", 1, "norm"): "k_gemv_norm_argmax_r4",
                 ("argmax", 1, ""): "k_gemv_argmax_r4", ("bias", 4, ""): "k_gemv_bias_m4",
                 ("bias", 4, "norm"): "k_gemv_norm_bias_m4", ("resid", 4, ""): "k_gemv_resid_m4",
                 ("silu", 4, ""): "k_gemv_silu_m4", ("silu", 4, "norm"): "k_gemv_norm_silu_m4",
                 ("bias", 1, "attn"): "k_gemv_attn_bias_r2", ("resid", 1, "attn"): "k_gemv_attn_resid_r2"}.get(
            (epi, mb, pro))
        if kname is None:
            raise NotImplementedError(f"no GEMV kernel for epilogue {epi} M={M} prologue={pro!r}")
        rows_per_wg = None
        if attn is not None:
            # two rows per wave (192 workgroups for N = 1536: 4.24 us, against 4.55 with four
            # rows and 5.18 with one); the 16-split variant when the partials need it
            rpw = 2
            if attn["nsplit"] > 8:
                kname = kname.replace("k_gemv_attn_", "k_gemv_attn16_")
        if epi == "bias" and M == 1 and N >= 65536 and pro == "":
            kname, rpw = "k_gemv_bias_r4", 4
        elif epi in ("bias", "resid") and M == 1 and pro == "" and K >= 4096:
            # long rows: the four waves of a workgroup split K, two rows per workgroup
            kname, rpw, rows_per_wg = f"k_gemv_{epi}_ks_r2", 2, 2
        o = self.new_storage(out_name, out_shape, "bfloat16")
        bias = self.contiguous(b_name) if b_name else None
        r = self.contiguous(resid) if resid else None
        wv2 = self.contiguous(w2) if w2 else None
        bv2 = self.contiguous(b2) if b2 else None
        rows_per_wg = rows_per_wg or 4 * rpw
        nblocks = (N + rows_per_wg - 1) // rows_per_wg
        # kernels with a prologue (RMSNorm) or a per-workgroup reduction (argmax) stride over row
        # blocks with a capped grid, so the prologue is paid once per workgroup (measured: the
        # norm+gate/up GEMV takes 13.6 us strided vs 17.1 us with one workgroup per block); the
        # others get one workgroup per row block so that all weight loads are in flight at once
        gx = min(nblocks, 1024) if (norm is not None or epi == "argmax") else nblocks
        slot = self.scratch(out_name + ".argmax", 8 * max(M, 1) * gx) if epi == "argmax" else None
        args = dict(x=self.ref(x) if x is not None else None, w=self.ref(w), bias=self.ref(bias) if bias else None,
                    out=self.ref(o), resid=self.ref(r) if r else None, w2=self.ref(wv2) if wv2 else None,
                    bias2=self.ref(bv2) if bv2 else None,
                    norm_w=self.ref(self.aligned16(self.contiguous(norm["w"]), norm["w"])) if norm else None,
                    argmax_slot=slot,
                    attn_o=attn["part_o"] if attn else None, attn_ml=attn["part_ml"] if attn else None,
                    M=M, ldx=K, ldo=N, ldr=N, N=N, K=K, eps=float(norm["eps"]) if norm else 0.0,
                    n_dtype=DTYPE_CODE[norm["n_dtype"]] if norm else 0,
                    flags=(1 if bias else 0) | (4 if bv2 else 0),
                    attn_heads=attn["H"] if attn else 0, attn_kvh=attn["KVH"] if attn else 0,
                    attn_splits=attn["nsplit"] if attn else 0)
        ins = [norm["x"] if norm else (attn["out"] + ".partials" if attn else x_name), w_name] + \
            [t for t in (b_name, resid, w2, b2) if t]
        if norm:
            ins.append(norm["w"])
        self.emit(LaunchStep(
            kind="gemv", kernel=kname, module="gemv", arg_struct="GemvArgs", args=args,
            grid=(gx, (M + mb - 1) // mb, 1), inputs=ins, outputs=[out_name],
            params={"M": M, "N": N, "K": K, "epilogue": epi, "norm": norm is not None, "prologue": pro,
                    "has_bias": bias is not None, "weights": 2 if w2 else 1, "transpose_b": True, "nodes": nodes}))
        self.views[out_name] = o
        if epi == "argmax":
            name, shape, dtype = argmax_out
            t = self.new_storage(name, shape, dtype)
            self.emit(LaunchStep(
                kind="reduction", kernel="k_argmax_finalize", module="gemv", arg_struct="ArgmaxFinalizeArgs",
                args=dict(slot=slot, out=self.ref(t), rows=M, parts=gx, out_dtype=DTYPE_CODE[dtype]),
                grid=(M, 1, 1), block=(256, 1, 1), inputs=[out_name], outputs=[name],
                params={"rows": M, "cols": N}))
            self.views[name] = t

    def emit_skinny_silu_norm(self, x_name: str, w, w_name: str, w2: str, b_name: str | None, b2: str | None,
                              out_name: str, out_shape, nodes: list[str]) -> bool:
        """SiLU(x W^T) * (x W2^T) for at most 32 rows whose pending RMSNorm is folded in
        (gemv.hip ``k_skinny_silu_norm_mt*``: each workgroup of 8 waves normalises the rows into
        LDS once, one 8 + 8-row tile per wave); False when ``x`` has no foldable norm or more rows."""
        norm = self.foldable_norm(x_name, set(nodes))
        if norm is None:
            return False
        N, K = w.shape
        xr = self.aligned16(self.contiguous(norm["x"]), norm["x"])
        M = xr.numel // K
        if M > 32 or (M > 16 and K > 1536) or xr.numel != M * K:
            return False
        o = self.new_storage(out_name, out_shape, "bfloat16")
        bias = self.contiguous(b_name) if b_name else None
        wv2 = self.aligned16(self.contiguous(w2), w2)
        bv2 = self.contiguous(b2) if b2 else None
        kname = ("k_skinny_silu_norm_mt2_k1536" if M > 16 else
                 "k_skinny_silu_norm_mt1_k1536" if K <= 1536 else "k_skinny_silu_norm_mt1_k2048")
        args = dict(x=self.ref(xr), w=self.ref(w), bias=self.ref(bias) if bias else None, out=self.ref(o),
                    resid=None, w2=self.ref(wv2), bias2=self.ref(bv2) if bv2 else None,
                    norm_w=self.ref(self.aligned16(self.contiguous(norm["w"]), norm["w"])), argmax_slot=None,
                    attn_o=None, attn_ml=None, M=M, ldx=K, ldo=N, ldr=N, N=N, K=K, eps=float(norm["eps"]),
                    n_dtype=DTYPE_CODE[norm["n_dtype"]], flags=(1 if bias else 0) | (4 if bv2 else 0),
                    attn_heads=0, attn_kvh=0, attn_splits=0)
        tiles = -(-N // 8)
        self.emit(LaunchStep(
            kind="gemm", kernel=kname, module="gemv", arg_struct="GemvArgs", args=args,
            grid=(-(-tiles // SKINNY_NORM_WAVES), 1, 1), block=(64 * SKINNY_NORM_WAVES, 1, 1),
            inputs=[norm["x"], w_name, w2, norm["w"]] + [t for t in (b_name, b2) if t], outputs=[out_name],
            params={"M": M, "N": N, "K": K, "epilogue": "silu", "norm": True, "has_bias": bias is not None,
                    "weights": 2, "transpose_b": True, "nodes": nodes, "mfma": True, "skinny": True}))
        self.views[out_name] = o
        return True

    def emit_gemm(self, x_name: str, w_name: str, b_name: str | None, out_name: str, out_shape, dtype: str, *,
                  epi: str, nodes: list[str], resid: str | None = None, w2: str | None = None,
                  b2: str | None = None) -> None:
        """MFMA GEMM (csrc/kernels/gemm.hip) for M >= GEMM_MIN_M: out = epi(x . W^T); a pending
        RMSNorm of ``x`` is materialised first (it is cheap next to the GEMM). Up to SKINNY_MAX_M
        bf16 rows take the skinny kernels instead."""
        w = self.aligned16(self.contiguous(w_name), w_name)
        N, K = w.shape
        if (epi == "silu" and dtype == "bfloat16" and K % 64 == 0 and 512 <= K <= SKINNY_NORM_MAX_K and w2
                and self.emit_skinny_silu_norm(x_name, w, w_name, w2, b_name, b2, out_name, out_shape, nodes)):
            return
        x = self.aligned16(self.contiguous(x_name), x_name)
        M = x.numel // K
        o = self.new_storage(out_name, out_shape, dtype)
        bias = self.contiguous(b_name) if b_name else None
        r = self.contiguous(resid) if resid else None
        wv2 = self.aligned16(self.contiguous(w2), w2) if w2 else None
        bv2 = self.contiguous(b2) if b2 else None
        if (epi == "silu" and SKINNY_MAX_M < M <= WIDE_MAX_M and M <= 128 and dtype == "bfloat16"
                and K % 64 == 0 and K >= 512):
            # one workgroup of 4 waves per WIDE_TA tiles of 8 gate + 8 up rows, over every row
            args = dict(x=self.ref(x), w=self.ref(w), bias=self.ref(bias) if bias else None, out=self.ref(o),
                        resid=None, w2=self.ref(wv2), bias2=self.ref(bv2) if bv2 else None, norm_w=None,
                        argmax_slot=None, attn_o=None, attn_ml=None, M=M, ldx=K, ldo=N, ldr=N, N=N, K=K, eps=0.0,
                        n_dtype=0, flags=(1 if bias else 0) | (4 if bv2 else 0), attn_heads=0, attn_kvh=0,
                        attn_splits=0)
            groups = -(-N // (8 * WIDE_TA))
            if M > 64 and WIDE_HALVES:
                # two workgroups per tile group, 64 rows each; b and b + 8 share a group
                kname, grid = "k_wide_silu_mt4x2", (-(-groups // 8) * 16, 1, 1)
            else:
                kname, grid = f"k_wide_silu_mt{4 if M <= 64 else 8}", (groups, 1, 1)
            self.emit(LaunchStep(
                kind="gemm", kernel=kname, module="gemv", arg_struct="GemvArgs",
                args=args, grid=grid, block=(256, 1, 1),
                inputs=[x_name, w_name, w2] + [t for t in (b_name, b2) if t], outputs=[out_name],
                params={"M": M, "N": N, "K": K, "epilogue": epi, "has_bias": bias is not None, "weights": 2,
                        "transpose_b": True, "nodes": nodes, "mfma": True, "wide": True}))
            self.views[out_name] = o
            return
        if M <= SKINNY_MAX_M and dtype == "bfloat16" and K % 64 == 0 and K >= 512 and epi in ("bias", "resid", "silu"):
            # SiLU: one wave per tile of 8 gate + 8 up rows. Bias / residual: 8 waves per tile of
            # 16 output rows (8 when that gives fewer than 256 tiles), splitting K.
            mt = 1 if M <= 16 else 2
            if epi == "silu":
                per, kname, block = 8, f"k_skinny_silu_mt{mt}", 64
            else:
                per = 8 if -(-N // 16) < GEMM_TARGET_WGS else 16
                kname, block = f"k_skinny_{epi}_mt{mt}" + ("_r8" if per == 8 else ""), 512
            args = dict(x=self.ref(x), w=self.ref(w), bias=self.ref(bias) if bias else None, out=self.ref(o),
                        resid=self.ref(r) if r else None, w2=self.ref(wv2) if wv2 else None,
                        bias2=self.ref(bv2) if bv2 else None, norm_w=None, argmax_slot=None, attn_o=None,
                        attn_ml=None, M=M, ldx=K, ldo=N, ldr=N, N=N, K=K, eps=0.0, n_dtype=0,
                        flags=(1 if bias else 0) | (4 if bv2 else 0), attn_heads=0, attn_kvh=0, attn_splits=0)
            self.emit(LaunchStep(
                kind="gemm", kernel=kname, module="gemv", arg_struct="GemvArgs", args=args,
                grid=(-(-N // per), 1, 1), block=(block, 1, 1),
                inputs=[x_name, w_name] + [t for t in (b_name, resid, w2, b2) if t], outputs=[out_name],
                params={"M": M, "N": N, "K": K, "epilogue": epi, "has_bias": bias is not None,
                        "weights": 2 if epi == "silu" else 1, "transpose_b": True, "nodes": nodes, "mfma": True,
                        "skinny": True}))
            self.views[out_name] = o
            return
        nw = 2 if epi == "silu" else 1
        bm, bn, ksplit, dma = gemm_tiling(M, N, K, nw)
        bk = 64 if K % 64 == 0 else 32
        kchunk = K
        if ksplit > 1:
            kchunk = ((K // bk + ksplit - 1) // ksplit) * bk
            ksplit = (K + kchunk - 1) // kchunk
        dt = "bf16" if dtype == "bfloat16" else "f16"
        part = self.scratch(out_name + ".kpart", ksplit * nw * M * N * 4) if ksplit > 1 else None
        args = dict(x=self.ref(x), w=self.ref(w), w2=self.ref(wv2) if wv2 else None,
                    bias=self.ref(bias) if bias else None, bias2=self.ref(bv2) if bv2 else None,
                    resid=self.ref(r) if r else None, out=self.ref(o), part=part, M=M, ldx=K, ldw=K, ldo=N, ldr=N,
                    sx=0, sw=0, so=0, batch=1, bdiv=1,
                    N=N, K=K, flags=(1 if bias else 0) | (2 if bv2 else 0), ksplit=ksplit, kchunk=kchunk, nw=nw)
        ins = [x_name, w_name] + [t for t in (b_name, resid, w2, b2) if t]
        params = {"M": M, "N": N, "K": K, "epilogue": epi, "has_bias": bias is not None, "weights": nw,
                  "transpose_b": True, "nodes": nodes, "mfma": True, "tile": (bm, bn), "ksplit": ksplit, "bk": bk,
                  "lds_direct": dma}
        self.emit(LaunchStep(
            kind="gemm", kernel=f"k_gemm_{dt}_{epi}_m{bm}n{bn}" + ("_k64d" if dma else "_k64" if bk == 64 else ""),
            module="gemm",
            arg_struct="GemmArgs", args=args,
            grid=((N + bn - 1) // bn, (M + bm - 1) // bm, ksplit), inputs=ins,
            outputs=[out_name + ".kpart" if ksplit > 1 else out_name], params=params))
        if ksplit > 1:
            self.emit(LaunchStep(
                kind="gemm", kernel=f"k_gemm_reduce_{dt}_{epi}", module="gemm", arg_struct="GemmArgs",
                args=dict(args), grid=grid1d(M * N), inputs=[out_name + ".kpart"] + ins[2:], outputs=[out_name],
                params=dict(params, reduce=True)))
        self.views[out_name] = o

    def emit_linear(self, x_name: str, w_name: str, b_name: str | None, out_name: str, out_shape, out_dtype: str,
                    resid: str | None, node_names: list[str]) -> None:
        x = self.contiguous(x_name)
        w = self.contiguous(w_name)
        K = x.shape[-1]
        N = w.shape[0]
        M = x.numel // K if K else 0
        ok = (x.dtype == w.dtype == out_dtype and x.dtype in ("bfloat16", "float16") and K % 8 == 0
              and (x.offset * 2) % 16 == 0 and (w.offset * 2) % 16 == 0)
        if b_name is not None:
            ok = ok and self.view(b_name).dtype == out_dtype
        if not ok:
            self.emit_linear_generic(x, w, b_name, out_name, out_shape, out_dtype, node_names)
            if resid is not None:
                raise NotImplementedError("residual epilogue on the generic path")
            return
        if M >= GEMM_MIN_M and K % 32 == 0 or skinny_rows(M, K, out_dtype):
            self.emit_gemm(x_name, w_name, b_name, out_name, out_shape, out_dtype,
                           epi="resid" if resid is not None else "bias", nodes=node_names, resid=resid)
            return
        o = self.new_storage(out_name, out_shape, out_dtype)
        bias = self.contiguous(b_name) if b_name is not None else None
        r = self.contiguous(resid) if resid is not None else None
        mb, rpw = (1, 4) if M <= 1 else (4, 2)
        kname = f"k_linear_{'bf16' if out_dtype == 'bfloat16' else 'f16'}_m{mb}"
        self.emit(LaunchStep(
            kind="gemm", kernel=kname, module="linear", arg_struct="LinearArgs",
            args=dict(x=self.ref(x), w=self.ref(w), bias=self.ref(bias) if bias else None, out=self.ref(o),
                      resid=self.ref(r) if r else None, M=M, ldx=K, ldo=N, ldr=N, N=N, K=K,
                      dtype=DTYPE_CODE[out_dtype], has_bias=int(bias is not None), has_resid=int(r is not None)),
            grid=((N + 4 * rpw - 1) // (4 * rpw), (M + mb - 1) // mb, 1),
            inputs=[x_name, w_name] + ([b_name] if b_name else []) + ([resid] if resid else []),
            outputs=[out_name], params={"M": M, "N": N, "K": K, "has_bias": bias is not None,
                                        "transpose_b": True, "nodes": node_names}))
        self.views[out_name] = o

    def emit_linear_generic(self, x: TView, w: TView, b_name, out_name, out_shape, out_dtype, node_names) -> None:
        K = x.shape[-1]
        M = x.numel // K
        N = w.shape[0]
        xm = V.restride(x, (M, K))
        wt = V.transpose(w, 0, 1)  # [K, N]
        tmp_name = out_name if b_name is None else out_name + ".mm"
        o = self.new_storage(tmp_name, (M, N), out_dtype)
        self.emit_bmm(xm, wt, o, [], [out_name])
        res = V.restride(o, out_shape)
        self.views[tmp_name] = res
        if b_name is not None:
            self.chains.pop(tmp_name, None)
            ch = _Chain(shape=tuple(out_shape), dtype=out_dtype)
            ch.ext = [res, V.broadcast_to(self.view(b_name), tuple(out_shape))]
            ch.ext_names = [tmp_name, b_name]
            ch.ops = [ChainOp("aten.add.Tensor", [("ext", 0), ("ext", 1)], out_dtype, {})]
            ch.tail = out_name
            ch.node_names = list(node_names)
            self.chains[out_name] = ch
            self.flush_chain(out_name)
        else:
            self.views[out_name] = res

    def emit_bmm(self, a: TView, b: TView, c: TView, ins: list[str], outs: list[str]) -> None:
        """c[..., M, N] = a[..., M, K] @ b[..., K, N] with broadcast batch dims (generic kernel)."""
        M, K = a.shape[-2], a.shape[-1]
        N = b.shape[-1]
        batch = tuple(c.shape[:-2])
        if len(batch) > 4:
            raise NotImplementedError("matmul batch rank > 4")
        ab = V.broadcast_to(a.with_(shape=a.shape[:-2], strides=a.strides[:-2]), batch) if batch else None
        bb = V.broadcast_to(b.with_(shape=b.shape[:-2], strides=b.strides[:-2]), batch) if batch else None
        pad = 4 - len(batch)
        self.emit(LaunchStep(
            kind="gemm_batched", kernel="k_bmm", module="basic", arg_struct="BmmArgs",
            args=dict(a=self.ref(a), b=self.ref(b), c=self.ref(c),
                      batch_shape=list(batch) + [1] * pad,
                      a_bstride=(list(ab.strides) if ab else []) + [0] * pad,
                      b_bstride=(list(bb.strides) if bb else []) + [0] * pad,
                      M=M, N=N, K=K, a_sm=a.strides[-2], a_sk=a.strides[-1], b_sk=b.strides[-2],
                      b_sn=b.strides[-1], nbatch=len(batch), a_dtype=DTYPE_CODE[a.dtype],
                      b_dtype=DTYPE_CODE[b.dtype], c_dtype=DTYPE_CODE[c.dtype]),
            grid=grid1d(c.numel), inputs=ins, outputs=outs,
            params={"batch": numel(batch), "M": M, "N": N, "K": K}))

    def lower_matmul(self, node: OpNode) -> None:
        a = self.view(node.inputs[0].name)
        b = self.view(node.inputs[1].name)
        out = node.outputs[0]
        sq_a = len(a.shape) == 1
        sq_b = len(b.shape) == 1
        if sq_a:
            a = a.with_(shape=(1,) + a.shape, strides=(0,) + a.strides)
        if sq_b:
            b = b.with_(shape=b.shape + (1,), strides=b.strides + (0,))
        full = tuple(out.shape)
        if sq_a:
            full = full[:-1] + (1, full[-1]) if len(full) else (1, 1)
        if sq_b:
            full = full + (1,)
        o = self.new_storage(out.name, full, out.dtype)
        if not (sq_a or sq_b) and self.emit_batched_gemm(a, b, o, [t.name for t in node.inputs], [out.name]):
            self.views[out.name] = V.restride(o, out.shape)
            return
        self.emit_bmm(a, b, o, [t.name for t in node.inputs], [out.name])
        self.views[out.name] = V.restride(o, out.shape)

    @staticmethod
    def _linear_batch_stride(shape, strides) -> int | None:
        """s such that the batch element with flat index b starts at b * s, or None."""
        s, span = None, 1
        for n, st in zip(reversed(shape), reversed(strides)):
            if n > 1:
                if s is None:
                    s = st // span if span else 0
                    if s * span != st:
                        return None
                elif st != s * span:
                    return None
            span *= n
        return s or 0

    def emit_batched_gemm(self, a: TView, b: TView, c: TView, ins: list[str], outs: list[str]) -> bool:
        """Batched c = a @ b on the MFMA GEMM when the layout allows it (bf16/fp16, K % 32 == 0,
        K-contiguous a, b either [N, K]- or [K, N]-contiguous, batch offsets linear in the flat
        batch index); returns False to leave the matmul to the generic kernel."""
        M, K, N = a.shape[-2], a.shape[-1], b.shape[-1]
        dt = c.dtype
        if not (a.dtype == b.dtype == dt and dt in ("bfloat16", "float16") and K % 32 == 0 and M * N >= 4096):
            return False
        if a.strides[-1] != 1 or a.strides[-2] % 8 or (a.offset * 2) % 16 or (b.offset * 2) % 16:
            return False
        if b.strides[-2] == 1 and b.strides[-1] % 8 == 0:
            kn, ldw = False, b.strides[-1]
        elif b.strides[-1] == 1 and b.strides[-2] % 8 == 0 and N % 8 == 0:
            kn, ldw = True, b.strides[-2]
        else:
            return False
        batch = tuple(c.shape[:-2])
        nb = numel(batch)
        ab = V.broadcast_to(a.with_(shape=a.shape[:-2], strides=a.strides[:-2]), batch) if batch else None
        bb = V.broadcast_to(b.with_(shape=b.shape[:-2], strides=b.strides[:-2]), batch) if batch else None
        sx = self._linear_batch_stride(batch, ab.strides) if batch else 0
        sw = self._linear_batch_stride(batch, bb.strides) if batch else 0
        if sx is None or sw is None or sx % 8 or sw % 8:
            return False
        tiles = [(128, 128), (64, 64)]
        for bm, bn in tiles:
            if ((M + bm - 1) // bm) * ((N + bn - 1) // bn) * nb >= GEMM_TARGET_WGS:
                break
        bk = 64 if K % 64 == 0 else 32
        name = (f"k_gemm_{'bf16' if dt == 'bfloat16' else 'f16'}_bias_m{bm}n{bn}" + ("_kn" if kn else "") +
                ("_k64" if bk == 64 else ""))
        args = dict(x=self.ref(a), w=self.ref(b), w2=None, bias=None, bias2=None, resid=None, out=self.ref(c),
                    part=None, M=M, ldx=a.strides[-2], ldw=ldw, ldo=N, ldr=N, sx=sx, sw=sw, so=M * N, batch=nb,
                    bdiv=1, N=N, K=K, flags=0, ksplit=1, kchunk=K, nw=1)
        self.emit(LaunchStep(
            kind="gemm", kernel=name, module="gemm", arg_struct="GemmArgs", args=args,
            grid=((N + bn - 1) // bn, (M + bm - 1) // bm, nb), inputs=ins, outputs=outs,
            params={"M": M, "N": N, "K": K, "batch": nb, "epilogue": "bias", "weights": 1, "mfma": True,
                    "tile": (bm, bn), "ksplit": 1, "bk": bk, "b_layout": "kn" if kn else "nk"}))
        return True

    def lower_addmm(self, node: OpNode) -> None:
        bias, m1, m2 = (t.name for t in node.inputs[:3])
        out = node.outputs[0]
        beta = float(node.attrs.get("beta", 1))
        alpha = float(node.attrs.get("alpha", 1))
        w2 = self.view(m2)
        if beta == 1 and alpha == 1 and len(w2.shape) == 2 and w2.strides == (1, w2.shape[0]):
            # mat2 is W^T of a contiguous W[N, K]
            wname = m2 + ".T"
            self.views[wname] = V.transpose(w2, 0, 1)
            self.emit_linear(m1, wname, bias, out.name, tuple(out.shape), out.dtype, None, [node.name])
            return
        a, b = self.view(m1), self.view(m2)
        o = self.new_storage(out.name + ".mm", out.shape, out.dtype)
        self.emit_bmm(a, b, o, [m1, m2], [out.name + ".mm"])
        self.views[out.name + ".mm"] = o
        ch = _Chain(shape=tuple(out.shape), dtype=out.dtype)
        ch.ext = [o, V.broadcast_to(self.view(bias), tuple(out.shape))]
        ch.ext_names = [out.name + ".mm", bias]
        ch.ops = [ChainOp("aten.mul.Tensor", [("ext", 0), ("scalar", alpha)], out.dtype, {}),
                  ChainOp("aten.add.Tensor", [("val", 0), ("ext", 1)], out.dtype, {"alpha": beta})]
        ch.tail = out.name
        ch.node_names = [node.name]
        self.chains[out.name] = ch

    def emit_softmax(self, x_name: str, mask_name: str | None, add_dtype: str, out_name: str, out_shape,
                     out_dtype: str, node_names: list[str]) -> None:
        x = self.view(x_name)
        if x.strides[-1] != 1:
            x = self.contiguous(x_name, x)
        shape = tuple(x.shape)
        cols = shape[-1]
        rows = x.numel // cols if cols else 0
        lead = list(shape[:-1])
        if len(lead) > 5:
            raise NotImplementedError("softmax rank > 6")
        xs = list(x.strides[:-1])
        margs = dict(mask=None, mask_lead_stride=[0] * 5, mask_col_stride=0, mask_dtype=0, has_mask=0)
        if mask_name is not None:
            m = V.broadcast_to(self.view(mask_name), shape)
            margs = dict(mask=self.ref(m), mask_lead_stride=list(m.strides[:-1]) + [0] * (5 - len(lead)),
                         mask_col_stride=m.strides[-1], mask_dtype=DTYPE_CODE[m.dtype], has_mask=1)
        o = self.new_storage(out_name, out_shape, out_dtype)
        self.emit(LaunchStep(
            kind="softmax", kernel="k_softmax", module="basic", arg_struct="SoftmaxArgs",
            args=dict(x=self.ref(x), out=self.ref(o), rows=rows, cols=cols,
                      lead_shape=lead + [1] * (5 - len(lead)), x_lead_stride=xs + [0] * (5 - len(lead)),
                      nlead=len(lead), x_dtype=DTYPE_CODE[x.dtype], add_dtype=DTYPE_CODE[add_dtype],
                      out_dtype=DTYPE_CODE[out_dtype], **margs),
            grid=(max(rows, 1), 1, 1), inputs=[x_name] + ([mask_name] if mask_name else []), outputs=[out_name],
            params={"rows": rows, "cols": cols, "masked": mask_name is not None, "nodes": node_names}))
        self.views[out_name] = o

    def lower_softmax(self, node: OpNode) -> None:
        x = node.inputs[0]
        out = node.outputs[0]
        dim = int(node.attrs.get("dim", -1)) % len(x.shape)
        if dim != len(x.shape) - 1:
            v = self.view(x.name)
            perm = [d for d in range(len(x.shape)) if d != dim] + [dim]
            pv = V.permute(v, perm)
            self.views[x.name + ".perm"] = pv
            self.emit_softmax(x.name + ".perm", None, x.dtype, out.name + ".perm", pv.shape, out.dtype, [node.name])
            inv = [perm.index(d) for d in range(len(perm))]
            self.views[out.name] = V.permute(self.views[out.name + ".perm"], inv)
            return
        self.emit_softmax(x.name, None, x.dtype, out.name, tuple(out.shape), out.dtype, [node.name])

    def lower_mean(self, node: OpNode) -> None:
        x = node.inputs[0]
        out = node.outputs[0]
        nd = len(x.shape)
        dims = node.attrs.get("dim", None)
        dims = list(range(nd)) if dims is None else ([dims] if isinstance(dims, int) else list(dims))
        dims = sorted(d % nd for d in dims)
        keep = [d for d in range(nd) if d not in dims]
        v = self.view(x.name)
        pv = V.permute(v, keep + dims)
        pv = self.contiguous(x.name, pv) if not pv.is_contiguous() else pv
        cols = numel([x.shape[d] for d in dims])
        rows = pv.numel // cols
        o = self.new_storage(out.name, out.shape, out.dtype)
        self.emit(mean_rows_step(self.ref(pv), self.ref(o), rows, cols, pv.dtype, out.dtype, [x.name], [out.name]))
        self.views[out.name] = o

    # ------------------------------------------------------------------ convolution network ops

    def emit_conv(self, conv: OpNode, out_name: str, *, bn: OpNode | None = None, resid: str | None = None,
                  relu: bool = False, nodes: list[str] | None = None) -> None:
        """conv2d (+ batch norm) (+ residual add) (+ ReLU) as one implicit-GEMM launch.

        Channels-last (NHWC) activations with Cin % 64 == 0 go to the MFMA GEMM (gemm.hip, conv
        epilogue): 16-byte channel loads and direct-to-LDS staging instead of 2-byte gathers.
        Otherwise conv.hip's NCHW kernel runs (e.g. the 3-channel stem), writing its output
        channels-last when the channels suit the GEMM path downstream."""
        xv = self.view(conv.inputs[0].name)
        if self.conv_nhwc and _is_nhwc(xv) and xv.shape[1] % 64 == 0 and xv.dtype in ("float16", "bfloat16") \
                and (xv.offset * 2) % 16 == 0:
            return self.emit_conv_nhwc(conv, out_name, xv, bn=bn, resid=resid, relu=relu, nodes=nodes)
        wv0 = self.view(conv.inputs[1].name)
        if self.conv_nhwc and len(xv.shape) == 4 and xv.shape[1] <= 4 and xv.dtype in ("float16", "bfloat16") \
                and wv0.dtype == xv.dtype and wv0.shape[0] % 8 == 0 and wv0.shape[2] <= 16 and wv0.shape[3] <= 16:
            return self.emit_conv_stem(conv, out_name, bn=bn, resid=resid, relu=relu, nodes=nodes)
        x = self.contiguous(conv.inputs[0].name)
        w = self.contiguous(conv.inputs[1].name)
        has_bias = len(conv.inputs) > 2
        N, Cin, H, W = x.shape
        Cout, _, KH, KW = w.shape
        out_t = conv.outputs[0]
        Ho, Wo = out_t.shape[2], out_t.shape[3]
        st = conv.attrs.get("stride", [1, 1])
        pd = conv.attrs.get("padding", [0, 0])
        st = [st, st] if isinstance(st, int) else list(st)
        pd = [pd, pd] if isinstance(pd, int) else list(pd)
        K = Cin * KH * KW
        dt = x.dtype
        bnv = [self.contiguous(t.name) for t in bn.inputs[1:5]] if bn is not None else [None] * 4
        M = N * Ho * Wo
        tiles = ((Cout + 127) // 128) * ((M + 127) // 128)
        # channels-last output (flag 16) when the next convolutions can take the GEMM path
        nhwc_out = (self.conv_nhwc and Cout % 64 == 0 and dt in ("float16", "bfloat16")
                    and not (tiles < 256 and K >= 1024) and (resid is None or _is_nhwc(self.view(resid))))
        if nhwc_out:
            ob = self.new_storage(out_name, [N, Ho, Wo, Cout], dt)
            o = ob.with_(shape=(N, Cout, Ho, Wo), strides=(Ho * Wo * Cout, 1, Wo * Cout, Cout))
            rv = self.view(resid) if resid else None
        else:
            o = ob = self.new_storage(out_name, [N, Cout, Ho, Wo], dt)
            rv = self.contiguous(resid) if resid else None
        flags = (1 if has_bias else 0) | (2 if bn is not None else 0) | (4 if rv is not None else 0) | (8 if relu else 0) \
            | (16 if nhwc_out else 0)
        vec = K % 8 == 0 and (w.offset * 2) % 16 == 0
        kname = f"k_conv_{'bf16' if dt == 'bfloat16' else 'f16'}" + ("" if vec else "_g")
        if vec and KH == KW == 1 and pd == [0, 0] and K % 32 == 0:
            kname += "_1x1"
        elif vec and KH == KW == 3:
            kname += "_3x3"
        if M + 256 >= 2 ** 31 or x.numel * 2 >= 2 ** 32:
            raise NotImplementedError("conv2d with 2^31 or more input elements or output pixels")
        ins = [conv.inputs[0].name, conv.inputs[1].name] + ([conv.inputs[2].name] if has_bias else []) + \
            ([t.name for t in bn.inputs[1:5]] if bn is not None else []) + ([resid] if resid else [])
        # few 128 x 128 tiles (small images deep in the network) and long K: split K across
        # workgroups (fp32 partials, then k_conv_reduce_* applies the epilogue). Measured at batch 32:
        # 3x3 512 -> 512 on 7 x 7 (52 tiles, K = 4608) 257 -> 65 us, 1x1 2048 -> 512 73 -> 33 us,
        # 3x3 128 -> 128 on 28 x 28 (196 tiles, K = 1152) 74 -> 67 us; at K = 512 the reduce pass
        # costs more than the split gains (1x1 512 -> 128 on 28 x 28: 26 -> 29 us), hence K >= 1024
        ksplit, kchunk = 1, K
        if tiles < 256 and K >= 1024 and M % 4 == 0:   # the reduce reads 4 pixels per load
            ksplit = max(1, min(8, (384 + tiles - 1) // tiles, K // 256))
            kchunk = ((K + 31) // 32 + ksplit - 1) // ksplit * 32
            ksplit = (K + kchunk - 1) // kchunk
        part = self.scratch(out_name + ".kpart", ksplit * Cout * M * 4) if ksplit > 1 else None
        args = dict(x=self.ref(x), w=self.ref(w), bias=self.ref(self.contiguous(conv.inputs[2].name)) if has_bias
                    else None, bn_w=self.ref(bnv[0]) if bn is not None else None,
                    bn_b=self.ref(bnv[1]) if bn is not None else None,
                    bn_mean=self.ref(bnv[2]) if bn is not None else None,
                    bn_var=self.ref(bnv[3]) if bn is not None else None,
                    resid=self.ref(rv) if rv is not None else None, out=self.ref(ob), part=part, M=M, N=N, Cin=Cin,
                    H=H, W=W, Cout=Cout, Ho=Ho, Wo=Wo, KH=KH, KW=KW, sh=st[0], sw=st[1], ph=pd[0], pw=pd[1], K=K,
                    eps=float(bn.attrs.get("eps", 1e-5)) if bn is not None else 0.0, flags=flags, ksplit=ksplit,
                    kchunk=kchunk)
        params = {"M": M, "N": Cout, "K": K, "kernel": [KH, KW], "stride": st, "padding": pd,
                  "batch_norm": bn is not None, "residual": rv is not None, "relu": relu, "mfma": True,
                  "ksplit": ksplit, "nhwc_out": nhwc_out, "nodes": nodes or [conv.name]}
        self.emit(LaunchStep(
            kind="conv", kernel=kname, module="conv", arg_struct="ConvArgs", args=args,
            grid=((Cout + 127) // 128, (M + 127) // 128, ksplit), inputs=ins,
            outputs=[out_name + ".kpart" if ksplit > 1 else out_name], params=params))
        if ksplit > 1:
            self.emit(LaunchStep(
                kind="conv", kernel=f"k_conv_reduce_{'bf16' if dt == 'bfloat16' else 'f16'}", module="conv",
                arg_struct="ConvArgs", args=dict(args), grid=grid1d(Cout * M // 4),
                inputs=[out_name + ".kpart"] + ins[2:], outputs=[out_name], params=dict(params, reduce=True)))
        self.views[out_name] = o

    def emit_conv_nhwc(self, conv: OpNode, out_name: str, xv: TView, *, bn: OpNode | None, resid: str | None,
                       relu: bool, nodes: list[str] | None) -> None:
        """conv2d on an NHWC image as an MFMA GEMM over [pixels, KH*KW*Cin] x [Cout, KH*KW*Cin]^T with
        the conv epilogue; writes NHWC. 1 x 1 / stride 1 / no padding reads the image rows as they
        are (_conv); other shapes gather one tap and 64 channels per K step (_convg, padded taps
        read a zeroed buffer). Weights [Cout, Cin, KH, KW] are read as [Cout, KH, KW, Cin]: a
        strided copy for KH*KW > 1 at the start of each run (bound weights can change between runs)."""
        wname = conv.inputs[1].name
        wv = self.view(wname)
        has_bias = len(conv.inputs) > 2
        N, Cin, H, W = xv.shape
        Cout, _, KH, KW = wv.shape
        out_t = conv.outputs[0]
        Ho, Wo = out_t.shape[2], out_t.shape[3]
        st = conv.attrs.get("stride", [1, 1])
        pd = conv.attrs.get("padding", [0, 0])
        st = [st, st] if isinstance(st, int) else list(st)
        pd = [pd, pd] if isinstance(pd, int) else list(pd)
        dt = xv.dtype
        K = KH * KW * Cin
        M = N * Ho * Wo
        if M + 256 >= 2 ** 31 or xv.numel >= 2 ** 31:
            raise NotImplementedError("conv2d with 2^31 or more input elements or output pixels")
        if KH * KW > 1:
            key = wname + ".ohwi"
            w = self.views.get(key)
            if w is None:
                w = self.new_storage(key, [Cout, KH, KW, Cin], dt)
                ent = (wname, wv, w, (Cin, KH, KW), (Cin, KH, KW))
                if self.is_constant(wv) and wv.is_contiguous():
                    self._ohwi.append(ent)   # one launch at the program start
                else:
                    self.emit(self._permute_step([ent]))
                self.views[key] = w
        else:
            w = self.aligned16(self.contiguous(wname), wname)
        plain = KH == KW == 1 and st == [1, 1] and pd == [0, 0]
        ob = self.new_storage(out_name, [N, Ho, Wo, Cout], dt)
        o = ob.with_(shape=(N, Cout, Ho, Wo), strides=(Ho * Wo * Cout, 1, Wo * Cout, Cout))
        rv = None
        if resid is not None:
            rv = self.view(resid)
            if not _is_nhwc(rv) or (rv.offset * 2) % 16:
                rb = self.new_storage(resid + ".nhwc", [rv.shape[0], rv.shape[2], rv.shape[3], rv.shape[1]], dt)
                rn = rb.with_(shape=rv.shape, strides=(rb.strides[0], 1, rb.strides[1], rb.strides[2]))
                self.emit_copy(rv, rn, [resid], [resid + ".nhwc"])
                rv = rb
        bnv = [self.contiguous(t.name) for t in bn.inputs[1:5]] if bn is not None else [None] * 4
        flags = (1 if has_bias else 0) | (2 if bn is not None else 0) | (4 if rv is not None else 0) | (8 if relu else 0)
        if CONV_NFAST and xv.numel > Cout * K:   # input larger than the weights: N tiles fastest
            flags |= 16
        bm, bn_, ksplit = conv_gemm_tiling(M, Cout, K)
        # always direct-to-LDS; K up to 1024 (at most 16 steps, where the pipeline depth buys little)
        # takes the 2-stage variant, whose smaller LDS footprint lets more workgroups share a CU
        # (the 56 x 56 3 x 3 convs, K = 576: 28 -> 25.5 us)
        stages = "d2" if K <= CONV_D2_MAX_K else "d"
        if plain and K <= CONV_D1_MAX_K and (bm, bn_) == (64, 64) and ksplit == 1:
            stages = "d1"   # few K steps: one stage of LDS (16 KB), up to eight workgroups per CU
        kchunk = K
        if ksplit > 1:
            kchunk = ((K // 64 + ksplit - 1) // ksplit) * 64
            ksplit = (K + kchunk - 1) // kchunk
        if self._conv_zero is None:
            self._conv_zero = self.scratch("conv.zero", 256, persistent=True)
        dts = "bf16" if dt == "bfloat16" else "f16"
        kname = f"k_gemm_{dts}_{'conv' if plain else 'convg'}_m{bm}n{bn_}_k64{stages}"
        part = self.scratch(out_name + ".kpart", ksplit * M * Cout * 4) if ksplit > 1 else None
        args = dict(x=self.ref(xv), w=self.ref(w), w2=None, bias=self.ref(self.contiguous(conv.inputs[2].name))
                    if has_bias else None, bias2=None, resid=self.ref(rv) if rv is not None else None,
                    out=self.ref(ob), part=part, M=M, ldx=Cin, ldw=K, ldo=Cout, ldr=Cout, sx=0, sw=0, so=0, batch=1,
                    bdiv=1, N=Cout, K=K, flags=flags, ksplit=ksplit, kchunk=kchunk, nw=1,
                    bn_w=self.ref(bnv[0]) if bn is not None else None,
                    bn_b=self.ref(bnv[1]) if bn is not None else None,
                    bn_mean=self.ref(bnv[2]) if bn is not None else None,
                    bn_var=self.ref(bnv[3]) if bn is not None else None,
                    zero=self._conv_zero, eps=float(bn.attrs.get("eps", 1e-5)) if bn is not None else 0.0,
                    cH=H, cW=W, cCin=Cin, cHo=Ho, cWo=Wo, cKW=KW, csh=st[0], csw=st[1], cph=pd[0], cpw=pd[1])
        ins = [conv.inputs[0].name, wname] + ([conv.inputs[2].name] if has_bias else []) + \
            ([t.name for t in bn.inputs[1:5]] if bn is not None else []) + ([resid] if resid else [])
        params = {"M": M, "N": Cout, "K": K, "kernel": [KH, KW], "stride": st, "padding": pd,
                  "batch_norm": bn is not None, "residual": rv is not None, "relu": relu, "mfma": True,
                  "ksplit": ksplit, "nhwc": True, "tile": (bm, bn_), "lds_direct": True, "stages": stages,
                  "nodes": nodes or [conv.name]}
        self.emit(LaunchStep(
            kind="conv", kernel=kname, module="gemm", arg_struct="GemmArgs", args=args,
            grid=((Cout + bn_ - 1) // bn_, (M + bm - 1) // bm, ksplit), inputs=ins,
            outputs=[out_name + ".kpart" if ksplit > 1 else out_name], params=params))
        if ksplit > 1:
            self.emit(LaunchStep(
                kind="conv", kernel=f"k_gemm_reduce_{dts}_conv", module="gemm", arg_struct="GemmArgs",
                args=dict(args), grid=grid1d(M * Cout), inputs=[out_name + ".kpart"] + ins[2:],
                outputs=[out_name], params=dict(params, reduce=True)))
        self.views[out_name] = o

    def emit_conv_stem(self, conv: OpNode, out_name: str, *, bn: OpNode | None, resid: str | None, relu: bool,
                       nodes: list[str] | None) -> None:
        """A conv on an image of at most 4 channels (a network's first layer, e.g. ResNet's 7 x 7 / 2 on
        RGB): the image is written once per run as a zero-bordered channels-last [N, Hp, Wp, 4] buffer
        (k_pad_nhwc4), the weights as [Cout, KHp, KWp, 4] with zeros past the kernel (KWp even, so a
        16-byte chunk is two neighbouring taps), and the _convp GEMM reads every tap in bounds with
        no checks. K = KHp * KWp * 4 (256 for 7 x 7) instead of 2-byte gathers over K = 147."""
        x = self.contiguous(conv.inputs[0].name)
        wname = conv.inputs[1].name
        wv = self.view(wname)
        has_bias = len(conv.inputs) > 2
        N, C, H, W = x.shape
        Cout, _, KH, KW = wv.shape
        Ho, Wo = conv.outputs[0].shape[2], conv.outputs[0].shape[3]
        st = conv.attrs.get("stride", [1, 1])
        pd = conv.attrs.get("padding", [0, 0])
        st = [st, st] if isinstance(st, int) else list(st)
        pd = [pd, pd] if isinstance(pd, int) else list(pd)
        dt = x.dtype
        kwp = KW + (KW & 1)
        khp = KH
        while (khp * kwp * 4) % 64:
            khp += 1
        K = khp * kwp * 4
        Hp = max(H + 2 * pd[0], (Ho - 1) * st[0] + khp)
        Wp = max(W + 2 * pd[1], (Wo - 1) * st[1] + kwp)
        M = N * Ho * Wo
        if M + 256 >= 2 ** 31 or N * Hp * Wp * 4 >= 2 ** 31:
            raise NotImplementedError("conv2d with 2^31 or more padded input elements or output pixels")
        xp = self.new_storage(conv.inputs[0].name + ".pad4", [N, Hp, Wp, 4], dt)
        self.emit(LaunchStep(
            kind="copy", kernel="k_pad_nhwc4", module="conv", arg_struct="PadNHWCArgs",
            args=dict(x=self.ref(x), out=self.ref(xp), n=N, C=C, H=H, W=W, Hp=Hp, Wp=Wp, top=pd[0], left=pd[1], pad=0),
            grid=grid1d(N * Hp * Wp), inputs=[conv.inputs[0].name], outputs=[xp.storage],
            params={"padded": [Hp, Wp]}))
        key = wname + ".pad4"
        w = self.views.get(key)
        if w is None:
            w = self.new_storage(key, [Cout, khp, kwp, 4], dt)
            ent = (wname, wv, w, (C, KH, KW), (4, khp, kwp))
            if self.is_constant(wv) and wv.is_contiguous():
                self._ohwi.append(ent)
            else:
                self.emit(self._permute_step([ent] if wv.is_contiguous() else [(wname, self.contiguous(wname), w,
                                                                                 (C, KH, KW), (4, khp, kwp))]))
            self.views[key] = w
        ob = self.new_storage(out_name, [N, Ho, Wo, Cout], dt)
        o = ob.with_(shape=(N, Cout, Ho, Wo), strides=(Ho * Wo * Cout, 1, Wo * Cout, Cout))
        rv = None
        if resid is not None:
            rv = self.view(resid)
            if not _is_nhwc(rv):
                rb = self.new_storage(resid + ".nhwc", [rv.shape[0], rv.shape[2], rv.shape[3], rv.shape[1]], dt)
                self.emit_copy(rv, rb.with_(shape=rv.shape, strides=(rb.strides[0], 1, rb.strides[1], rb.strides[2])),
                               [resid], [resid + ".nhwc"])
                rv = rb
        bnv = [self.contiguous(t.name) for t in bn.inputs[1:5]] if bn is not None else [None] * 4
        flags = (1 if has_bias else 0) | (2 if bn is not None else 0) | (4 if rv is not None else 0) | (8 if relu else 0)
        bm, bn_, _ = conv_gemm_tiling(M, Cout, K)
        dts = "bf16" if dt == "bfloat16" else "f16"
        args = dict(x=self.ref(xp), w=self.ref(w), w2=None, bias=self.ref(self.contiguous(conv.inputs[2].name))
                    if has_bias else None, bias2=None, resid=self.ref(rv) if rv is not None else None,
                    out=self.ref(ob), part=None, M=M, ldx=0, ldw=K, ldo=Cout, ldr=Cout, sx=0, sw=0, so=0, batch=1,
                    bdiv=1, N=Cout, K=K, flags=flags, ksplit=1, kchunk=K, nw=1,
                    bn_w=self.ref(bnv[0]) if bn is not None else None,
                    bn_b=self.ref(bnv[1]) if bn is not None else None,
                    bn_mean=self.ref(bnv[2]) if bn is not None else None,
                    bn_var=self.ref(bnv[3]) if bn is not None else None,
                    zero=None, eps=float(bn.attrs.get("eps", 1e-5)) if bn is not None else 0.0,
                    cH=Hp, cW=Wp, cCin=4, cHo=Ho, cWo=Wo, cKW=kwp, csh=st[0], csw=st[1], cph=0, cpw=0)
        ins = [conv.inputs[0].name, wname] + ([conv.inputs[2].name] if has_bias else []) + \
            ([t.name for t in bn.inputs[1:5]] if bn is not None else []) + ([resid] if resid else [])
        self.emit(LaunchStep(
            kind="conv", kernel=f"k_gemm_{dts}_convp_m{bm}n{bn_}_k64d2", module="gemm", arg_struct="GemmArgs",
            args=args, grid=((Cout + bn_ - 1) // bn_, (M + bm - 1) // bm, 1), inputs=ins, outputs=[out_name],
            params={"M": M, "N": Cout, "K": K, "kernel": [KH, KW], "stride": st, "padding": pd,
                    "batch_norm": bn is not None, "residual": rv is not None, "relu": relu, "mfma": True,
                    "ksplit": 1, "nhwc": True, "tile": (bm, bn_), "lds_direct": True, "stages": "d2",
                    "padded_taps": [khp, kwp, 4], "K_alg": C * KH * KW, "nodes": nodes or [conv.name]}))
        self.views[out_name] = o

    def lower_conv2d(self, node: OpNode) -> None:
        self.emit_conv(node, node.outputs[0].name)

    def lower_batch_norm(self, node: OpNode) -> None:
        x = self.contiguous(node.inputs[0].name)
        out = node.outputs[0]
        ps = [self.contiguous(t.name) for t in node.inputs[1:5]]
        if len({p.dtype for p in ps}) != 1 or out.dtype != x.dtype:
            raise NotImplementedError("batch_norm: weight, bias, mean and var of one dtype, output of the input's")
        o = self.new_storage(out.name, out.shape, out.dtype)
        hw = numel(x.shape[2:]) if len(x.shape) > 2 else 1
        self.emit(LaunchStep(
            kind="elementwise", kernel="k_batchnorm", module="conv", arg_struct="BatchNormArgs",
            args=dict(x=self.ref(x), w=self.ref(ps[0]), b=self.ref(ps[1]), mean=self.ref(ps[2]), var=self.ref(ps[3]),
                      out=self.ref(o), n=x.numel, hw=hw, C=x.shape[1], eps=float(node.attrs.get("eps", 1e-5)),
                      dtype=DTYPE_CODE[x.dtype], relu=0, p_dtype=DTYPE_CODE[ps[0].dtype], pad=0),
            grid=grid1d(x.numel), inputs=[t.name for t in node.inputs], outputs=[out.name], params={}))
        self.views[out.name] = o

    def lower_max_pool2d(self, node: OpNode) -> None:
        xv = self.view(node.inputs[0].name)
        if _is_nhwc(xv) and xv.shape[1] % 8 == 0 and (xv.offset * 2) % 16 == 0 and \
                xv.dtype in ("float16", "bfloat16"):
            return self._max_pool2d_nhwc(node, xv)
        x = self.contiguous(node.inputs[0].name)
        out = node.outputs[0]
        ks = node.attrs.get("kernel_size", [2, 2])
        ks = [ks, ks] if isinstance(ks, int) else list(ks)
        st = node.attrs.get("stride", None) or ks
        st = [st, st] if isinstance(st, int) else list(st)
        pd = node.attrs.get("padding", [0, 0])
        pd = [pd, pd] if isinstance(pd, int) else list(pd)
        N, C, H, W = x.shape
        Ho, Wo = out.shape[2], out.shape[3]
        o = self.new_storage(out.name, out.shape, out.dtype)
        self.emit(LaunchStep(
            kind="reduction", kernel="k_maxpool2d", module="conv", arg_struct="PoolArgs",
            args=dict(x=self.ref(x), out=self.ref(o), planes=N * C, H=H, W=W, Ho=Ho, Wo=Wo, kh=ks[0], kw=ks[1],
                      sh=st[0], sw=st[1], ph=pd[0], pw=pd[1], dtype=DTYPE_CODE[x.dtype], C=0),
            grid=grid1d(N * C * Ho * Wo), inputs=[node.inputs[0].name], outputs=[out.name], params={}))
        self.views[out.name] = o

    def _max_pool2d_nhwc(self, node: OpNode, xv: TView) -> None:
        """Max pooling of a channels-last image into a channels-last result (8 channels per thread)."""
        out = node.outputs[0]
        ks = node.attrs.get("kernel_size", [2, 2])
        ks = [ks, ks] if isinstance(ks, int) else list(ks)
        st = node.attrs.get("stride", None) or ks
        st = [st, st] if isinstance(st, int) else list(st)
        pd = node.attrs.get("padding", [0, 0])
        pd = [pd, pd] if isinstance(pd, int) else list(pd)
        N, C, H, W = xv.shape
        Ho, Wo = out.shape[2], out.shape[3]
        ob = self.new_storage(out.name, [N, Ho, Wo, C], out.dtype)
        self.emit(LaunchStep(
            kind="reduction", kernel=f"k_maxpool2d_nhwc_{'bf16' if xv.dtype == 'bfloat16' else 'f16'}",
            module="conv", arg_struct="PoolArgs",
            args=dict(x=self.ref(xv), out=self.ref(ob), planes=N, H=H, W=W, Ho=Ho, Wo=Wo, kh=ks[0], kw=ks[1],
                      sh=st[0], sw=st[1], ph=pd[0], pw=pd[1], dtype=DTYPE_CODE[xv.dtype], C=C),
            grid=grid1d(N * Ho * Wo * C // 8), inputs=[node.inputs[0].name], outputs=[out.name],
            params={"nhwc": True}))
        self.views[out.name] = ob.with_(shape=(N, C, Ho, Wo), strides=(Ho * Wo * C, 1, Wo * C, C))

    def lower_adaptive_avg_pool2d(self, node: OpNode) -> None:
        """Global average pooling (output 1 x 1): the mean over H*W of each (n, c) plane."""
        xv = self.view(node.inputs[0].name)
        out = node.outputs[0]
        if _is_nhwc(xv) and xv.shape[1] % 8 == 0 and (xv.offset * 2) % 16 == 0 and \
                xv.dtype in ("float16", "bfloat16") and out.dtype == xv.dtype:
            N, C, H, W = xv.shape
            o = self.new_storage(out.name, out.shape, out.dtype)   # [N, C, 1, 1]: the same bytes in either layout
            self.emit(LaunchStep(
                kind="reduction", kernel=f"k_mean_nhwc_{'bf16' if xv.dtype == 'bfloat16' else 'f16'}", module="conv",
                arg_struct="MeanNHWCArgs", args=dict(x=self.ref(xv), out=self.ref(o), n=N, hw=H * W, c=C),
                grid=grid1d(N * C // 8), inputs=[node.inputs[0].name], outputs=[out.name], params={"nhwc": True}))
            self.views[out.name] = o
            return
        x = self.contiguous(node.inputs[0].name)
        N, C, H, W = x.shape
        o = self.new_storage(out.name, out.shape, out.dtype)
        self.emit(mean_rows_step(self.ref(x), self.ref(o), N * C, H * W, x.dtype, out.dtype, [node.inputs[0].name],
                                 [out.name]))
        self.views[out.name] = o

    def lower_argmax(self, node: OpNode) -> None:
        x = node.inputs[0]
        out = node.outputs[0]
        v = self.view(x.name)
        dim = node.attrs.get("dim", None)
        if dim is None:
            pv = self.contiguous(x.name, v)
            pv = V.restride(pv, (1, pv.numel))
        else:
            dim = int(dim) % len(x.shape)
            perm = [d for d in range(len(x.shape)) if d != dim] + [dim]
            pv = V.permute(v, perm)
            if not pv.is_contiguous():
                pv = self.contiguous(x.name, pv)
        cols = pv.shape[-1]
        rows = pv.numel // cols
        o = self.new_storage(out.name, out.shape, out.dtype)
        if (pv.dtype in ("bfloat16", "float16") and cols % 8 == 0 and cols >= 4096 and (pv.offset * 2) % 16 == 0
                and out.dtype in ("int64", "int32") and cols < 2 ** 32):
            # long rows: split across workgroups (16-byte loads), then one key per row segment
            # is reduced by k_argmax_finalize (same tie and NaN rules as k_argmax)
            parts = (cols + 8191) // 8192
            seg = ((cols + parts - 1) // parts + 7) // 8 * 8
            slot = self.scratch(out.name + ".argmax", 8 * rows * parts)
            self.emit(LaunchStep(
                kind="reduction", kernel="k_argmax_part", module="gemv", arg_struct="ArgmaxPartArgs",
                args=dict(x=self.ref(pv), slot=slot, rows=rows, cols=cols, seg=seg, x_dtype=DTYPE_CODE[pv.dtype],
                          parts=parts),
                grid=(parts, max(rows, 1), 1), inputs=[x.name], outputs=[out.name + ".argmax"],
                params={"rows": rows, "cols": cols, "parts": parts}))
            self.emit(LaunchStep(
                kind="reduction", kernel="k_argmax_finalize", module="gemv", arg_struct="ArgmaxFinalizeArgs",
                args=dict(slot=slot, out=self.ref(o), rows=rows, parts=parts, out_dtype=DTYPE_CODE[out.dtype]),
                grid=(max(rows, 1), 1, 1), inputs=[out.name + ".argmax"], outputs=[out.name],
                params={"rows": rows, "parts": parts}))
            self.views[out.name] = o
            return
        self.emit(LaunchStep(
            kind="reduction", kernel="k_argmax", module="basic", arg_struct="ReduceLastArgs",
            args=dict(x=self.ref(pv), out=self.ref(o), rows=rows, cols=cols, x_dtype=DTYPE_CODE[pv.dtype],
                      out_dtype=DTYPE_CODE[out.dtype]),
            grid=(max(rows, 1), 1, 1), inputs=[x.name], outputs=[out.name], params={"rows": rows, "cols": cols}))
        self.views[out.name] = o

    def lower_embedding(self, node: OpNode) -> None:
        w_t, idx_t = node.inputs[0], node.inputs[1]
        out = node.outputs[0]
        w = self.contiguous(w_t.name)
        ids = self.contiguous(idx_t.name)
        o = self.new_storage(out.name, out.shape, out.dtype)
        n = ids.numel
        self.emit(LaunchStep(
            kind="special", kernel="k_embedding", module="basic", arg_struct="EmbeddingArgs",
            args=dict(w=self.ref(w), ids=self.ref(ids), out=self.ref(o), n_ids=n, vocab=w.shape[0],
                      row_bytes=numel(w.shape[1:]) * ELEM_SIZE[w.dtype], ids_dtype=DTYPE_CODE[ids.dtype]),
            grid=(max(n, 1), 1, 1), inputs=[w_t.name, idx_t.name], outputs=[out.name],
            params={"seq_len": n, "embed_dim": numel(w.shape[1:])}))
        self.views[out.name] = o

    def lower_rope_table(self, node: OpNode) -> None:
        """cos/sin tables are emitted when first read (fused RoPE epilogues compute their own)."""
        done = []

        def emit(node=node):
            if not done:
                done.append(True)
                self._rope_table_now(node)

        for o in node.outputs[:2]:
            self.lazy[o.name] = emit

    def _rope_table_now(self, node: OpNode) -> None:
        for o in node.outputs[:2]:
            self.lazy.pop(o.name, None)
        inv_t, pos_t = node.inputs[0], node.inputs[1]
        cos_s, sin_s = node.outputs[0], node.outputs[1]
        inv = self.contiguous(inv_t.name)
        pos = self.contiguous(pos_t.name)
        if inv.dtype != "float32":   # HF upcasts: inv_freq[None, :, None].float()
            f32 = self.new_storage(inv_t.name + ".f32", inv.shape, "float32")
            self.emit_copy(inv, f32, [inv_t.name], [inv_t.name + ".f32"])
            inv = f32
        half = inv.numel
        S = pos.numel
        c = self.new_storage(cos_s.name, cos_s.shape, cos_s.dtype)
        s = self.new_storage(sin_s.name, sin_s.shape, sin_s.dtype)
        self.emit(LaunchStep(
            kind="special", kernel="k_rope_table", module="basic", arg_struct="RopeTableArgs",
            args=dict(inv_freq=self.ref(inv), pos=self.ref(pos), cos_out=self.ref(c), sin_out=self.ref(s), S=S,
                      half=half, pos_dtype=DTYPE_CODE[pos.dtype], out_dtype=DTYPE_CODE[cos_s.dtype],
                      scaling=float(node.attrs.get("attention_scaling", 1.0))),
            grid=(max(S, 1), 1, 1), block=(max(64, ((2 * half + 63) // 64) * 64), 1, 1),
            inputs=[inv_t.name, pos_t.name], outputs=[cos_s.name, sin_s.name],
            params={"seq_len": S, "head_dim": 2 * half}))
        self.views[cos_s.name] = c
        self.views[sin_s.name] = s

    def _collapse(self, shape, strides) -> int | None:
        """Single stride covering ``shape`` as one flattened dim, or None."""
        st = None
        expect = None
        for s, t in zip(reversed(shape), reversed(strides)):
            if s == 1:
                continue
            if st is None:
                st, expect = t, t * s
            elif t != expect:
                return None
            else:
                expect = t * s
        return st if st is not None else 0

    def lower_index_copy(self, node: OpNode) -> None:
        self_t, idx_t, src_t = node.inputs[0], node.inputs[1], node.inputs[2]
        out = node.outputs[0]
        dim = int(node.attrs.get("dim", 0)) % len(self_t.shape)
        tv = self.view(self_t.name)
        st = self.storages[tv.storage]
        inplace = (self.inplace_inputs and st.kind == "input" and len(self.consumers.get(self_t.name, [])) == 1
                   and tv.is_contiguous() and tv.offset == 0 and tv.numel * tv.itemsize == st.nbytes
                   and self_t.name not in self.graph_output_names)
        if inplace:
            self.flush_chains_reading(tv.storage)
            dst = tv
            self.mutated_inputs.add(tv.storage)
        else:
            dst = self.new_storage(out.name, out.shape, out.dtype)
            self.emit_copy(tv, dst, [self_t.name], [out.name])
        src = self.view(src_t.name)
        shape = list(tv.shape)
        outer = numel(shape[:dim])
        inner = numel(shape[dim + 1:])
        nidx = src.shape[dim]
        so = self._collapse(src.shape[:dim], src.strides[:dim])
        si = self._collapse(src.shape[dim + 1:], src.strides[dim + 1:])
        if so is None or si is None or (inner > 1 and si == 0):
            src = self.contiguous(src_t.name, src)
            so = self._collapse(src.shape[:dim], src.strides[:dim])
            si = self._collapse(src.shape[dim + 1:], src.strides[dim + 1:])
        sj = src.strides[dim]
        idx = self.contiguous(idx_t.name)
        total = outer * nidx * inner
        self.emit(LaunchStep(
            kind="special", kernel="k_index_copy", module="basic", arg_struct="IndexCopyArgs",
            args=dict(dst=self.ref(dst), src=self.ref(src), index=self.ref(idx), outer=outer, dim_size=shape[dim],
                      inner=inner, nidx=nidx, src_so=so if outer > 1 else 0, src_sj=sj, src_si=si if inner > 1 else 0,
                      idx_dtype=DTYPE_CODE[idx.dtype], elem_bytes=ELEM_SIZE[dst.dtype]),
            grid=grid1d(total), inputs=[self_t.name, idx_t.name, src_t.name], outputs=[out.name],
            params={"outer_size": outer, "dim_size": shape[dim], "inner_size": inner, "num_indices": nidx,
                    "inplace": inplace}))
        self.views[out.name] = dst

    def lower_full(self, node: OpNode) -> None:
        out = node.outputs[0]
        o = self.new_storage(out.name, out.shape, out.dtype)
        n = o.numel
        self.emit(LaunchStep(
            kind="special", kernel="k_fill", module="basic", arg_struct="FillArgs",
            args=dict(out=self.ref(o), n=n, value=float(node.attrs.get("fill_value", 0.0)),
                      dtype=DTYPE_CODE[out.dtype]),
            grid=grid1d(n), inputs=[], outputs=[out.name], params={"total": n}))
        self.views[out.name] = o

    def lower_cat(self, node: OpNode) -> None:
        out = node.outputs[0]
        nd = len(out.shape)
        dim = int(node.attrs.get("dim", 0)) % nd
        o = self.new_storage(out.name, out.shape, out.dtype)
        pos = 0
        for t in node.inputs:
            if len(t.shape) == 1 and t.shape[0] == 0:
                continue
            v = self.view(t.name)
            n = v.shape[dim]
            dst = V.slice_(o, dim, pos, pos + n)
            self.emit_copy(v, dst.with_(dtype=out.dtype), [t.name], [out.name])
            pos += n
        self.views[out.name] = o

    # ------------------------------------------------------------------ driver

    def run(self, patterns) -> None:
        for pat in patterns:
            pat(self)
        for node in self.g.nodes:
            if node.name in self.claimed:
                emitter = self.claimed[node.name]
                if emitter is not None:
                    emitter()
                continue
            self.lower_node(node)
        for o in self.g.graph_outputs:
            self.view(o.name)
        self.emit_weight_permutes()

    def _permute_step(self, chunk: list) -> LaunchStep:
        """One k_permute_ohwi launch over up to OHWI_MAX (name, src, dst, (cin, kh, kw), (cp, khp, kwp))."""
        from hip_runtime.kernels import OHWI_MAX

        start, tot = [], 0
        for e in chunk:
            start.append(tot)
            tot += e[2].numel
        pad = OHWI_MAX - len(chunk)
        col = lambda f: [f(e) for e in chunk] + [1] * pad
        return LaunchStep(
            kind="copy", kernel="k_permute_ohwi", module="conv", arg_struct="PermuteOHWIArgs",
            args=dict(src=[self.ref(e[1]) for e in chunk] + [None] * pad,
                      dst=[self.ref(e[2]) for e in chunk] + [None] * pad,
                      start=start + [tot] * (pad + 1), cin=col(lambda e: e[3][0]), kh=col(lambda e: e[3][1]),
                      kw=col(lambda e: e[3][2]), cp=col(lambda e: e[4][0]), khp=col(lambda e: e[4][1]),
                      kwp=col(lambda e: e[4][2]), n=len(chunk), pad=0),
            grid=grid1d(tot // 8), inputs=[e[0] for e in chunk], outputs=[e[2].storage for e in chunk],
            params={"tensors": len(chunk), "elements": tot})

    def emit_weight_permutes(self) -> None:
        """The OHWI copies of bound conv weights, in launches of up to OHWI_MAX tensors placed first in
        the program (they depend on nothing else), re-run every execution like any step."""
        from hip_runtime.kernels import OHWI_MAX

        self.steps[:0] = [self._permute_step(self._ohwi[c:c + OHWI_MAX]) for c in range(0, len(self._ohwi), OHWI_MAX)]
        self._ohwi = []

    def is_constant(self, v: TView) -> bool:
        """True for a view of a bound weight: memory that no launch of the program writes."""
        st = self.storages.get(v.storage)
        return st is not None and st.kind == "weight" and v.storage not in self.mutated_inputs

    def lower_node(self, node: OpNode) -> None:
        op = node.op_type
        cat = classify_op(op)
        if cat == OpCategory.NOOP:
            return
        if cat == OpCategory.ELEMENTWISE:
            return self.lower_elementwise(node)
        if cat == OpCategory.SHAPE_ALIAS:
            return self.lower_alias(node)
        table = {
            "aten.linear.default": self.lower_linear,
            "aten.matmul.default": self.lower_matmul,
            "aten.mm.default": self.lower_matmul,
            "aten.bmm.default": self.lower_matmul,
            "aten.addmm.default": self.lower_addmm,
            "aten.softmax.int": self.lower_softmax,
            "aten._softmax.default": self.lower_softmax,
            "aten.mean.dim": self.lower_mean,
            "aten.argmax.default": self.lower_argmax,
            "aten.embedding.default": self.lower_embedding,
            "wrap_with_set_grad_enabled": self.lower_rope_table,
            "aten.index_copy.default": self.lower_index_copy,
            "aten.full.default": self.lower_full,
            "aten.cat.default": self.lower_cat,
            "aten.conv2d.default": self.lower_conv2d,
            "aten.batch_norm.default": self.lower_batch_norm,
            "aten.max_pool2d.default": self.lower_max_pool2d,
            "aten.adaptive_avg_pool2d.default": self.lower_adaptive_avg_pool2d,
        }
        fn = table.get(op)
        if fn is None:
            raise NotImplementedError(f"HIP backend has no lowering for {op} (node {node.name})")
        fn(node)


def analyze_subgraph(graph: IRGraph, inplace_inputs: bool = True, fuse: bool = True,
                     exact_attention: bool = False, fold_attention: bool | None = None) -> Lowering:
    from hip_compiler.patterns import DEFAULT_PATTERNS

    low = Lowering(graph, inplace_inputs=inplace_inputs, exact_attention=exact_attention,
                   fold_attention=fold_attention)
    low.run(DEFAULT_PATTERNS if fuse else [])
    return low


__all__ = ["Lowering", "analyze_subgraph", "grid1d", "math"]
