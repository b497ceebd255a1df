"""Pattern pre-passes of the HIP subgraph compiler.

Each pass looks for an op sequence, checks that every intermediate tensor is read
only inside the sequence, claims the nodes and registers an emitter that runs at
the position of the sequence's last node. Counterparts in the reference:

* ``rmsnorm``: `cuda_compiler/subgraph_analyzer.py:667-756` (emitted at cs:866-882)
  — ``[to(f32)] → pow(·,2) → mean(-1, keepdim) → add(eps) → rsqrt → mul(h, r) →
  [to(dtype)] → mul(w, ·)`` becomes one ``k_rmsnorm`` launch; eps is read from the
  add's ``other`` attribute (the reference falls back to a hard-coded 1e-6, D10).
* ``masked_softmax``: cs:759-789 (cs:884-906) — ``add(scores, mask) → softmax(-1)``
  becomes one ``k_softmax`` launch whose mask is read through broadcast strides
  (the reference indexes the mask as if it had the scores' shape, D4).
* ``decode_attention``: the GQA matcher of cs:85-160 and the decode chain of
  `npu_compiler/fusion_patterns.py:225-371` — ``[repeat_kv] → transpose(2,3) →
  matmul(q, ·) → mul(scale) → add(mask) → softmax → [to] → [dropout] →
  matmul(·, [repeat_kv] v)`` with a single query position becomes the two-kernel
  split-KV attention of ``csrc/kernels/attention.hip``.
"""

from __future__ import annotations

from hip_compiler import views as V
from hip_compiler.program import DTYPE_CODE, LaunchStep
from npu_compiler.ir_reader import OpNode

# a split-K reduce with the residual epilogue and the RMSNorm reading its result run as one
# kernel (k_gemm_reduce_*_resid_norm); off = two launches with the same results
FUSE_REDUCE_NORM = True

_PASS = ("aten._assert_tensor_metadata.default",)


class _Ctx:
    def __init__(self, low):
        self.low = low
        self.index = {n.name: i for i, n in enumerate(low.g.nodes)}

    def consumers(self, tname: str) -> list[OpNode]:
        return [n for n in self.low.consumers.get(tname, []) if n.op_type not in _PASS]

    def only(self, tname: str, op: str | tuple) -> OpNode | None:
        cs = self.consumers(tname)
        ops = (op,) if isinstance(op, str) else op
        if len(cs) == 1 and cs[0].op_type in ops and cs[0].name not in self.low.claimed:
            return cs[0]
        return None

    def private(self, tname: str, inside: set[str]) -> bool:
        """True when ``tname`` is read only by nodes in ``inside`` and is not a graph output."""
        if tname in self.low.graph_output_names:
            return False
        return all(n.name in inside for n in self.consumers(tname))

    def claim(self, nodes: list[OpNode], emitter) -> None:
        last = max(nodes, key=lambda n: self.index[n.name])
        for n in nodes:
            self.low.claimed[n.name] = None
        self.low.claimed[last.name] = emitter


def _scalar_other(node: OpNode) -> float | None:
    if len(node.inputs) == 1 and "other" in node.attrs:
        return float(node.attrs["other"])
    return None


# ---------------------------------------------------------------------------------- RMSNorm

def rmsnorm(low) -> None:
    cx = _Ctx(low)
    for pow_n in low.g.nodes:
        if pow_n.op_type != "aten.pow.Tensor_Scalar" or pow_n.name in low.claimed:
            continue
        if float(pow_n.attrs.get("exponent", 0)) != 2.0:
            continue
        h = pow_n.inputs[0]
        mean_n = cx.only(pow_n.outputs[0].name, "aten.mean.dim")
        if mean_n is None:
            continue
        dims = mean_n.attrs.get("dim", [-1])
        dims = [dims] if isinstance(dims, int) else list(dims or [])
        nd = len(h.shape)
        if [d % nd for d in dims] != [nd - 1] or not mean_n.attrs.get("keepdim", False):
            continue
        add_n = cx.only(mean_n.outputs[0].name, "aten.add.Tensor")
        if add_n is None or _scalar_other(add_n) is None:
            continue
        eps = _scalar_other(add_n)
        rs_n = cx.only(add_n.outputs[0].name, "aten.rsqrt.default")
        if rs_n is None:
            continue
        m1 = cx.only(rs_n.outputs[0].name, "aten.mul.Tensor")
        if m1 is None or len(m1.inputs) != 2 or h.name not in {t.name for t in m1.inputs}:
            continue
        chain = [pow_n, mean_n, add_n, rs_n, m1]
        cur = m1
        cast = cx.only(m1.outputs[0].name, "aten.to.dtype")
        if cast is not None:
            chain.append(cast)
            cur = cast
        m2 = cx.only(cur.outputs[0].name, "aten.mul.Tensor")
        if m2 is None or len(m2.inputs) != 2:
            continue
        w = next((t for t in m2.inputs if t.name != cur.outputs[0].name), None)
        if w is None or len(w.shape) != 1 or w.shape[0] != h.shape[-1]:
            continue
        chain.append(m2)
        # the leading to(f32) is folded when h is read only by pow and mul(h, r)
        x = h
        h_prod = low.producer.get(h.name)
        if (h_prod is not None and h_prod.op_type == "aten.to.dtype" and h_prod.name not in low.claimed
                and cx.private(h.name, {pow_n.name, m1.name})):
            chain.insert(0, h_prod)
            x = h_prod.inputs[0]
        inside = {n.name for n in chain}
        if not all(cx.private(n.outputs[0].name, inside) for n in chain[:-1]):
            continue
        n_dtype = cast.outputs[0].dtype if cast is not None else m1.outputs[0].dtype
        out = m2.outputs[0]

        def emit(x=x, w=w, out=out, eps=eps, n_dtype=n_dtype, names=[n.name for n in chain]):
            xv = low.contiguous(x.name)
            wv = low.contiguous(w.name)
            cols = xv.shape[-1]
            rows = xv.numel // cols
            o = low.new_storage(out.name, out.shape, out.dtype)
            # one wave per row with 16-byte accesses for 16-bit rows that fit (k_rmsnorm_w)
            half = ("bfloat16", "float16")
            wave = (xv.dtype in half and wv.dtype == xv.dtype and out.dtype in half and cols % 8 == 0
                    and cols <= 4096 and (xv.offset * 2) % 16 == 0 and (wv.offset * 2) % 16 == 0)
            # x was just produced by a split-K reduce with the residual epilogue (o_proj or down_proj
            # + residual of a prefill-sized GEMM): that launch becomes reduce + residual + RMSNorm
            prev = low.steps[-1] if low.steps else None
            if (FUSE_REDUCE_NORM and wave and out.dtype == xv.dtype and prev is not None and prev.params.get("reduce")
                    and prev.params.get("epilogue") == "resid" and prev.outputs == [x.name]
                    and prev.args.get("nw", 1) == 1 and prev.args["N"] == cols <= 2048 and prev.args["M"] == rows
                    and prev.args["ldo"] == cols and prev.args["out"] == low.ref(xv)):
                pa = prev.args
                low.steps[-1] = LaunchStep(
                    kind="gemm", kernel=f"k_gemm_reduce_{'bf16' if xv.dtype == 'bfloat16' else 'f16'}_resid_norm",
                    module="gemm", arg_struct="ReduceNormArgs",
                    args=dict(part=pa["part"], bias=pa["bias"] if pa["flags"] & 1 else None, resid=pa["resid"],
                              out=pa["out"], norm_w=low.ref(wv), norm_out=low.ref(o), M=rows, ldr=pa["ldr"],
                              ldo=cols, ldn=cols, N=cols, ksplit=pa["ksplit"], eps=eps,
                              n_dtype=DTYPE_CODE[n_dtype], flags=pa["flags"] & 1),
                    grid=(rows, 1, 1), inputs=prev.inputs + [w.name], outputs=prev.outputs + [out.name],
                    params=dict(prev.params, norm=True, norm_nodes=names))
                low.views[out.name] = o
                return
            low.emit(LaunchStep(
                kind="rmsnorm", kernel="k_rmsnorm_w" if wave else "k_rmsnorm", module="basic", arg_struct="RMSNormArgs",
                args=dict(x=low.ref(xv), w=low.ref(wv), out=low.ref(o), rows=rows, ldx=cols, ldo=cols, cols=cols,
                          eps=eps, x_dtype=DTYPE_CODE[xv.dtype], w_dtype=DTYPE_CODE[wv.dtype],
                          n_dtype=DTYPE_CODE[n_dtype], out_dtype=DTYPE_CODE[out.dtype]),
                grid=(max((rows + 3) // 4 if wave else rows, 1), 1, 1), inputs=[x.name, w.name], outputs=[out.name],
                params={"rows": rows, "cols": cols, "eps": eps, "nodes": names}))
            low.views[out.name] = o

        # emitted only if some consumer needs the normalised tensor itself; a fused GEMV
        # that reads it folds the same computation into its prologue instead
        cx.claim(chain, None)
        low.lazy[out.name] = emit
        w_dt = w.dtype
        low.rms_info[out.name] = {"x": x.name, "w": w.name, "eps": eps, "n_dtype": n_dtype, "x_dtype": x.dtype,
                                  "w_dtype": w_dt, "out_dtype": out.dtype}


# ---------------------------------------------------------------------------------- masked softmax

def masked_softmax(low) -> None:
    cx = _Ctx(low)
    for add_n in low.g.nodes:
        if add_n.op_type != "aten.add.Tensor" or add_n.name in low.claimed or len(add_n.inputs) != 2:
            continue
        sm = cx.only(add_n.outputs[0].name, ("aten.softmax.int", "aten._softmax.default"))
        if sm is None:
            continue
        shape = add_n.outputs[0].shape
        dim = int(sm.attrs.get("dim", -1)) % len(shape)
        if dim != len(shape) - 1 or tuple(add_n.inputs[0].shape) != tuple(shape):
            continue
        if float(add_n.attrs.get("alpha", 1)) != 1.0:
            continue
        x, m = add_n.inputs[0], add_n.inputs[1]
        out = sm.outputs[0]

        def emit(x=x, m=m, add_dtype=add_n.outputs[0].dtype, out=out, names=[add_n.name, sm.name]):
            low.emit_softmax(x.name, m.name, add_dtype, out.name, tuple(out.shape), out.dtype, names)

        cx.claim([add_n, sm], emit)


# ---------------------------------------------------------------------------------- decode attention

def _unrepeat(cx: _Ctx, t_name: str, want_heads: int, inside: list[OpNode]) -> str | None:
    """Follow ``reshape ← expand ← unsqueeze(2)`` back from a [B,H,S,D] operand to the KV tensor."""
    low = cx.low
    r = low.producer.get(t_name)
    if r is None:
        return t_name
    if r.op_type not in ("aten.reshape.default", "aten.view.default", "aten._unsafe_view.default"):
        return t_name
    e = low.producer.get(r.inputs[0].name)
    if e is None or e.op_type != "aten.expand.default":
        return None
    u = low.producer.get(e.inputs[0].name)
    if u is None or u.op_type != "aten.unsqueeze.default":
        return None
    src = u.inputs[0]
    if len(src.shape) != 4 or len(e.outputs[0].shape) != 5:
        return None
    kvh, rep = src.shape[1], e.outputs[0].shape[2]
    if kvh * rep != want_heads or e.inputs[0].shape[2] != 1:
        return None
    for n in (u, e):
        if len(cx.consumers(n.outputs[0].name)) != 1:
            return None
    inside += [u, e, r]
    return src.name


def decode_attention(low) -> None:
    cx = _Ctx(low)
    for mm1 in low.g.nodes:
        if mm1.op_type != "aten.matmul.default" or mm1.name in low.claimed:
            continue
        q_t, kt_t = mm1.inputs[0], mm1.inputs[1]
        if len(q_t.shape) != 4 or q_t.shape[0] != 1:
            continue
        T = q_t.shape[2]   # 1: decode; >= 16: prefill (the MFMA kernel)
        if T != 1 and (T < 16 or low.exact_attention):
            continue
        H, D = q_t.shape[1], q_t.shape[3]
        if D != 128:
            continue
        tr = low.producer.get(kt_t.name)
        if tr is None or tr.op_type != "aten.transpose.int":
            continue
        if sorted([int(tr.attrs.get("dim0", 0)) % 4, int(tr.attrs.get("dim1", 1)) % 4]) != [2, 3]:
            continue
        if len(cx.consumers(tr.outputs[0].name)) != 1:
            continue
        nodes: list[OpNode] = [tr, mm1]
        k_name = _unrepeat(cx, tr.inputs[0].name, H, nodes)
        if k_name is None:
            continue
        mul_n = cx.only(mm1.outputs[0].name, "aten.mul.Tensor")
        if mul_n is None or _scalar_other(mul_n) is None:
            continue
        scale = _scalar_other(mul_n)
        nodes.append(mul_n)
        add_n = cx.only(mul_n.outputs[0].name, "aten.add.Tensor")
        mask_name = None
        cur = mul_n
        if add_n is not None and len(add_n.inputs) == 2 and float(add_n.attrs.get("alpha", 1)) == 1.0:
            mask_name = add_n.inputs[1].name if add_n.inputs[0].name == mul_n.outputs[0].name else add_n.inputs[0].name
            nodes.append(add_n)
            cur = add_n
        sm = cx.only(cur.outputs[0].name, ("aten.softmax.int", "aten._softmax.default"))
        if sm is None or int(sm.attrs.get("dim", -1)) % 4 != 3:
            continue
        nodes.append(sm)
        cur = sm
        for op in ("aten.to.dtype", "aten.dropout.default"):
            nx = cx.only(cur.outputs[0].name, op)
            if nx is not None:
                if op == "aten.dropout.default" and nx.attrs.get("train", False) and nx.attrs.get("p", 0.0):
                    break
                nodes.append(nx)
                cur = nx
        mm2 = cx.only(cur.outputs[0].name, "aten.matmul.default")
        if mm2 is None or mm2.inputs[0].name != cur.outputs[0].name:
            continue
        v_name = _unrepeat(cx, mm2.inputs[1].name, H, nodes)
        if v_name is None:
            continue
        nodes.append(mm2)
        dt = q_t.dtype
        if dt not in ("bfloat16", "float16"):
            continue
        if not (mm1.outputs[0].dtype == mul_n.outputs[0].dtype == cur.outputs[0].dtype == mm2.outputs[0].dtype == dt):
            continue
        k_spec = next(t for n in nodes for t in n.inputs if t.name == k_name) if k_name != tr.inputs[0].name \
            else tr.inputs[0]
        kvh = k_spec.shape[1]
        S = k_spec.shape[2]
        if H % kvh or H // kvh > 8 or k_spec.shape[3] != D or S > 64 * 1024:
            continue
        add_dtype = add_n.outputs[0].dtype if mask_name is not None else dt
        if mask_name is not None and T > 1:
            mdt = next(t for t in add_n.inputs if t.name == mask_name).dtype
            if mdt not in (dt, "float32"):
                continue
        if mask_name is not None:
            ms = next(t for t in add_n.inputs if t.name == mask_name).shape
            if len(ms) > 4 or ms[-1] != S or any(s != 1 for s in ms[:-2]) or (len(ms) > 1 and ms[-2] not in (1, T)):
                continue
        inside = {n.name for n in nodes}
        if not all(cx.private(n.outputs[0].name, inside) for n in nodes[:-1]):
            continue
        out = mm2.outputs[0]

        def emit(q=q_t.name, k=k_name, v=v_name, mask=mask_name, out=out, scale=scale, H=H, kvh=kvh, S=S,
                 add_dtype=add_dtype, dt=dt, names=[n.name for n in nodes], T=T):
            if T > 1:
                _emit_prefill_attention(low, q, k, v, mask, out, scale, H, kvh, S, T, add_dtype, dt, names)
            elif low.exact_attention:
                _emit_decode_attention(low, q, k, v, mask, out, scale, H, kvh, S, add_dtype, dt, names)
            else:
                _emit_flash_attention(low, q, k, v, mask, out, scale, H, kvh, S, add_dtype, dt, names)

        cx.claim(nodes, emit)


def _emit_prefill_attention(low, q, k, v, mask, out, scale, H, kvh, S, T, add_dtype, dt, names) -> None:
    """T queries (prefill) on MFMA, flash style (csrc/kernels/attention.hip, k_attn_prefill). The
    output is stored [T, H, D] and exposed as the [1, H, T, D] view the graph expects, so the
    transpose(1, 2) + reshape in front of o_proj is a view, not a copy."""
    D = 128
    qv = low.view(q)
    if list(qv.strides[2:]) != [D, 1] or (qv.offset * 2) % 16:
        qv = low.contiguous(q, qv)
    kv_ = low.contiguous(k)
    vv_ = low.contiguous(v)
    if (kv_.offset * 2) % 16 or (vv_.offset * 2) % 16 or (qv.offset * 2) % 16:
        raise NotImplementedError("attention operands must be 16-byte aligned")
    margs = dict(mask=None, mask_row_stride=0, mask_col_stride=0, mask_dtype=-1, blk_limit=None)
    if mask is not None:
        mv = low.view(mask)
        if mv.dtype not in (dt, "float32"):
            raise NotImplementedError("prefill attention mask must have the model dtype or fp32")
        if mv.dtype != "float32":
            # the kernel reads four 16-bit mask entries per 8-byte load: unit column stride,
            # rows and base 8-byte aligned
            if S % 4:
                raise NotImplementedError("prefill attention with a 16-bit mask needs S % 4 == 0")
            rs = mv.strides[-2] if len(mv.shape) > 1 and mv.shape[-2] == T else 0
            if mv.strides[-1] != 1 or rs % 4 or (mv.offset * 2) % 16:
                mv = low.aligned16(low.contiguous(mask), mask)
        row = mv.strides[-2] if len(mv.shape) > 1 and mv.shape[-2] == T else 0
        margs = dict(mask=low.ref(mv), mask_row_stride=row, mask_col_stride=mv.strides[-1],
                     mask_dtype=DTYPE_CODE[mv.dtype], blk_limit=_mask_extent(low, mask, mv, row, T, S))
    st = low.new_storage(out.name, [1, T, H, D], dt)
    args = dict(q=low.ref(qv), k=low.ref(kv_), v=low.ref(vv_), out=low.ref(st), T=T, S=S, q_head_stride=qv.strides[1],
                kv_head_stride=kv_.strides[1], H=H, KVH=kvh, scale=float(scale), add_dtype=DTYPE_CODE[add_dtype],
                dtype=DTYPE_CODE[dt], **margs)
    kname = "k_attn_prefill" + ("" if dt == "bfloat16" else "_f16") + \
        ("_nomask" if mask is None else ("_f32mask" if margs["mask_dtype"] == DTYPE_CODE["float32"] else ""))
    low.emit(LaunchStep(kind="attention", kernel=kname,
                        module="attention", arg_struct="PrefillAttnArgs", args=args, grid=((T + 31) // 32, H, 1),
                        inputs=[q, k, v] + ([mask] if mask else []), outputs=[out.name],
                        params={"T": T, "S": S, "heads": H, "kv_heads": kvh, "nodes": names}))
    low.views[out.name] = st.with_(shape=(1, H, T, D), strides=(T * H * D, D, H * D, 1))


def _mask_extent(low, name: str, mv, row: int, T: int, S: int):
    """Per block of 32 query rows, how many 32-position blocks the mask leaves open at most
    (``k_mask_extent``), computed once per distinct mask view and shared by every layer's
    prefill attention."""
    key = (mv.storage, mv.offset, tuple(mv.shape), tuple(mv.strides), row, T, S)
    ref = low.mask_extents.get(key)
    if ref is None:
        nqb = (T + 31) // 32
        ref = low.scratch(name + ".extent", 4 * nqb)
        low.emit(LaunchStep(kind="special", kernel="k_mask_extent", module="attention", arg_struct="MaskExtentArgs",
                            args=dict(mask=low.ref(mv), nblk_out=ref, T=T, S=S, row_stride=row,
                                      col_stride=mv.strides[-1], mask_dtype=DTYPE_CODE[mv.dtype]),
                            grid=(nqb, 1, 1), block=(1024, 1, 1), inputs=[name], outputs=[ref.storage],
                            params={"T": T, "S": S}))
        low.mask_extents[key] = ref
    return ref


def _emit_flash_attention(low, q, k, v, mask, out, scale, H, kvh, S, add_dtype, dt, names) -> None:
    """Split-S partials now; the combine is emitted lazily (or folded into the next GEMV)."""
    D = 128
    G = H // kvh
    qv = low.view(q)
    if qv.strides[-1] != 1:
        qv = low.contiguous(q, qv)
    kv_ = low.contiguous(k)
    vv_ = low.contiguous(v)
    if (kv_.offset * 2) % 16 or (vv_.offset * 2) % 16:
        raise NotImplementedError("attention caches must be 16-byte aligned")
    # 64 positions per split (4 waves) with a combine kernel; when the combine can fold into
    # the next GEMV's prologue (at most 16 splits and 16 heads) 128 positions (8 waves, up to
    # S = 2048) or 256 (16 waves, up to S = 4096), which leaves 2x / 4x fewer partials for every
    # workgroup of that GEMV to read (measured at S = 2048: 8 waves + 16-split fold 9.2 us,
    # 16 waves + 8-split fold 9.6 us, 4 waves + combine + o_proj 12.5 us)
    waves = 4
    if low.fold_attn_combine and H <= 16:
        waves = 8 if S <= 16 * 128 else (16 if S <= 16 * 256 else 4)
    spl = 16 * waves
    nsplit = (S + spl - 1) // spl
    margs = dict(mask=None, mask_stride=0, mask_dtype=-1)
    if mask is not None:
        mv = low.view(mask)
        margs = dict(mask=low.ref(mv), mask_stride=mv.strides[-1], mask_dtype=DTYPE_CODE[mv.dtype])
    part_o = low.scratch(out.name + ".part_o", kvh * nsplit * G * D * 2)   # bf16, normalised per split
    part_ml = low.scratch(out.name + ".part_ml", kvh * nsplit * G * 2 * 4)
    args = dict(q=low.ref(qv), k=low.ref(kv_), v=low.ref(vv_), part_o=part_o, part_ml=part_ml, S=S,
                q_head_stride=qv.strides[1], kv_head_stride=kv_.strides[1], H=H, KVH=kvh, nsplit=nsplit, spl=spl,
                scale=float(scale), add_dtype=DTYPE_CODE[add_dtype], dtype=DTYPE_CODE[dt], **margs)
    ins = [q, k, v] + ([mask] if mask else [])
    params = {"kv_heads": kvh, "q_per_kv": G, "seq_len": S, "head_dim": D, "nsplit": nsplit, "spl": spl,
              "nodes": names}
    # long caches (more than 32 splits): each split reads its mask first and skips its K / V rows
    # when every position is -inf, so a 32k-position cache at position 2k reads 2k positions' rows
    chk = waves == 4 and nsplit > 32 and mask is not None
    kname = ("k_attn_flash_chk" if chk else {4: "k_attn_flash", 8: "k_attn_flash_w8", 16: "k_attn_flash_w16"}[waves]) + \
        ("" if dt == "bfloat16" else "_f16")
    low.emit(LaunchStep(kind="attention", kernel=kname, module="attention", arg_struct="FlashArgs",
                        args=args, grid=(nsplit, kvh, G), block=(64 * waves, 1, 1), inputs=ins,
                        outputs=[out.name + ".partials"], params=params))

    def combine():
        o = low.new_storage(out.name, out.shape, out.dtype)
        low.emit(LaunchStep(kind="attention", kernel="k_attn_combine", module="attention", arg_struct="CombineArgs",
                            args=dict(part_o=part_o, part_ml=part_ml, out=low.ref(o), H=H, KVH=kvh, nsplit=nsplit,
                                      dtype=DTYPE_CODE[dt]),
                            grid=(H, 1, 1), block=(D, 1, 1), inputs=[out.name + ".partials"], outputs=[out.name],
                            params=params))
        low.views[out.name] = o

    low.lazy[out.name] = combine
    low.attn_info[out.name] = {"part_o": part_o, "part_ml": part_ml, "H": H, "KVH": kvh, "nsplit": nsplit,
                               "shape": list(out.shape), "out": out.name}


def _emit_decode_attention(low, q, k, v, mask, out, scale, H, kvh, S, add_dtype, dt, names) -> None:
    D = 128
    G = H // kvh
    qv = low.view(q)
    if qv.strides[-1] != 1 or (qv.offset * 2) % 4:
        qv = low.contiguous(q, qv)
    kv_ = low.contiguous(k)
    vv_ = low.contiguous(v)
    if (kv_.offset * 2) % 16 or (vv_.offset * 2) % 16:
        raise NotImplementedError("attention caches must be 16-byte aligned")
    ntiles = (S + 63) // 64
    margs = dict(mask=None, mask_stride=0, mask_dtype=-1)
    if mask is not None:
        mv = low.view(mask)
        margs = dict(mask=low.ref(mv), mask_stride=mv.strides[-1], mask_dtype=DTYPE_CODE[mv.dtype])
    o = low.new_storage(out.name, out.shape, out.dtype)
    scores = low.scratch(out.name + ".scores", H * S * 4)
    stats = low.scratch(out.name + ".stats", H * ntiles * 2 * 4)
    args = dict(q=low.ref(qv), k=low.ref(kv_), v=low.ref(vv_), out=low.ref(o), scores=scores, stats=stats,
                S=S, q_head_stride=qv.strides[1], kv_head_stride=kv_.strides[1], H=H, KVH=kvh, D=D,
                ntiles=ntiles, scale=float(scale), add_dtype=DTYPE_CODE[add_dtype], dtype=DTYPE_CODE[dt], **margs)
    ins = [q, k, v] + ([mask] if mask else [])
    params = {"kv_heads": kvh, "q_per_kv": G, "seq_len": S, "head_dim": D, "ntiles": ntiles, "nodes": names}
    low.emit(LaunchStep(kind="attention", kernel="k_attn_scores", module="attention", arg_struct="DecodeAttnArgs",
                        args=args, grid=(ntiles, kvh, 1), inputs=ins, outputs=[out.name + ".scores"], params=params))
    oargs = dict(scores=scores, stats=stats, v=low.ref(vv_), mask=margs["mask"], out=low.ref(o), S=S,
                 kv_head_stride=vv_.strides[1], mask_stride=margs["mask_stride"], H=H, KVH=kvh, ntiles=ntiles,
                 mask_dtype=margs["mask_dtype"], dtype=DTYPE_CODE[dt])
    low.emit(LaunchStep(kind="attention", kernel="k_attn_out", module="attention", arg_struct="AttnOutArgs",
                        args=oargs, grid=(D // 8, kvh, 1), inputs=[out.name + ".scores", v],
                        outputs=[out.name], params=params))
    low.views[out.name] = o


# ---------------------------------------------------------------------------------- fused decode GEMVs

def _linear_parts(n: OpNode):
    """(x, w, bias or None) of a 2-D-weight ``aten.linear`` node, or None."""
    if n.op_type != "aten.linear.default" or len(n.inputs) < 2 or len(n.inputs[1].shape) != 2:
        return None
    return n.inputs[0], n.inputs[1], (n.inputs[2] if len(n.inputs) > 2 else None)


def _gemv_candidate(low, n: OpNode) -> bool:
    p = _linear_parts(n)
    if p is None or n.name in low.claimed:
        return False
    x, w, b = p
    return (low.gemv_ok(x.name, w.name, n.outputs[0].dtype, x.dtype) and (b is None or b.dtype == "bfloat16")
            and x.shape[-1] == w.shape[1])


def gate_up_silu(low) -> None:
    """``mul(silu(linear(x, Wg)), linear(x, Wu))`` → one GEMV over both weights with a SiLU·mul epilogue."""
    cx = _Ctx(low)
    for mul_n in low.g.nodes:
        if mul_n.op_type != "aten.mul.Tensor" or mul_n.name in low.claimed or len(mul_n.inputs) != 2:
            continue
        a, b = (low.producer.get(t.name) for t in mul_n.inputs)
        for silu_n, lu in ((a, b), (b, a)):
            if silu_n is None or lu is None or silu_n.op_type != "aten.silu.default":
                continue
            lg = low.producer.get(silu_n.inputs[0].name)
            if lg is None or not _gemv_candidate(low, lg) or not _gemv_candidate(low, lu) or lg is lu:
                continue
            (xg, wg, bg), (xu, wu, bu) = _linear_parts(lg), _linear_parts(lu)
            if xg.name != xu.name or wg.shape != wu.shape or (bg is None) != (bu is None):
                continue
            nodes = [lg, silu_n, lu, mul_n]
            if not (cx.private(lg.outputs[0].name, {silu_n.name}) and cx.private(silu_n.outputs[0].name, {mul_n.name})
                    and cx.private(lu.outputs[0].name, {mul_n.name})):
                continue
            out = mul_n.outputs[0]
            names = [n.name for n in nodes]

            def emit(x=xg.name, wg=wg.name, bg=bg.name if bg else None, wu=wu.name, bu=bu.name if bu else None,
                     out=out, names=names):
                low.emit_gemv(x, wg, bg, out.name, tuple(out.shape), epi="silu", nodes=names + _readers(low, x, names),
                              w2=wu, b2=bu)

            cx.claim(nodes, emit)
            break


def _readers(low, x: str, names: list[str]) -> list[str]:
    """Names of other claimed GEMV nodes that share ``x`` (so a norm on ``x`` can still be folded)."""
    return [n.name for n in low.consumers.get(x, []) if n.name not in names and n.name in low.claimed]


def linear_resid(low) -> None:
    """``add(r, linear(x, W))`` (either operand order) → GEMV with a residual epilogue."""
    cx = _Ctx(low)
    for add_n in low.g.nodes:
        if add_n.op_type != "aten.add.Tensor" or add_n.name in low.claimed or len(add_n.inputs) != 2:
            continue
        if float(add_n.attrs.get("alpha", 1)) != 1.0:
            continue
        for lin_t, r_t in ((add_n.inputs[1], add_n.inputs[0]), (add_n.inputs[0], add_n.inputs[1])):
            lin = low.producer.get(lin_t.name)
            if lin is None or not _gemv_candidate(low, lin) or lin_t.name == r_t.name:
                continue
            if tuple(r_t.shape) != tuple(add_n.outputs[0].shape) or r_t.dtype != "bfloat16":
                continue
            if tuple(lin_t.shape) != tuple(add_n.outputs[0].shape) or not cx.private(lin_t.name, {add_n.name}):
                continue
            x, w, b = _linear_parts(lin)
            out = add_n.outputs[0]
            names = [lin.name, add_n.name]

            def emit(x=x.name, w=w.name, b=b.name if b else None, r=r_t.name, out=out, names=names):
                low.emit_gemv(x, w, b, out.name, tuple(out.shape), epi="resid", resid=r,
                              nodes=names + _readers(low, x, names))

            cx.claim([lin, add_n], emit)
            break


def linear_argmax(low) -> None:
    """``argmax(linear(x, W), dim=-1)`` → GEMV whose epilogue also reduces the argmax (first index)."""
    cx = _Ctx(low)
    for am in low.g.nodes:
        if am.op_type != "aten.argmax.default" or am.name in low.claimed or am.attrs.get("keepdim", False):
            continue
        dim = am.attrs.get("dim", None)
        src = am.inputs[0]
        if dim is None or int(dim) % len(src.shape) != len(src.shape) - 1:
            continue
        lin = low.producer.get(src.name)
        if lin is None or not _gemv_candidate(low, lin):
            continue
        if any(n.name != am.name for n in cx.consumers(src.name)):
            continue
        x, w, b = _linear_parts(lin)
        rows = 1
        for s in src.shape[:-1]:
            rows *= s
        if rows != 1:
            continue
        out = am.outputs[0]
        names = [lin.name, am.name]

        def emit(x=x.name, w=w.name, b=b.name if b else None, src=src, out=out, names=names):
            low.emit_gemv(x, w, b, src.name, tuple(src.shape), epi="argmax", nodes=names + _readers(low, x, names),
                          argmax_out=(out.name, tuple(out.shape), out.dtype))

        cx.claim([lin, am], emit)


def _heads(cx: _Ctx, lin: OpNode):
    """``linear → view [B, T, n, D] → transpose(1, 2)`` with T == 1: returns (view, transpose, n, D) or None."""
    v = cx.only(lin.outputs[0].name, ("aten.view.default", "aten.reshape.default", "aten._unsafe_view.default"))
    if v is None or len(v.outputs[0].shape) != 4 or v.outputs[0].shape[:2] != [1, 1]:
        return None
    t = cx.only(v.outputs[0].name, "aten.transpose.int")
    if t is None or sorted([int(t.attrs.get("dim0", 0)) % 4, int(t.attrs.get("dim1", 1)) % 4]) != [1, 2]:
        return None
    return v, t, v.outputs[0].shape[2], v.outputs[0].shape[3]


def _rope_source(low, t_name: str):
    """(rope node, output index) when ``t_name`` is ``unsqueeze(getitem(rope, i), 1)``."""
    u = low.producer.get(t_name)
    if u is None or u.op_type != "aten.unsqueeze.default" or int(u.attrs.get("dim", 0)) != 1:
        return None
    g = low.producer.get(u.inputs[0].name)
    if g is None or g.op_type != "<built-in function getitem>":
        return None
    idx = int(g.attrs.get("index", 0))
    src = g.inputs[idx] if idx < len(g.inputs) else g.inputs[0]
    r = low.producer.get(src.name)
    if r is None or r.op_type != "wrap_with_set_grad_enabled":
        return None
    return r, [o.name for o in r.outputs].index(src.name)


def _rope_chain(cx: _Ctx, x_name: str, D: int):
    """Match ``add(mul(x, cos), mul(cat(neg(x[..., D/2:]), x[..., :D/2]), sin))``.

    Returns (nodes, output name, rope node) or None.
    """
    low = cx.low
    cs = cx.consumers(x_name)
    if len(cs) != 3 or any(n.name in low.claimed for n in cs):
        return None
    muls = [n for n in cs if n.op_type == "aten.mul.Tensor"]
    slices = [n for n in cs if n.op_type == "aten.slice.Tensor"]
    if len(muls) != 1 or len(slices) != 2:
        return None
    half = D // 2

    def rng(s):
        return (int(s.attrs.get("dim", 0)) % 4, int(s.attrs.get("start", 0) or 0),
                min(int(s.attrs.get("end", D)), D), int(s.attrs.get("step", 1)))

    lo = next((s for s in slices if rng(s) == (3, 0, half, 1)), None)
    hi = next((s for s in slices if rng(s) == (3, half, D, 1)), None)
    if lo is None or hi is None:
        return None
    neg = cx.only(hi.outputs[0].name, "aten.neg.default")
    if neg is None:
        return None
    cat = cx.only(neg.outputs[0].name, "aten.cat.default")
    if (cat is None or [t.name for t in cat.inputs] != [neg.outputs[0].name, lo.outputs[0].name]
            or int(cat.attrs.get("dim", 0)) % 4 != 3 or cx.consumers(lo.outputs[0].name) != [cat]):
        return None
    m2 = cx.only(cat.outputs[0].name, "aten.mul.Tensor")
    m1 = muls[0]
    if m2 is None or len(m1.inputs) != 2 or len(m2.inputs) != 2:
        return None
    cos_t = next(t for t in m1.inputs if t.name != x_name)
    sin_t = next(t for t in m2.inputs if t.name != cat.outputs[0].name)
    cs_src, sn_src = _rope_source(low, cos_t.name), _rope_source(low, sin_t.name)
    if cs_src is None or sn_src is None or cs_src[0] is not sn_src[0] or (cs_src[1], sn_src[1]) != (0, 1):
        return None
    add = cx.only(m1.outputs[0].name, "aten.add.Tensor")
    if add is None or cx.consumers(m2.outputs[0].name) != [add] or float(add.attrs.get("alpha", 1)) != 1.0:
        return None
    if add.inputs[0].name != m1.outputs[0].name:
        return None
    nodes = [m1, lo, hi, neg, cat, m2, add]
    if not all(n.outputs[0].dtype == "bfloat16" for n in nodes):
        return None
    return nodes, add.outputs[0].name, cs_src[0]


def _inplace_target(low, cx: _Ctx, t_name: str):
    """``index_copy(past, cpos, t, dim=2)`` updatable in place: returns (node, past, cpos) or None."""
    ic = cx.only(t_name, "aten.index_copy.default")
    if ic is None or int(ic.attrs.get("dim", 0)) % 4 != 2 or ic.inputs[2].name != t_name:
        return None
    past, cpos = ic.inputs[0], ic.inputs[1]
    st = low.storages.get(past.name)
    if (st is None or st.kind != "input" or len(low.consumers.get(past.name, [])) != 1
            or past.name in low.graph_output_names or not low.inplace_inputs or cpos.shape != [1]):
        return None
    return ic, past.name, cpos.name


def qkv_rope(low) -> None:
    """Three projections of one activation row — q with RoPE, k with RoPE written to the K cache,
    v written to the V cache — become one ``k_qkv_rope`` launch (RMSNorm folded in when pending)."""
    cx = _Ctx(low)
    by_x: dict[str, dict] = {}
    for lin in low.g.nodes:
        if not _gemv_candidate(low, lin):
            continue
        x, w, b = _linear_parts(lin)
        hd = _heads(cx, lin)
        if hd is None:
            continue
        vnode, tnode, nh, D = hd
        if D % 2 or D > 256:
            continue
        xname = tnode.outputs[0].name
        rope = _rope_chain(cx, xname, D)
        entry = {"lin": lin, "w": w, "b": b, "nh": nh, "D": D, "nodes": [lin, vnode, tnode]}
        if rope is not None:
            rnodes, rout, rnode = rope
            entry["nodes"] += rnodes
            entry["rope"] = rnode
            tgt = _inplace_target(low, cx, rout)
            if tgt is None:
                if rout in low.graph_output_names:
                    continue
                entry["role"], entry["out"] = "q", rout
            else:
                entry["role"], entry["ic"], entry["past"], entry["cpos"] = "k", *tgt
                entry["nodes"].append(tgt[0])
        else:
            tgt = _inplace_target(low, cx, xname)
            if tgt is None:
                continue
            entry["role"], entry["ic"], entry["past"], entry["cpos"] = "v", *tgt
            entry["nodes"].append(tgt[0])
        by_x.setdefault(x.name, {}).setdefault(entry["role"], []).append(entry)
    for xname, roles in by_x.items():
        if any(len(roles.get(r, [])) != 1 for r in ("q", "k", "v")):
            continue
        q, k, v = roles["q"][0], roles["k"][0], roles["v"][0]
        if not (q["D"] == k["D"] == v["D"] and k["nh"] == v["nh"] and q["rope"] is k["rope"]
                and k["cpos"] == v["cpos"] and q["nh"] % k["nh"] == 0):
            continue
        if len({q["b"] is None, k["b"] is None, v["b"] is None}) != 1 or not _rope_inputs_ok(q["rope"], 1):
            continue
        K = q["w"].shape[1]
        if K > 3072 or any(e["w"].shape != [e["nh"] * e["D"], K] for e in (q, k, v)):
            continue
        past_k = low.views[k["past"]]
        if list(past_k.shape[:2]) != [1, k["nh"]] or past_k.shape[3] != k["D"]:
            continue
        nodes = q["nodes"] + k["nodes"] + v["nodes"]
        names = [n.name for n in nodes]

        def emit(xname=xname, q=q, k=k, v=v, names=names):
            _emit_qkv(low, xname, q, k, v, names)

        cx.claim(nodes, emit)


def _rope_inputs_ok(rnode, n_pos: int) -> bool:
    """The fused RoPE kernels compute cos / sin from an fp32 ``inv_freq`` and one
    position per token; anything else stays on the unfused lowering."""
    inv, pos = rnode.inputs[0], rnode.inputs[1]
    n = 1
    for d in pos.shape:
        n *= int(d)
    return inv.dtype == "float32" and n == n_pos


def _emit_qkv(low, xname, q, k, v, names) -> None:
    norm = low.foldable_norm(xname, set(names))
    x = low.contiguous(norm["x"] if norm else xname)
    rope = q["rope"]
    inv = low.contiguous(rope.inputs[0].name)
    pos = low.contiguous(rope.inputs[1].name)
    cpos = low.contiguous(k["cpos"])
    if inv.dtype != "float32" or pos.numel != 1:
        raise NotImplementedError("fused RoPE needs fp32 inv_freq and one position")
    if pos.dtype not in ("int64", "int32") or cpos.dtype not in ("int64", "int32"):
        raise NotImplementedError("fused RoPE reads int64 or int32 positions")
    H, KVH, D = q["nh"], k["nh"], q["D"]
    K = x.shape[-1]
    if K % 8 or K > 3072:
        raise NotImplementedError("fused q/k/v needs hidden % 8 == 0 and <= 3072 (staged in LDS)")
    x = low.aligned16(x, norm["x"] if norm else xname)
    nw = low.aligned16(low.contiguous(norm["w"]), norm["w"]) if norm else None
    qo = low.new_storage(q["out"], [1, H, 1, D], "bfloat16")
    kc, vc = low.views[k["past"]], low.views[v["past"]]
    args = dict(x=low.ref(x), norm_w=low.ref(nw) if norm else None,
                wq=low.ref(low.contiguous(q["w"].name)), bq=low.ref(low.contiguous(q["b"].name)) if q["b"] else None,
                wk=low.ref(low.contiguous(k["w"].name)), bk=low.ref(low.contiguous(k["b"].name)) if k["b"] else None,
                wv=low.ref(low.contiguous(v["w"].name)), bv=low.ref(low.contiguous(v["b"].name)) if v["b"] else None,
                inv_freq=low.ref(inv), pos_ids=low.ref(pos), cache_pos=low.ref(cpos), q_out=low.ref(qo),
                k_dst=low.ref(kc), v_dst=low.ref(vc), kv_head_stride=kc.strides[1], cache_len=kc.shape[2],
                K=K, H=H, KVH=KVH, D=D, eps=float(norm["eps"]) if norm else 0.0,
                n_dtype=DTYPE_CODE[norm["n_dtype"]] if norm else 0,
                flags=(1 if norm else 0) | (2 if q["b"] else 0) | 4 | 8 | 16 | 32,
                pos_dtype=DTYPE_CODE[pos.dtype], cpos_dtype=DTYPE_CODE[cpos.dtype],
                rope_scaling=float(rope.attrs.get("attention_scaling", 1.0)))
    tasks = (H * D + 2 * KVH * D) // 2
    ins = [norm["x"] if norm else xname, q["w"].name, k["w"].name, v["w"].name, k["cpos"], k["past"], v["past"]]
    # three 512-element chunks per weight row and lane cover K <= 1536 (no chunk past K is issued)
    low.emit(LaunchStep(kind="gemv", kernel="k_qkv_rope_k1536" if K <= 1536 else "k_qkv_rope", module="gemv",
                        arg_struct="QKVArgs", args=args,
                        grid=((tasks + 3) // 4, 1, 1), inputs=ins,
                        outputs=[q["out"], k["ic"].outputs[0].name, v["ic"].outputs[0].name],
                        params={"M": 1, "N": H * D + 2 * KVH * D, "K": K, "epilogue": "qkv_rope",
                                "norm": norm is not None, "has_bias": q["b"] is not None, "nodes": names}))
    low.views[q["out"]] = qo
    low.views[k["ic"].outputs[0].name] = kc
    low.views[v["ic"].outputs[0].name] = vc
    low.mutated_inputs.update({kc.storage, vc.storage})


# ------------------------------------------------------------------ prefill q/k/v + RoPE + cache

def _heads_t(cx: _Ctx, lin: OpNode):
    """``linear → view [1, T, n, D] → transpose(1, 2)`` for any T: (view, transpose, T, n, D) or None."""
    v = cx.only(lin.outputs[0].name, ("aten.view.default", "aten.reshape.default", "aten._unsafe_view.default"))
    if v is None or len(v.outputs[0].shape) != 4 or v.outputs[0].shape[0] != 1:
        return None
    t = cx.only(v.outputs[0].name, "aten.transpose.int")
    if t is None or sorted([int(t.attrs.get("dim0", 0)) % 4, int(t.attrs.get("dim1", 1)) % 4]) != [1, 2]:
        return None
    _, T, n, D = v.outputs[0].shape
    return v, t, T, n, D


def _inplace_target_t(low, cx: _Ctx, t_name: str, T: int):
    """``index_copy(past, cpos, t, dim=2)`` with T positions, updatable in place: (node, past, cpos) or None."""
    ic = cx.only(t_name, "aten.index_copy.default")
    if ic is None or int(ic.attrs.get("dim", 0)) % 4 != 2 or ic.inputs[2].name != t_name:
        return None
    past, cpos = ic.inputs[0], ic.inputs[1]
    st = low.storages.get(past.name)
    if (st is None or st.kind != "input" or len(low.consumers.get(past.name, [])) != 1
            or past.name in low.graph_output_names or not low.inplace_inputs or cpos.shape != [T]):
        return None
    return ic, past.name, cpos.name


def qkv_rope_prefill(low) -> None:
    """Prefill (T >= GEMM_MIN_M tokens): the q, k and v projections of one activation — q and k
    rotated, k and v written into their caches in place — become one grouped MFMA GEMM (q | k | v
    columns) and one ``k_rope_cache`` launch, instead of three GEMMs, the rotate-half chains and
    two index_copy launches."""
    from hip_compiler.subgraph_analyzer import GEMM_MIN_M
    cx = _Ctx(low)
    by_x: dict[str, dict] = {}
    for lin in low.g.nodes:
        p = _linear_parts(lin)
        if p is None or lin.name in low.claimed:
            continue
        x, w, b = p
        if x.dtype != "bfloat16" or w.dtype != "bfloat16" or (b is not None and b.dtype != "bfloat16"):
            continue
        hd = _heads_t(cx, lin)
        if hd is None:
            continue
        vnode, tnode, T, nh, D = hd
        if T < GEMM_MIN_M or D % 2 or D > 128 or x.shape[-1] != w.shape[1]:
            continue
        xname = tnode.outputs[0].name
        rope = _rope_chain(cx, xname, D)
        entry = {"lin": lin, "w": w, "b": b, "nh": nh, "D": D, "T": T, "nodes": [lin, vnode, tnode]}
        if rope is not None:
            rnodes, rout, rnode = rope
            entry["nodes"] += rnodes
            entry["rope"] = rnode
            tgt = _inplace_target_t(low, cx, rout, T)
            if tgt is None:
                if rout in low.graph_output_names:
                    continue
                entry["role"], entry["out"] = "q", rout
            else:
                entry["role"], entry["ic"], entry["past"], entry["cpos"] = "k", *tgt
                entry["nodes"].append(tgt[0])
        else:
            tgt = _inplace_target_t(low, cx, xname, T)
            if tgt is None:
                continue
            entry["role"], entry["ic"], entry["past"], entry["cpos"] = "v", *tgt
            entry["nodes"].append(tgt[0])
        by_x.setdefault(x.name, {}).setdefault(entry["role"], []).append(entry)
    for xname, roles in by_x.items():
        if any(len(roles.get(r, [])) != 1 for r in ("q", "k", "v")):
            continue
        q, k, v = roles["q"][0], roles["k"][0], roles["v"][0]
        if not (q["D"] == k["D"] == v["D"] and q["T"] == k["T"] == v["T"] and k["nh"] == v["nh"]
                and q["rope"] is k["rope"] and k["cpos"] == v["cpos"] and q["nh"] % k["nh"] == 0):
            continue
        if len({q["b"] is None, k["b"] is None, v["b"] is None}) != 1 or not _rope_inputs_ok(q["rope"], q["T"]):
            continue
        K = q["w"].shape[1]
        if K % 32 or any(e["w"].shape != [e["nh"] * e["D"], K] for e in (q, k, v)):
            continue
        if (q["nh"] * q["D"]) % 64 or (k["nh"] * k["D"]) % 64:   # tile-aligned column groups
            continue
        past_k = low.views[k["past"]]
        if list(past_k.shape[:2]) != [1, k["nh"]] or past_k.shape[3] != k["D"]:
            continue
        nodes = q["nodes"] + k["nodes"] + v["nodes"]
        names = [n.name for n in nodes]

        def emit(xname=xname, q=q, k=k, v=v, names=names):
            _emit_qkv_prefill(low, xname, q, k, v, names)

        cx.claim(nodes, emit)


def _emit_qkv_prefill(low, xname, q, k, v, names) -> None:
    from hip_compiler.subgraph_analyzer import gemm_tiling
    x = low.aligned16(low.contiguous(xname), xname)   # a pending RMSNorm is materialised here
    rope = q["rope"]
    inv = low.contiguous(rope.inputs[0].name)
    pos = low.contiguous(rope.inputs[1].name)
    cpos = low.contiguous(k["cpos"])
    H, KVH, D, T = q["nh"], k["nh"], q["D"], q["T"]
    K = x.shape[-1]
    if inv.dtype != "float32" or pos.numel != T or x.numel != T * K:
        raise NotImplementedError("prefill RoPE needs fp32 inv_freq and one position per token")
    if pos.dtype not in ("int64", "int32") or cpos.dtype not in ("int64", "int32"):
        raise NotImplementedError("prefill RoPE reads int64 or int32 positions")
    N = (H + 2 * KVH) * D
    n1, n2 = H * D, (H + KVH) * D
    bm, bn, _, dma = gemm_tiling(T, N, K)
    if n1 % bn or n2 % bn:
        bn = 64
    bk = 64 if K % 64 == 0 else 32
    if bm == 64 and bn == 128:   # grouped kernels come in 64 x 64 and 128 x 128
        bn = 64
    ws = [low.aligned16(low.contiguous(e["w"].name), e["w"].name) for e in (q, k, v)]
    bs = [low.contiguous(e["b"].name) if e["b"] is not None else None for e in (q, k, v)]
    y = low.new_storage(q["out"] + ".qkv", [T, N], "bfloat16")
    args = dict(x=low.ref(x), w=low.ref(ws[0]), w2=low.ref(ws[1]), w3=low.ref(ws[2]),
                bias=low.ref(bs[0]) if bs[0] else None, bias2=low.ref(bs[1]) if bs[1] else None,
                bias3=low.ref(bs[2]) if bs[2] else None, resid=None, out=low.ref(y), part=None,
                M=T, ldx=K, ldw=K, ldo=N, ldr=N, sx=0, sw=0, so=0, batch=1, bdiv=1, N=N, K=K,
                flags=1 if bs[0] else 0, ksplit=1, kchunk=K, nw=1, n1=n1, n2=n2)
    ins = [xname] + [e["w"].name for e in (q, k, v)] + [e["b"].name for e in (q, k, v) if e["b"] is not None]
    low.emit(LaunchStep(kind="gemm", kernel=f"k_gemm_bf16_grp_m{bm}n{bn}" + ("_k64d" if dma else "_k64" if bk == 64
                                                                               else ""),
                        module="gemm", arg_struct="GemmArgs", args=args,
                        grid=((N + bn - 1) // bn, (T + bm - 1) // bm, 1), inputs=ins, outputs=[y.storage],
                        params={"M": T, "N": N, "K": K, "epilogue": "bias", "groups": [n1, n2], "mfma": True,
                                "tile": (bm, bn), "ksplit": 1, "bk": bk, "lds_direct": dma, "nodes": names}))
    qo = low.new_storage(q["out"], [1, H, T, D], "bfloat16")
    kc, vc = low.views[k["past"]], low.views[v["past"]]
    rargs = dict(y=low.ref(y), inv_freq=low.ref(inv), pos_ids=low.ref(pos), cache_pos=low.ref(cpos), q_out=low.ref(qo),
                 k_dst=low.ref(kc), v_dst=low.ref(vc), ldy=N, kv_head_stride=kc.strides[1], cache_len=kc.shape[2],
                 T=T, H=H, KVH=KVH, D=D, flags=4 | 8 | 16 | 32, pos_dtype=DTYPE_CODE[pos.dtype],
                 cpos_dtype=DTYPE_CODE[cpos.dtype], dtype=DTYPE_CODE["bfloat16"],
                 rope_scaling=float(rope.attrs.get("attention_scaling", 1.0)))
    low.emit(LaunchStep(kind="gemv", kernel="k_rope_cache", module="gemv", arg_struct="RopeCacheArgs", args=rargs,
                        grid=((T * (H + 2 * KVH) + 3) // 4, 1, 1), inputs=[y.storage, k["cpos"], k["past"], v["past"]],
                        outputs=[q["out"], k["ic"].outputs[0].name, v["ic"].outputs[0].name],
                        params={"T": T, "heads": [H, KVH], "nodes": names}))
    low.views[q["out"]] = qo
    low.views[k["ic"].outputs[0].name] = kc
    low.views[v["ic"].outputs[0].name] = vc
    low.mutated_inputs.update({kc.storage, vc.storage})


# ------------------------------------------------------------------ conv + BN (+ add) (+ ReLU)

def conv_bn_act(low) -> None:
    """``conv2d -> batch_norm [-> add(., r)] [-> relu]`` with private intermediates -> one implicit-GEMM
    launch whose epilogue applies the inference batch norm, the residual add and the ReLU
    (the Conv+BN+ReLU and Add+ReLU fusions of the reference's ResNet path)."""
    cx = _Ctx(low)
    for conv in low.g.nodes:
        if conv.op_type != "aten.conv2d.default" or conv.name in low.claimed:
            continue
        if len(conv.outputs[0].shape) != 4 or conv.outputs[0].dtype not in ("float16", "bfloat16"):
            continue
        bn = cx.only(conv.outputs[0].name, "aten.batch_norm.default")
        if bn is None or bn.attrs.get("training", False) or not cx.private(conv.outputs[0].name, {bn.name}):
            continue
        if bn.inputs[0].name != conv.outputs[0].name or any(t.dtype != conv.outputs[0].dtype for t in bn.inputs[1:5]):
            continue
        nodes, tail, resid, relu = [conv, bn], bn.outputs[0], None, False
        add = cx.only(tail.name, ("aten.add.Tensor",))
        if (add is not None and len(add.inputs) == 2 and float(add.attrs.get("alpha", 1)) == 1.0
                and cx.private(tail.name, {add.name})):
            other = add.inputs[1] if add.inputs[0].name == tail.name else add.inputs[0]
            if (other.name != tail.name and tuple(other.shape) == tuple(tail.shape) and other.dtype == tail.dtype
                    and add.outputs[0].dtype == tail.dtype):
                nodes, tail, resid = nodes + [add], add.outputs[0], other.name
        r = cx.only(tail.name, ("aten.relu.default", "aten.relu_.default"))
        if r is not None and cx.private(tail.name, {r.name}):
            nodes, tail, relu = nodes + [r], r.outputs[0], True

        def emit(conv=conv, bn=bn, resid=resid, relu=relu, out=tail.name, names=[n.name for n in nodes]):
            low.emit_conv(conv, out, bn=bn, resid=resid, relu=relu, nodes=names)

        cx.claim(nodes, emit)


DEFAULT_PATTERNS = [decode_attention, rmsnorm, qkv_rope, qkv_rope_prefill, gate_up_silu, linear_argmax, linear_resid,
                    masked_softmax,
                    conv_bn_act]

__all__ = ["DEFAULT_PATTERNS", "rmsnorm", "masked_softmax", "decode_attention", "V"]
