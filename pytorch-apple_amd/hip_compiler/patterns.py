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
            low.emit(LaunchStep(
                kind="rmsnorm", kernel="k_rmsnorm", module="basic", arg_struct="RMSNormArgs",
                args=dict(x=low.ref(xv), w=low.ref(wv), out=low.ref(o), rows=rows, ldx=cols, ldo=cols, cols=cols,
                          eps=eps, x_dtype=DTYPE_CODE[xv.dtype], w_dtype=DTYPE_CODE[wv.dtype],
                          n_dtype=DTYPE_CODE[n_dtype], out_dtype=DTYPE_CODE[out.dtype]),
                grid=(max(rows, 1), 1, 1), inputs=[x.name, w.name], outputs=[out.name],
                params={"rows": rows, "cols": cols, "eps": eps, "nodes": names}))
            low.views[out.name] = o

        cx.claim(chain, emit)


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
        if len(q_t.shape) != 4 or q_t.shape[0] != 1 or q_t.shape[2] != 1:
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
        if H % kvh or H // kvh > 8 or k_spec.shape[3] != D:
            continue
        add_dtype = add_n.outputs[0].dtype if mask_name is not None else dt
        if mask_name is not None:
            ms = next(t for t in add_n.inputs if t.name == mask_name).shape
            if len(ms) > 4 or ms[-1] != S or any(s != 1 for s in ms[:-1]):
                continue
        inside = {n.name for n in nodes}
        if not all(cx.private(n.outputs[0].name, inside) for n in nodes[:-1]):
            continue
        out = mm2.outputs[0]

        def emit(q=q_t.name, k=k_name, v=v_name, mask=mask_name, out=out, scale=scale, H=H, kvh=kvh, S=S,
                 add_dtype=add_dtype, dt=dt, names=[n.name for n in nodes]):
            _emit_decode_attention(low, q, k, v, mask, out, scale, H, kvh, S, add_dtype, dt, names)

        cx.claim(nodes, emit)


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
    part = low.scratch(out.name + ".part", kvh * ntiles * G * D * 4)
    counters = low.scratch(out.name + ".tickets", kvh * 4, persistent=True)
    args = dict(q=low.ref(qv), k=low.ref(kv_), v=low.ref(vv_), out=low.ref(o), scores=scores, stats=stats,
                part=part, counters=counters, S=S, q_head_stride=qv.strides[1], kv_head_stride=kv_.strides[1],
                H=H, KVH=kvh, D=D, ntiles=ntiles, scale=float(scale), add_dtype=DTYPE_CODE[add_dtype],
                dtype=DTYPE_CODE[dt], **margs)
    ins = [q, k, v] + ([mask] if mask else [])
    params = {"kv_heads": kvh, "q_per_kv": G, "seq_len": S, "head_dim": D, "ntiles": ntiles, "nodes": names}
    low.emit(LaunchStep(kind="attention", kernel="k_attn_scores", module="attention", arg_struct="DecodeAttnArgs",
                        args=args, grid=(ntiles, kvh, 1), inputs=ins, outputs=[out.name + ".scores"], params=params))
    low.emit(LaunchStep(kind="attention", kernel="k_attn_pv", module="attention", arg_struct="DecodeAttnArgs",
                        args=dict(args), grid=(ntiles, kvh, 1), inputs=ins + [out.name + ".scores"],
                        outputs=[out.name], params=params))
    low.views[out.name] = o


DEFAULT_PATTERNS = [decode_attention, rmsnorm, masked_softmax]

__all__ = ["DEFAULT_PATTERNS", "rmsnorm", "masked_softmax", "decode_attention", "V"]
