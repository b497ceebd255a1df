"""Oracle (test infrastructure only): numpy restatement of the CPU fallback's per-op semantics.

The reference checks device results against its CPU fallback, which runs every IR
node through ATen on the host (`npu_runtime/cpu_fallback.py:32-72`, via the
absent third-party ``torch_ir`` 0.2.2, `uv.lock:1575-1584`). This module restates
those semantics independently of torch, in numpy: every op computes in fp32 (or
fp64 for accumulations) and rounds its result once to the IR dtype of its output;
bf16 rounding is round-to-nearest-even on the fp32 bit pattern; bf16 tensors are
carried as uint16 bit patterns, as at the reference's host boundary
(`cpu_fallback.py:178-194`).

Pinned by (see ``tests/test_oracle.py``): the index_copy known-answer vectors of
`tests/test_index_copy.py:23-117`, the CPU-fallback KATs of
`tests/test_cpu_fallback.py:22-173`, the RoPE closed form of
`tests/test_extended_kernels.py:546-600`, the decode-attention closed form of
`tests/test_extended_kernels.py:621-640`, the RMSNorm/gated-MLP formulas of
`tests/test_composed_blocks.py:31-41,206-211`, invariants (softmax rows sum to 1,
GQA equals repeat_kv + MHA, argmax first-index ties) and ATen itself for the
rounding of each elementwise op.
"""

from __future__ import annotations

import numpy as np

FLOAT = {"float32", "float16", "bfloat16", "float64"}


# ---------------------------------------------------------------------------- bf16 helpers

def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 → bf16 bit pattern (quiet NaNs kept NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Value of ``x`` after storing it in ``dtype`` (as fp32 for float dtypes)."""
    x = np.asarray(x)
    if dtype == "bfloat16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x.astype(np.float32)))
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "float32":
        return x.astype(np.float32)
    if dtype == "float64":
        return x.astype(np.float64)
    if dtype in ("int64", "int32"):
        return x.astype(np.int64 if dtype == "int64" else np.int32)
    if dtype == "bool":
        return x.astype(bool)
    raise ValueError(dtype)


def to_value(arr: np.ndarray, dtype: str) -> np.ndarray:
    """Host array (uint16 for bf16) → compute value (fp32 for floats)."""
    if dtype == "bfloat16":
        return bf16_bits_to_f32(arr.view(np.uint16) if arr.dtype != np.uint16 else arr)
    if dtype in ("float16", "float32"):
        return np.asarray(arr).astype(np.float32)
    return np.asarray(arr)


def to_host(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x)
    if dtype == "float16":
        return np.asarray(x).astype(np.float16)
    if dtype == "float32":
        return np.asarray(x).astype(np.float32)
    return round_to(x, dtype)


# ---------------------------------------------------------------------------- closed forms

def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, dtype: str = "bfloat16") -> np.ndarray:
    """HF Qwen2RMSNorm with its rounding points: ``w * (x*rsqrt(mean(x^2)+eps)).to(dtype)``."""
    h = x.astype(np.float32)
    var = (h.astype(np.float64) ** 2).mean(-1, keepdims=True).astype(np.float32)
    n = round_to(h * (np.float32(1.0) / np.sqrt(var + np.float32(eps))), dtype)
    return round_to(w * n, dtype)


def rope_tables(inv_freq: np.ndarray, positions: np.ndarray, dtype: str = "bfloat16"):
    """cos/sin of ``cat(freqs, freqs)`` with ``freqs = pos * inv_freq`` (`test_extended_kernels.py:556-559`)."""
    f = positions.astype(np.float32)[:, None] * inv_freq.astype(np.float32)[None, :]
    emb = np.concatenate([f, f], axis=-1)
    return round_to(np.cos(emb), dtype), round_to(np.sin(emb), dtype)


def decode_attention(q, k, v, mask, scale, dtype: str = "bfloat16"):
    """One-token GQA attention with the model's rounding points.

    q [H, D], k/v [KVH, S, D], mask [S] (additive, model dtype). Returns [H, D].
    Follows the eager chain: s = r(q.k); s = r(s*scale); s = r(s+mask);
    p = r(softmax_f32(s)); o = r(sum p*v), r = rounding to ``dtype``.
    """
    H, D = q.shape
    kvh = k.shape[0]
    g = H // kvh
    out = np.zeros((H, D), dtype=np.float32)
    for h in range(H):
        kk = k[h // g].astype(np.float64)
        vv = v[h // g].astype(np.float64)
        s = round_to((kk @ q[h].astype(np.float64)).astype(np.float32), dtype)
        s = round_to(s * np.float32(scale), dtype)
        if mask is not None:
            s = round_to(s + mask.astype(np.float32), dtype)
        p = softmax_f32(s)
        p = round_to(p, dtype)
        out[h] = round_to((p.astype(np.float64) @ vv).astype(np.float32), dtype)
    return out


def softmax_f32(s: np.ndarray, axis: int = -1) -> np.ndarray:
    s = s.astype(np.float32)
    m = np.max(s, axis=axis, keepdims=True)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp((s - m).astype(np.float64))
    tot = e.sum(axis=axis, keepdims=True)
    return (e * (1.0 / tot)).astype(np.float32)


def index_copy(dst: np.ndarray, dim: int, index: np.ndarray, src: np.ndarray) -> np.ndarray:
    """Out-of-place ``dst.index_copy(dim, index, src)`` (bit-exact)."""
    out = np.array(dst, copy=True)
    sl = [slice(None)] * out.ndim
    for j, i in enumerate(np.asarray(index).reshape(-1)):
        sl_d = list(sl)
        sl_d[dim] = int(i)
        sl_s = list(sl)
        sl_s[dim] = j
        out[tuple(sl_d)] = src[tuple(sl_s)]
    return out


def argmax_first(x: np.ndarray, axis: int = -1) -> np.ndarray:
    return np.argmax(x, axis=axis)


# ---------------------------------------------------------------------------- IR walker

def _linear(x, w, b, out_dtype):
    acc = x.astype(np.float64) @ w.astype(np.float64).T
    if b is not None:
        acc = acc + b.astype(np.float64)
    return round_to(acc.astype(np.float32), out_dtype)


def _matmul(a, b, out_dtype):
    return round_to(np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32), out_dtype)


def _bin(op, a, b, out_dtype, alpha=1.0):
    fl = out_dtype in FLOAT
    if fl:
        a = np.asarray(a, dtype=np.float32)
        b = np.asarray(b, dtype=np.float32)
    if op == "add":
        r = a + (np.float32(alpha) * b if alpha != 1 else b)
    elif op == "sub":
        r = a - (np.float32(alpha) * b if alpha != 1 else b)
    elif op == "mul":
        r = a * b
    elif op == "div":
        r = np.asarray(a, np.float32) / np.asarray(b, np.float32)
    elif op in ("maximum", "minimum"):   # NaN in either operand gives NaN (torch.maximum / minimum)
        r = np.maximum(a, b) if op == "maximum" else np.minimum(a, b)
    else:
        raise ValueError(op)
    return round_to(r, out_dtype)


def _unary(op, a, out_dtype):
    x = np.asarray(a, dtype=np.float32) if out_dtype in FLOAT else np.asarray(a)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
        if op == "neg":
            r = -x
        elif op == "rsqrt":
            r = np.float32(1.0) / np.sqrt(x)
        elif op == "silu":
            r = x / (np.float32(1.0) + np.exp(-x))
        elif op == "relu":
            r = np.where(np.isnan(x), x, np.maximum(x, np.float32(0)))
        elif op == "cos":
            r = np.cos(x)
        elif op == "sin":
            r = np.sin(x)
        elif op == "exp":
            r = np.exp(x)
        elif op == "sigmoid":
            r = np.float32(1) / (np.float32(1) + np.exp(-x))
        elif op == "tanh":
            r = np.tanh(x)
        elif op == "sqrt":
            r = np.sqrt(x)
        elif op == "abs":
            r = np.abs(x)
        elif op == "reciprocal":
            r = np.float32(1.0) / x
        else:
            raise ValueError(op)
    return round_to(r, out_dtype)


def run_node(node: dict, env: dict) -> None:
    op = node["op_type"]
    ins = [env[t["name"]] for t in node.get("inputs", [])]
    outs = node.get("outputs", [])
    a = node.get("attrs", {}) or {}
    od = outs[0]["dtype"] if outs else None
    oshape = tuple(outs[0]["shape"]) if outs else ()
    short = op.split(".")[1] if op.startswith("aten.") else op

    def put(v, i=0):
        env[outs[i]["name"]] = v

    if op == "aten._assert_tensor_metadata.default":
        return
    if op == "<built-in function getitem>":
        idx = int(a.get("index", 0))
        put(ins[idx] if idx < len(ins) else ins[0])
        return
    if op == "wrap_with_set_grad_enabled":
        pos = np.asarray(ins[1]).reshape(-1)
        c, s = rope_tables(ins[0], pos, od)
        sc = float(a.get("attention_scaling", 1.0))
        if sc != 1.0:
            f = pos.astype(np.float32)[:, None] * ins[0].astype(np.float32)[None, :]
            emb = np.concatenate([f, f], -1)
            c, s = round_to(np.cos(emb) * sc, od), round_to(np.sin(emb) * sc, od)
        put(c.reshape(oshape), 0)
        put(s.reshape(oshape), 1)
        return
    if short in ("add", "sub", "mul", "div", "add_", "mul_", "maximum", "minimum"):
        other = ins[1] if len(ins) > 1 else np.float32(a["other"]) if od in FLOAT else a["other"]
        put(_bin(short.rstrip("_"), ins[0], other, od, float(a.get("alpha", 1.0))))
        return
    if short in ("neg", "rsqrt", "silu", "relu", "relu_", "cos", "sin", "exp", "sigmoid", "tanh", "sqrt", "abs",
                 "reciprocal"):
        put(_unary(short.rstrip("_"), ins[0], od))
        return
    if op == "aten.pow.Tensor_Scalar":
        e = float(a.get("exponent", 2))
        x = np.asarray(ins[0], np.float32)
        put(round_to(x * x if e == 2 else np.power(x, np.float32(e)), od))
        return
    if op in ("aten.to.dtype", "aten._to_copy.default", "aten.clone.default", "aten.contiguous.default",
              "aten.alias.default", "aten.detach.default", "aten.detach_.default"):
        put(round_to(ins[0], od))
        return
    if op == "aten.dropout.default":
        put(ins[0])
        return
    if op == "aten.linear.default":
        put(_linear(ins[0], ins[1], ins[2] if len(ins) > 2 else None, od))
        return
    if op in ("aten.matmul.default", "aten.mm.default", "aten.bmm.default"):
        put(_matmul(ins[0], ins[1], od))
        return
    if op == "aten.addmm.default":
        acc = np.float64(a.get("beta", 1)) * ins[0].astype(np.float64) + \
            np.float64(a.get("alpha", 1)) * (ins[1].astype(np.float64) @ ins[2].astype(np.float64))
        put(round_to(acc.astype(np.float32), od))
        return
    if op == "aten.embedding.default":
        put(ins[0][np.asarray(ins[1]).astype(np.int64)])
        return
    if op in ("aten.view.default", "aten.reshape.default", "aten._unsafe_view.default", "aten.flatten.using_ints",
              "aten.unsqueeze.default", "aten.squeeze.dim", "aten.squeeze.default"):
        put(np.reshape(ins[0], oshape))
        return
    if op == "aten.transpose.int":
        put(np.swapaxes(ins[0], int(a.get("dim0", 0)), int(a.get("dim1", 1))))
        return
    if op == "aten.t.default":
        put(ins[0].T)
        return
    if op == "aten.permute.default":
        put(np.transpose(ins[0], a["dims"]))
        return
    if op == "aten.expand.default":
        put(np.broadcast_to(ins[0], oshape))
        return
    if op == "aten.slice.Tensor":
        dim = int(a.get("dim", 0))
        sl = [slice(None)] * np.ndim(ins[0])
        end = a.get("end", None)
        end = None if end is None or end >= 2 ** 62 else int(end)
        sl[dim] = slice(int(a.get("start", 0) or 0), end, int(a.get("step", 1)))
        put(ins[0][tuple(sl)])
        return
    if op == "aten.select.int":
        put(np.take(ins[0], int(a.get("index", 0)), axis=int(a.get("dim", 0))))
        return
    if op == "aten.cat.default":
        put(np.concatenate([x for x in ins if not (np.ndim(x) == 1 and np.shape(x)[0] == 0)], axis=int(a.get("dim", 0))))
        return
    if op == "aten.mean.dim":
        dims = a.get("dim", None)
        dims = tuple(range(np.ndim(ins[0]))) if dims is None else tuple([dims] if isinstance(dims, int) else dims)
        m = np.asarray(ins[0], np.float64).mean(axis=dims, keepdims=bool(a.get("keepdim", False)))
        put(round_to(m.astype(np.float32), od))
        return
    if op in ("aten.softmax.int", "aten._softmax.default"):
        put(round_to(softmax_f32(np.asarray(ins[0], np.float32), int(a.get("dim", -1))), od))
        return
    if op == "aten.index_copy.default":
        put(index_copy(ins[0], int(a.get("dim", 0)), ins[1], ins[2]))
        return
    if op == "aten.argmax.default":
        dim = a.get("dim", None)
        x = np.asarray(ins[0])
        r = np.argmax(x.reshape(-1)) if dim is None else np.argmax(x, axis=int(dim))
        if a.get("keepdim", False) and dim is not None:
            r = np.expand_dims(r, int(dim))
        put(np.asarray(r, dtype=np.int64).reshape(oshape))
        return
    if op == "aten.full.default":
        put(round_to(np.full(oshape, a.get("fill_value", 0.0), dtype=np.float64), od))
        return
    raise NotImplementedError(f"oracle has no rule for {op}")


def run_ir(ir: dict, inputs: dict, weights: dict) -> dict:
    """Evaluate a whole IR dict. Host arrays in (bf16 as uint16), host arrays out."""
    env: dict = {}
    for g in ir["graph_inputs"]:
        env[g["name"]] = to_value(np.asarray(inputs[g["name"]]), g.get("dtype", "float32"))
    rev = {sd: ph for ph, sd in ir.get("weight_name_mapping", {}).items()}
    for w in ir["weights"]:
        arr = weights[w["name"]] if w["name"] in weights else weights[rev[w["name"]]]
        val = to_value(np.asarray(arr), w.get("dtype", "float32"))
        env[rev.get(w["name"], w["name"])] = val
        env.setdefault(w["name"], val)
    for n in ir["nodes"]:
        run_node(n, env)
    return {o["name"]: to_host(env[o["name"]], o.get("dtype", "float32")) for o in ir["graph_outputs"]}
