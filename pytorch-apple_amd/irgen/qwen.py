"""IR builders for the Qwen2.5-1.5B-architecture workloads.

The op sequence restates HF ``Qwen2ForCausalLM`` eager decoding as the reference
exports it with its ``_IndexCopyCache`` (`examples/extract_qwen_ir.py:68-131`):
RMSNorm = ``to(f32) → pow 2 → mean(-1, keepdim) → add eps → rsqrt → mul x →
to(bf16) → mul(weight, ·)``; q/k/v ``linear`` with bias → ``view`` →
``transpose(1,2)``; RoPE = ``q·cos + cat(−q[64:], q[:64])·sin`` with cos/sin from
``wrap_with_set_grad_enabled(inv_freq, position_ids)``; ``index_copy(dim 2,
cache_position)`` on the static K/V caches; ``repeat_kv`` as ``unsqueeze →
expand → reshape``; ``transpose(2,3) → matmul → mul(1/√d) → add(mask) →
softmax(f32) → to(bf16) → dropout(0) → matmul``; ``transpose → contiguous →
reshape → linear o → add residual``; gated MLP; final norm; tied ``lm_head``.

Graph inputs follow `examples/extract_qwen_ir.py:255-267`: ``input_ids`` int64
[1,1], ``attention_mask`` [1,1,1,S], ``position_ids`` int64 [1,1],
``cache_position`` int64 [1], then per layer the K and V caches [1,KVH,S,D].
Outputs are logits [1,1,V] and the 2·L updated caches; with ``argmax=True`` a
trailing ``aten.argmax.default(logits, -1)`` node adds ``next_token`` [1,1] int64
(the host-side ``np.argmax`` of `examples/run_qwen.py:125,180` moved into the
graph so that a greedy loop can stay on the device). The mask is emitted in the
model dtype (bf16) so that ``scores + mask`` stays bf16 as in the model.
"""

from __future__ import annotations

from dataclasses import dataclass

from irgen.builder import IRBuilder, T

INT64_MAX = 9223372036854775807


@dataclass(frozen=True)
class QwenConfig:
    hidden: int = 1536
    intermediate: int = 8960
    layers: int = 28
    heads: int = 12
    kv_heads: int = 2
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    tie_embeddings: bool = True
    dtype: str = "bfloat16"


QWEN2_5_1_5B = QwenConfig()


def rmsnorm(b: IRBuilder, x: T, w: T, eps: float) -> T:
    h = b.op("aten.to.dtype", [x], {"dtype": "float32"}, base="to")
    p = b.op("aten.pow.Tensor_Scalar", [h], {"exponent": 2})
    m = b.op("aten.mean.dim", [p], {"dim": [-1], "keepdim": True})
    a = b.op("aten.add.Tensor", [m], {"other": eps})
    r = b.op("aten.rsqrt.default", [a])
    n = b.op("aten.mul.Tensor", [h, r])
    nb = b.op("aten.to.dtype", [n], {"dtype": x.dtype}, base="to")
    return b.op("aten.mul.Tensor", [w, nb])


def linear(b: IRBuilder, x: T, w: T, bias: T | None = None) -> T:
    return b.op("aten.linear.default", [x, w] + ([bias] if bias is not None else []))


def rotate_half(b: IRBuilder, x: T) -> T:
    half = x.shape[-1] // 2
    x1 = b.op("aten.slice.Tensor", [x], {"dim": 3, "start": 0, "end": half})
    x2 = b.op("aten.slice.Tensor", [x], {"dim": 3, "start": half, "end": INT64_MAX})
    nx2 = b.op("aten.neg.default", [x2])
    return b.op("aten.cat.default", [nx2, x1], {"dim": -1})


def apply_rope(b: IRBuilder, x: T, cos_u: T, sin_u: T) -> T:
    xc = b.op("aten.mul.Tensor", [x, cos_u])
    xs = b.op("aten.mul.Tensor", [rotate_half(b, x), sin_u])
    return b.op("aten.add.Tensor", [xc, xs])


def repeat_kv(b: IRBuilder, x: T, n_rep: int) -> T:
    bsz, kvh, s, d = x.shape
    u = b.op("aten.unsqueeze.default", [x], {"dim": 2})
    e = b.op("aten.expand.default", [u], {"size": [bsz, kvh, n_rep, s, d]})
    return b.op("aten.reshape.default", [e], {"shape": [bsz, kvh * n_rep, s, d]})


def rope_tables(b: IRBuilder, cfg: QwenConfig, position_ids: T) -> tuple[T, T]:
    inv_freq = b.weight("model.rotary_emb.inv_freq", [cfg.head_dim // 2], "float32", buffer=True)
    cs = b.op("wrap_with_set_grad_enabled", [inv_freq, position_ids], n_out=2, out_dtype=cfg.dtype,
              base="wrap_with_set_grad_enabled")
    return b.getitem(cs, 0), b.getitem(cs, 1)


def attention_block(b: IRBuilder, cfg: QwenConfig, li: int, x: T, cos: T, sin: T, mask: T,
                    cache_position: T, past_k: T, past_v: T) -> tuple[T, T, T]:
    """q/k/v projections, RoPE, cache update, GQA attention and o_proj for one layer."""
    pre = f"model.layers.{li}.self_attn."
    dt = cfg.dtype
    H, KVH, D, Hd = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.hidden
    wq = b.weight(pre + "q_proj.weight", [H * D, Hd], dt)
    bq = b.weight(pre + "q_proj.bias", [H * D], dt)
    wk = b.weight(pre + "k_proj.weight", [KVH * D, Hd], dt)
    bk = b.weight(pre + "k_proj.bias", [KVH * D], dt)
    wv = b.weight(pre + "v_proj.weight", [KVH * D, Hd], dt)
    bv = b.weight(pre + "v_proj.bias", [KVH * D], dt)
    wo = b.weight(pre + "o_proj.weight", [Hd, H * D], dt)
    bsz, q_len = x.shape[0], x.shape[1]

    def heads(t: T, n: int) -> T:
        v = b.op("aten.view.default", [t], {"size": [bsz, q_len, n, D]})
        return b.op("aten.transpose.int", [v], {"dim0": 1, "dim1": 2})

    q = heads(linear(b, x, wq, bq), H)
    k = heads(linear(b, x, wk, bk), KVH)
    v = heads(linear(b, x, wv, bv), KVH)
    cos_u = b.op("aten.unsqueeze.default", [cos], {"dim": 1})
    sin_u = b.op("aten.unsqueeze.default", [sin], {"dim": 1})
    q = apply_rope(b, q, cos_u, sin_u)
    k = apply_rope(b, k, cos_u, sin_u)
    kc = b.op("aten.index_copy.default", [past_k, cache_position, k], {"dim": 2})
    vc = b.op("aten.index_copy.default", [past_v, cache_position, v], {"dim": 2})
    kr = repeat_kv(b, kc, H // KVH)
    vr = repeat_kv(b, vc, H // KVH)
    kt = b.op("aten.transpose.int", [kr], {"dim0": 2, "dim1": 3})
    s = b.op("aten.matmul.default", [q, kt])
    s = b.op("aten.mul.Tensor", [s], {"other": D ** -0.5})
    s = b.op("aten.add.Tensor", [s, mask])
    p = b.op("aten.softmax.int", [s], {"dim": -1, "dtype": "float32"})
    p = b.op("aten.to.dtype", [p], {"dtype": dt}, base="to")
    p = b.op("aten.dropout.default", [p], {"p": 0.0, "train": False})
    o = b.op("aten.matmul.default", [p, vr])
    o = b.op("aten.transpose.int", [o], {"dim0": 1, "dim1": 2})
    o = b.op("aten.contiguous.default", [o])
    o = b.op("aten.reshape.default", [o], {"shape": [bsz, q_len, H * D]})
    return linear(b, o, wo), kc, vc


def mlp_block(b: IRBuilder, cfg: QwenConfig, pre: str, x: T, norm_key: str) -> T:
    """RMSNorm → gate/up → SiLU(gate)·up → down → + residual."""
    dt = cfg.dtype
    wn = b.weight(norm_key, [cfg.hidden], dt)
    wg = b.weight(pre + "gate_proj.weight", [cfg.intermediate, cfg.hidden], dt)
    wu = b.weight(pre + "up_proj.weight", [cfg.intermediate, cfg.hidden], dt)
    wd = b.weight(pre + "down_proj.weight", [cfg.hidden, cfg.intermediate], dt)
    h = rmsnorm(b, x, wn, cfg.eps)
    g = b.op("aten.silu.default", [linear(b, h, wg)])
    gu = b.op("aten.mul.Tensor", [g, linear(b, h, wu)])
    return b.op("aten.add.Tensor", [x, linear(b, gu, wd)])


def build_mlp_ir(tokens: int, cfg: QwenConfig = QWEN2_5_1_5B) -> dict:
    """cfg1: x [T, hidden] → RMSNorm → gate/up → SiLU·up → down → + x."""
    b = IRBuilder("Qwen2.5_MLP")
    x = b.input("x", [tokens, cfg.hidden], cfg.dtype)
    b.output(mlp_block(b, cfg, "mlp.", x, "post_attention_layernorm.weight"))
    return b.to_dict()


def build_attention_ir(kv_len: int, cfg: QWEN2_5_1_5B.__class__ = QWEN2_5_1_5B, residual: bool = False) -> dict:
    """cfg2: one decode-token attention block over a [1, KVH, kv_len, D] cache. With
    ``residual`` the block is a decoder layer's first half: input RMSNorm before it and the
    block's input added to its output."""
    b = IRBuilder("Qwen2.5_Attention")
    x = b.input("hidden_states", [1, 1, cfg.hidden], cfg.dtype)
    mask = b.input("attention_mask", [1, 1, 1, kv_len], cfg.dtype)
    pos = b.input("position_ids", [1, 1], "int64")
    cpos = b.input("cache_position", [1], "int64")
    pk = b.input("past_key_0", [1, cfg.kv_heads, kv_len, cfg.head_dim], cfg.dtype)
    pv = b.input("past_value_0", [1, cfg.kv_heads, kv_len, cfg.head_dim], cfg.dtype)
    cos, sin = rope_tables(b, cfg, pos)
    h = x
    if residual:
        h = rmsnorm(b, x, b.weight("model.layers.0.input_layernorm.weight", [cfg.hidden], cfg.dtype), cfg.eps)
    out, kc, vc = attention_block(b, cfg, 0, h, cos, sin, mask, cpos, pk, pv)
    if residual:
        out = b.op("aten.add.Tensor", [x, out])
    b.output(out, kc, vc)
    return b.to_dict()


def build_decode_ir(max_cache_len: int, cfg: QwenConfig = QWEN2_5_1_5B, argmax: bool = False,
                    tokens: int = 1) -> dict:
    """cfg3: one full decode step over static caches of length ``max_cache_len``; with
    ``tokens`` > 1 the same graph is a prefill of that many tokens (cfg4: ``tokens`` =
    ``max_cache_len`` = 512, causal mask [1, 1, T, S] as an input)."""
    b = IRBuilder("Qwen2.5_Decode" if tokens == 1 else "Qwen2.5_Prefill")
    ids = b.input("input_ids", [1, tokens], "int64")
    mask = b.input("attention_mask", [1, 1, tokens, max_cache_len], cfg.dtype)
    pos = b.input("position_ids", [1, tokens], "int64")
    cpos = b.input("cache_position", [tokens], "int64")
    caches = []
    for li in range(cfg.layers):
        caches.append((b.input(f"past_key_{li}", [1, cfg.kv_heads, max_cache_len, cfg.head_dim], cfg.dtype),
                       b.input(f"past_value_{li}", [1, cfg.kv_heads, max_cache_len, cfg.head_dim], cfg.dtype)))
    emb = b.weight("model.embed_tokens.weight", [cfg.vocab, cfg.hidden], cfg.dtype)
    x = b.op("aten.embedding.default", [emb, ids])
    cos, sin = rope_tables(b, cfg, pos)
    new_caches = []
    for li in range(cfg.layers):
        pre = f"model.layers.{li}."
        wn = b.weight(pre + "input_layernorm.weight", [cfg.hidden], cfg.dtype)
        h = rmsnorm(b, x, wn, cfg.eps)
        a, kc, vc = attention_block(b, cfg, li, h, cos, sin, mask, cpos, *caches[li])
        x = b.op("aten.add.Tensor", [x, a])
        x = mlp_block(b, cfg, pre + "mlp.", x, pre + "post_attention_layernorm.weight")
        new_caches += [kc, vc]
    wf = b.weight("model.norm.weight", [cfg.hidden], cfg.dtype)
    h = rmsnorm(b, x, wf, cfg.eps)
    lm = emb if cfg.tie_embeddings else b.weight("lm_head.weight", [cfg.vocab, cfg.hidden], cfg.dtype)
    logits = linear(b, h, lm)
    b.output(logits, *new_caches)
    if argmax:
        b.output(b.op("aten.argmax.default", [logits], {"dim": -1}, base="next_token"))
    return b.to_dict()


def inv_freq(cfg: QwenConfig = QWEN2_5_1_5B):
    """``1 / theta^(2i/d)`` in fp32, the HF default rotary init with the config's theta."""
    import torch

    return 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.int64).float() / cfg.head_dim))
