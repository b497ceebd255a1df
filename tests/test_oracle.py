"""Pins the numpy oracle (oracle/numpy_ref.py) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle (a dropped rounding,
a transposed operand, a wrong sign or index) fails it: known-answer vectors of the
reference's own tests, closed forms, invariants, brute force in float64, and ATen
(the CPU fallback's engine) on the same graphs.
"""

import numpy as np
import pytest
import torch

from oracle import numpy_ref as R


def test_bf16_rounding_matches_torch_bit_for_bit():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 20000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.0 + 2 ** -8,
                                  1.0 + 2 ** -8 + 2 ** -9, 1.0 + 3 * 2 ** -8], np.float32)]).astype(np.float32)
    ours = R.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    assert np.isnan(R.bf16_bits_to_f32(R.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]


@pytest.mark.parametrize("case", [
    # tests/test_index_copy.py:23-117 (values restated as vectors)
    (np.array([10, 20, 30, 40, 50.]), 0, [2], np.array([99.]), np.array([10, 20, 99, 40, 50.])),
    (np.arange(8.), 0, [1, 3, 5], np.array([100, 200, 300.]), np.array([0, 100, 2, 200, 4, 300, 6, 7.])),
    (np.arange(12.).reshape(4, 3), 0, [1, 3], np.array([[100, 101, 102], [300, 301, 302.]]),
     np.array([[0, 1, 2], [100, 101, 102], [6, 7, 8], [300, 301, 302.]])),
])
def test_index_copy_known_answers(case):
    dst, dim, idx, src, exp = case
    out = R.index_copy(dst, dim, np.array(idx), src)
    assert np.array_equal(out, exp)
    assert not np.array_equal(dst, exp)       # out of place


def test_index_copy_kv_shape_known_answer():
    rng = np.random.default_rng(42)
    cache = rng.standard_normal((1, 2, 8, 4))
    src = rng.standard_normal((1, 2, 1, 4))
    out = R.index_copy(cache, 2, np.array([5]), src)
    exp = cache.copy()
    exp[:, :, 5:6, :] = src
    assert np.array_equal(out, exp)


def test_rope_tables_closed_form():
    """tests/test_extended_kernels.py:546-600: cos/sin(cat(pos*inv_freq, pos*inv_freq))."""
    half = 64
    inv = (1.0 / (1e6 ** (np.arange(half, dtype=np.float32) / half))).astype(np.float32)
    pos = np.array([0, 1, 42, 1024, 2047])
    c, s = R.rope_tables(inv, pos, "float32")
    f = pos[:, None].astype(np.float64) * inv[None, :].astype(np.float64)
    np.testing.assert_allclose(c, np.cos(np.concatenate([f, f], 1)), atol=2e-4)
    np.testing.assert_allclose(s, np.sin(np.concatenate([f, f], 1)), atol=2e-4)
    assert np.array_equal(c[:, :half], c[:, half:])       # duplicated halves, not interleaved
    assert np.allclose(c[0], 1.0) and np.allclose(s[0], 0.0)


def test_rotary_node_attention_scaling_branch():
    """The rotary node's ``attention_scaling`` (transformers' dynamic / YaRN rope types scale cos
    and sin): the oracle's branch against the closed form evaluated in float64 and rounded once
    (at most one bf16 ulp apart: the float32 cos/sin may differ from float64 in the last fp32
    ulp) and against the CPU fallback's ATen evaluation; the unscaled tables differ."""
    import torch

    from npu_runtime.aten_executor import run_node as aten_run_node

    half, sc = 64, 0.7
    inv = (1.0 / (1e6 ** (np.arange(half, dtype=np.float32) / half))).astype(np.float32)
    pos = np.array([[0, 5, 1000, 2047, 32767]], dtype=np.int64)
    node = {"name": "rot", "op_type": "wrap_with_set_grad_enabled",
            "inputs": [{"name": "inv_freq", "shape": [half], "dtype": "float32"},
                       {"name": "pos", "shape": [1, 5], "dtype": "int64"}],
            "outputs": [{"name": "cos", "shape": [1, 5, 2 * half], "dtype": "bfloat16"},
                        {"name": "sin", "shape": [1, 5, 2 * half], "dtype": "bfloat16"}],
            "attrs": {"attention_scaling": sc}}
    env = {"inv_freq": inv, "pos": pos}
    R.run_node(node, env)
    # the angle as HF forms it (float32 product), its cos / sin in float64, one rounding
    f = (pos.reshape(-1)[:, None].astype(np.float32) * inv[None, :]).astype(np.float64)
    emb = np.concatenate([f, f], 1)
    for name, fn in (("cos", np.cos), ("sin", np.sin)):
        got = np.asarray(env[name], np.float32).reshape(5, 2 * half)
        exp = R.round_to(fn(emb) * sc, "bfloat16").reshape(5, 2 * half)
        ulp = np.maximum(np.abs(exp) * 2.0 ** -7, 1e-6)
        assert np.all(np.abs(got - exp) <= ulp), name
        unscaled = R.round_to(fn(emb), "bfloat16").reshape(5, 2 * half)
        assert not np.allclose(got, unscaled, atol=1e-3)            # the scaling is applied
    tenv = {"inv_freq": torch.from_numpy(inv), "pos": torch.from_numpy(pos)}
    aten_run_node(node, tenv)
    for name in ("cos", "sin"):
        a = tenv[name].float().numpy().reshape(5, 2 * half)
        o = np.asarray(env[name], np.float32).reshape(5, 2 * half)
        assert np.all(np.abs(a - o) <= np.maximum(np.abs(a) * 2.0 ** -7, 1e-6)), name


def _brute_attention(Q, K, V, mask, scale):
    """tests/test_extended_kernels.py:621-640 in float64 (no intermediate rounding)."""
    out = np.zeros(Q.shape)
    g = Q.shape[0] // K.shape[0]
    for h in range(Q.shape[0]):
        s = K[h // g].astype(np.float64) @ Q[h].astype(np.float64) * scale + mask
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[h // g]
    return out


@pytest.mark.parametrize("H,KVH,S,valid", [(2, 2, 16, 8), (4, 4, 32, 32), (12, 2, 129, 10), (12, 2, 300, 1)])
def test_decode_attention_vs_brute_force(H, KVH, S, valid):
    rng = np.random.default_rng(42)
    D = 128
    q = R.round_to(rng.standard_normal((H, D)).astype(np.float32), "bfloat16")
    k = R.round_to(rng.standard_normal((KVH, S, D)).astype(np.float32), "bfloat16")
    v = R.round_to(rng.standard_normal((KVH, S, D)).astype(np.float32), "bfloat16")
    mask = np.full(S, -np.inf, np.float32)
    mask[:valid] = 0
    got = R.decode_attention(q, k, v, mask, D ** -0.5)
    ref = _brute_attention(q, k, v, mask, D ** -0.5)
    np.testing.assert_allclose(got, ref, rtol=5e-2, atol=1e-2)
    if valid == 1:   # one valid position: output is exactly that V row (rounded)
        assert np.array_equal(got, R.round_to(np.repeat(v[:, 0], H // KVH, axis=0), "bfloat16"))


def test_gqa_equals_repeat_kv_then_mha():
    rng = np.random.default_rng(1)
    q = R.round_to(rng.standard_normal((12, 128)).astype(np.float32), "bfloat16")
    k = R.round_to(rng.standard_normal((2, 64, 128)).astype(np.float32), "bfloat16")
    v = R.round_to(rng.standard_normal((2, 64, 128)).astype(np.float32), "bfloat16")
    gqa = R.decode_attention(q, k, v, None, 128 ** -0.5)
    mha = R.decode_attention(q, np.repeat(k, 6, axis=0), np.repeat(v, 6, axis=0), None, 128 ** -0.5)
    assert np.array_equal(gqa, mha)


def test_softmax_invariants():
    rng = np.random.default_rng(3)
    s = rng.standard_normal((5, 300)).astype(np.float32) * 4
    s[:, 200:] = -np.inf
    p = R.softmax_f32(s)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-6)
    assert np.all(p[:, 200:] == 0)


def test_rmsnorm_matches_hf_formula_in_torch():
    """HF Qwen2RMSNorm (transformers modeling_qwen2.py): w * (x * rsqrt(mean(x^2) + eps)).to(bf16)."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16, 1536, generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn(1536, generator=g)).bfloat16()
    h = x.float()
    ref = w * (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    got = R.rmsnorm(R.bf16_bits_to_f32(x.view(torch.uint16).numpy()),
                    R.bf16_bits_to_f32(w.view(torch.uint16).numpy()), 1e-6)
    r = R.bf16_bits_to_f32(ref.view(torch.uint16).numpy())
    assert (got == r).mean() > 0.995
    np.testing.assert_allclose(got, r, rtol=1e-2)


def test_argmax_first_index_on_ties():
    x = np.array([[1.0, 3.0, 3.0, 2.0], [0.0, 0.0, 0.0, 0.0]])
    assert R.argmax_first(x).tolist() == [1, 0]


def _graph_agreement(ir, inputs, weights):
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    ex = DAGExecutor(partition(ir, lambda *_: False), None)
    ex.load_weights(weights)
    aten = ex.execute(inputs)
    ours = R.run_ir(ir, inputs, weights)
    res = {}
    for k in aten:
        a, b = np.asarray(aten[k]), np.asarray(ours[k])
        if a.dtype == np.uint16:
            fa, fb = R.bf16_bits_to_f32(a), R.bf16_bits_to_f32(b)
            res[k] = ((a == b).mean(), float(np.abs(fa - fb).max() / max(np.abs(fa).max(), 1e-6)))
        else:
            res[k] = (float((a == b).mean()), 0.0)
    return res


def test_oracle_agrees_with_aten_on_mlp_block():
    from irgen.qwen import QwenConfig, build_mlp_ir
    from irgen.workloads import make_weights, mlp_inputs, to_host

    cfg = QwenConfig(hidden=256, intermediate=512)
    ir = build_mlp_ir(4, cfg)
    w = {k: to_host(v) for k, v in make_weights(ir, cfg, norm_std=0.02).items()}
    x = {k: to_host(v) for k, v in mlp_inputs(4, cfg).items()}
    for bitexact, rel in _graph_agreement(ir, x, w).values():
        assert bitexact > 0.99 and rel < 1e-2


def test_oracle_agrees_with_aten_on_decode_step():
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights, to_host

    cfg = QwenConfig(hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000)
    ir = build_decode_ir(64, cfg, argmax=True)
    w = {k: to_host(v) for k, v in make_weights(ir, cfg).items()}
    x = {k: to_host(v) for k, v in decode_inputs(64, 40, cfg).items()}
    res = _graph_agreement(ir, x, w)
    for name, (bitexact, rel) in res.items():
        assert rel < 2e-2, name
    assert res["next_token"][0] == 1.0


def test_planted_mistake_is_caught(monkeypatch):
    """Dropping the bf16 rounding of RMSNorm's normalised value must break the ATen agreement."""
    from irgen.qwen import QwenConfig, build_mlp_ir
    from irgen.workloads import make_weights, mlp_inputs, to_host

    cfg = QwenConfig(hidden=256, intermediate=512)
    ir = build_mlp_ir(4, cfg)
    w = {k: to_host(v) for k, v in make_weights(ir, cfg, norm_std=0.02).items()}
    x = {k: to_host(v) for k, v in mlp_inputs(4, cfg).items()}
    orig = R.run_node

    def broken(node, env):
        if node["op_type"] == "aten.to.dtype" and node["outputs"][0]["dtype"] == "bfloat16":
            env[node["outputs"][0]["name"]] = np.asarray(env[node["inputs"][0]["name"]], np.float32)
            return
        orig(node, env)

    monkeypatch.setattr(R, "run_node", broken)
    (bitexact, _), = _graph_agreement(ir, x, w).values()
    assert bitexact < 0.99
