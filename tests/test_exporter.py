"""IR producer (torch.export → reference IR schema), safetensors loading and the
prefill → decode generation loop, on the CPU.

The HF ``Qwen2ForCausalLM`` of this image's transformers is the outside reference:
the exported graph run through the CPU fallback (``DAGExecutor`` with an all-CPU
plan, ATen) must equal HF's own eager forward bit for bit, since both execute the
same ATen ops in the same order; the exported op sequence must follow the
hand-written ``irgen`` builder's, and both must lower to the same launch list.
"""

import json

import numpy as np
import pytest
import torch

transformers = pytest.importorskip("transformers")

S = 128


def tiny_config(layers=2, tie=True, theta=1e6):
    from transformers import Qwen2Config

    cfg = Qwen2Config(hidden_size=512, intermediate_size=1024, num_hidden_layers=layers, num_attention_heads=4,
                      num_key_value_heads=2, head_dim=128, vocab_size=4096, rope_theta=theta,
                      tie_word_embeddings=tie, rms_norm_eps=1e-6, max_position_embeddings=4096)
    cfg._attn_implementation = "eager"
    return cfg


def hf_model(cfg, seed=0):
    from transformers import Qwen2ForCausalLM

    from irgen.hf_qwen import to_dtype_keep_rotary

    torch.manual_seed(seed)
    return to_dtype_keep_rotary(Qwen2ForCausalLM(cfg).eval())


@pytest.fixture(scope="module")
def model():
    return hf_model(tiny_config())


@pytest.fixture(scope="module")
def graphs(model):
    from irgen.hf_qwen import export_qwen

    return export_qwen(model, S, tokens=1, argmax=True), export_qwen(model, S, tokens=16, argmax=True)


def ir_weights(model, ir):
    sd = dict(model.state_dict())
    sd.update(dict(model.named_buffers()))
    return {w["name"]: sd[w["name"]] for w in ir["weights"]}


def host(t):
    t = t.contiguous()
    return t.view(torch.uint16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def cpu_executor(ir, weights):
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    ex = DAGExecutor(partition(ir, lambda *_: False), None)
    ex.load_weights(weights)
    return ex


def as_torch(a, like):
    a = np.asarray(a)
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.view(torch.bfloat16) if like.dtype == torch.bfloat16 else t


def decode_args(model, pos, seed=1):
    g = torch.Generator().manual_seed(seed)
    cfg = model.config
    kv = [torch.randn(1, 2, S, 128, generator=g).to(torch.bfloat16) for _ in range(2 * cfg.num_hidden_layers)]
    mask = torch.zeros(1, 1, 1, S, dtype=torch.bfloat16)
    mask[..., pos + 1:] = float("-inf")
    ids = torch.randint(0, cfg.vocab_size, (1, 1), generator=g)
    return (ids, mask, torch.tensor([[pos]]), torch.tensor([pos]), *kv)


def prefill_args(model, T=16, seed=2):
    g = torch.Generator().manual_seed(seed)
    cfg = model.config
    kv = [torch.zeros(1, 2, S, 128, dtype=torch.bfloat16) for _ in range(2 * cfg.num_hidden_layers)]
    mask = torch.full((T, S), float("-inf"))
    mask[:, :T] = torch.triu(torch.full((T, T), float("-inf")), diagonal=1)
    ids = torch.randint(0, cfg.vocab_size, (1, T), generator=g)
    ar = torch.arange(T)
    return (ids, mask.to(torch.bfloat16).reshape(1, 1, T, S), ar.reshape(1, T), ar, *kv)


@pytest.mark.parametrize("which", ["decode", "prefill"])
def test_exported_graph_through_cpu_fallback_equals_hf_forward_bit_for_bit(model, graphs, which):
    from irgen.hf_qwen import QwenStaticWrapper

    ir = graphs[0] if which == "decode" else graphs[1]
    args = decode_args(model, 100) if which == "decode" else prefill_args(model)
    with torch.no_grad():
        ref = QwenStaticWrapper(model, model.config.num_hidden_layers, argmax=True)(*args)
    ex = cpu_executor(ir, ir_weights(model, ir))
    out = ex.execute({s["name"]: host(a) for s, a in zip(ir["graph_inputs"], args)})
    assert len(ir["graph_outputs"]) == len(ref)
    for spec, r in zip(ir["graph_outputs"], ref):
        got = as_torch(out[spec["name"]], r).reshape(r.shape)
        assert torch.equal(got, r), spec["name"]


def _ops(ir, drop):
    return [n["op_type"] for n in ir["nodes"] if n["op_type"] not in drop]


@pytest.mark.parametrize("tokens", [1, 16])
def test_exported_ops_follow_the_irgen_builder(model, graphs, tokens):
    """Same ATen op sequence as ``irgen.qwen.build_decode_ir``, apart from what this
    image's transformers does differently from the reference's: an ``alias`` (the
    ``logits_to_keep`` slice) before the lm_head, and for one token no ``contiguous``
    before the head reshape (export drops it there, the tensor already being
    contiguous)."""
    from irgen.qwen import QwenConfig, build_decode_ir

    ir = graphs[0] if tokens == 1 else graphs[1]
    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    ref = build_decode_ir(S, cfg, argmax=True, tokens=tokens)
    assert _ops(ir, {"aten.alias.default", "aten.contiguous.default"}) == _ops(ref, {"aten.contiguous.default"})
    if tokens > 1:
        assert _ops(ir, {"aten.alias.default"}) == _ops(ref, set())
    assert [g["name"] for g in ir["graph_inputs"]] == [g["name"] for g in ref["graph_inputs"]]
    assert [(g["shape"], g["dtype"]) for g in ir["graph_inputs"]] == [(g["shape"], g["dtype"]) for g in ref["graph_inputs"]]
    assert [(g["shape"], g["dtype"]) for g in ir["graph_outputs"]] == [(g["shape"], g["dtype"]) for g in ref["graph_outputs"]]
    # tied embeddings: one matrix, named by the lm_head here and by the embedding in irgen
    tied = {"lm_head.weight": "model.embed_tokens.weight"}
    assert {tied.get(w["name"], w["name"]) for w in ir["weights"]} == {w["name"] for w in ref["weights"]}
    rot = [n for n in ir["nodes"] if n["op_type"] == "wrap_with_set_grad_enabled"]
    assert len(rot) == 1 and [i["name"] for i in rot[0]["inputs"]][1] == "position_ids"
    assert rot[0]["attrs"] == {}   # attention_scaling 1


@pytest.mark.parametrize("tokens", [1, 16])
def test_exported_graph_lowers_to_the_irgen_launch_list(graphs, tokens):
    from hip_compiler import compile_subgraph
    from irgen.qwen import QwenConfig, build_decode_ir

    ir = graphs[0] if tokens == 1 else graphs[1]
    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    a = compile_subgraph(ir)
    b = compile_subgraph(build_decode_ir(S, cfg, argmax=True, tokens=tokens))
    assert [(s.kernel, s.grid) for s in a.steps] == [(s.kernel, s.grid) for s in b.steps]
    assert a.arena_bytes == b.arena_bytes


def test_bf16_inv_freq_takes_the_unfused_rotary_and_still_compiles():
    """A model cast wholesale to bf16 (inv_freq rounded) is outside the fused RoPE
    kernels' contract; the q/k/v group then lowers op by op instead of failing."""
    from hip_compiler import compile_subgraph
    from irgen.hf_qwen import export_qwen
    from transformers import Qwen2ForCausalLM

    with torch.device("meta"):
        m = Qwen2ForCausalLM(tiny_config()).eval().to(torch.bfloat16)
    ir = export_qwen(m, S, tokens=1)
    kernels = [s.kernel for s in compile_subgraph(ir).steps]
    assert "k_rope_table" in kernels and not any(k.startswith("k_qkv_rope") for k in kernels)


def test_kv_mapping_record(graphs):
    from irgen.hf_qwen import kv_mapping

    dec, pre = graphs
    m = kv_mapping(pre, dec, 2, 16, S)
    assert json.loads(json.dumps(m)) == m
    assert (m["num_layers"], m["prefill_seq_len"], m["max_cache_len"]) == (2, 16, S)
    dnodes = {o["name"]: n for n in dec["nodes"] for o in n["outputs"]}
    pnodes = {o["name"]: n for n in pre["nodes"] for o in n["outputs"]}
    for i, layer in enumerate(m["layers"]):
        assert (layer["decode_key_input"], layer["decode_value_input"]) == (f"past_key_{i}", f"past_value_{i}")
        for k in ("decode_key_output", "decode_value_output"):
            assert dnodes[layer[k]]["op_type"] == "aten.index_copy.default"
        for k in ("prefill_key_output", "prefill_value_output"):
            assert pnodes[layer[k]]["op_type"] == "aten.index_copy.default"
        # the cache the decode output updates is the decode input of the same layer and kind
        assert dnodes[layer["decode_key_output"]]["inputs"][0]["name"] == layer["decode_key_input"]
        assert dnodes[layer["decode_value_output"]]["inputs"][0]["name"] == layer["decode_value_input"]


class _Odd(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = torch.nn.Linear(16, 24, bias=False)
        self.register_buffer("scale", torch.linspace(0.5, 1.5, 24))

    def forward(self, x):
        with torch.no_grad():
            s = self.scale.exp() + 1.0
        y = self.lin(x) * s
        y = y.view(2, -1, 6) + 0.25
        return torch.softmax(y, dim=-1), y.sum(dim=1)


def test_non_rotary_no_grad_region_is_inlined_and_attrs_follow_the_schema():
    from irgen.exporter import extract_ir
    from npu_runtime.aten_executor import run_node

    torch.manual_seed(0)
    m = _Odd().eval()
    x = torch.randn(2, 3, 16)
    ir = extract_ir(m, (x,), model_name="odd", input_names=["x"])
    ops = [n["op_type"] for n in ir["nodes"]]
    assert "wrap_with_set_grad_enabled" not in ops and "aten.exp.default" in ops
    view = next(n for n in ir["nodes"] if n["op_type"] == "aten.view.default")
    assert view["attrs"]["size"] == [2, 12, 6]             # -1 resolved from the output shape
    add = next(n for n in ir["nodes"] if n["op_type"] == "aten.add.Tensor" and "other" in n["attrs"])
    assert len(add["inputs"]) == 1                          # the scalar-binary form
    lin = next(n for n in ir["nodes"] if n["op_type"] == "aten.linear.default")
    assert len(lin["inputs"]) == 2                          # no bias
    assert {w["name"] for w in ir["weights"]} == {"lin.weight", "scale"}
    env = {"x": x}
    sd = dict(m.state_dict())
    for ph, key in ir["weight_name_mapping"].items():
        env[ph] = sd[key]
    with torch.no_grad():
        for n in ir["nodes"]:
            run_node(n, env)
        ref = m(x)
    for spec, r in zip(ir["graph_outputs"], ref):
        assert torch.equal(env[spec["name"]], r)


@pytest.mark.parametrize("shard", [False, True])
def test_safetensors_loader_matches_the_state_dict(model, graphs, tmp_path, shard):
    from npu_runtime.hf_weights import load_safetensors_weights

    kw = {"max_shard_size": "2MB"} if shard else {}
    model.save_pretrained(str(tmp_path), safe_serialization=True, **kw)
    assert (tmp_path / "model.safetensors.index.json").exists() == shard
    ir = graphs[0]
    got = load_safetensors_weights(str(tmp_path), ir)
    ref = ir_weights(model, ir)
    assert set(got) == set(ref)
    for k, v in ref.items():
        assert got[k].dtype == v.dtype and torch.equal(got[k], v), k


def test_safetensors_loader_synthesises_inv_freq_with_the_configs_theta(tmp_path):
    """inv_freq is not in a checkpoint (a non-persistent buffer); it is rebuilt in fp32
    with rope_theta from config.json, bit-equal to what HF computes."""
    from npu_runtime.hf_weights import load_safetensors_weights

    m = hf_model(tiny_config(layers=1, theta=10000.0), seed=3)
    m.save_pretrained(str(tmp_path), safe_serialization=True)
    ir = {"weights": [{"name": "model.rotary_emb.inv_freq", "shape": [64], "dtype": "float32"},
                      {"name": "lifted_tensor_0", "shape": [0], "dtype": "bfloat16"}]}
    got = load_safetensors_weights(str(tmp_path), ir)
    assert torch.equal(got["model.rotary_emb.inv_freq"], m.model.rotary_emb.inv_freq)
    assert got["lifted_tensor_0"].numel() == 0
    with pytest.raises(KeyError):
        load_safetensors_weights(str(tmp_path), {"weights": [{"name": "nope.weight", "shape": [1], "dtype": "bfloat16"}]})


def _hf_static_greedy(model, prompt, T, max_tokens):
    """The reference's loop (`examples/run_qwen.py:84-200`) driven through HF's own
    forward over the same static caches: padded prefill, then one token per step."""
    from irgen.hf_qwen import QwenStaticWrapper
    from npu_runtime.generation import decode_mask, prefill_mask

    L = model.config.num_hidden_layers
    w = QwenStaticWrapper(model, L)
    n = len(prompt)
    ids = torch.zeros(1, T, dtype=torch.int64)
    ids[0, :n] = torch.tensor(prompt)
    kv = [torch.zeros(1, 2, S, 128, dtype=torch.bfloat16) for _ in range(2 * L)]
    bf = lambda a: torch.from_numpy(a).view(torch.bfloat16)   # noqa: E731
    ar = torch.arange(T)
    with torch.no_grad():
        out = w(ids, bf(prefill_mask(T, S, n)), ar.reshape(1, T), ar, *kv)
        toks = [int(torch.argmax(out[0][0, n - 1].float()))]
        kv = list(out[1:])
        for step in range(max_tokens - 1):
            pos = n + step
            out = w(torch.tensor([[toks[-1]]]), bf(decode_mask(S, pos)), torch.tensor([[pos]]), torch.tensor([pos]),
                    *kv)
            toks.append(int(torch.argmax(out[0][0, -1].float())))
            kv = list(out[1:])
    return toks


def test_greedy_generator_on_the_cpu_fallback_equals_hfs_own_loop(model, graphs):
    """Padded 16-token prefill graph with an 11-token prompt, then 6 decode steps, both
    graphs through all-CPU DAGExecutors; tokens equal HF's forward driven by the
    reference's loop, and the prompt's first token equals HF ``generate``'s."""
    from irgen.hf_qwen import kv_mapping
    from npu_runtime.generation import GreedyGenerator

    dec, pre = graphs
    prompt = [int(t) for t in torch.randint(0, 4096, (11,), generator=torch.Generator().manual_seed(5))]
    gen = GreedyGenerator(cpu_executor(pre, ir_weights(model, pre)), cpu_executor(dec, ir_weights(model, dec)),
                          kv_mapping(pre, dec, 2, 16, S), pre, dec)
    res = gen.generate(prompt, 7)
    assert res.prompt_len == 11 and len(res.tokens) == 7
    assert res.tokens == _hf_static_greedy(model, prompt, 16, 7)
    with torch.no_grad():
        hf = model.generate(torch.tensor([prompt]), max_new_tokens=1, do_sample=False)
    assert int(hf[0, -1]) == res.tokens[0]
    # stopping at EOS drops the EOS token and everything after it, as the reference does
    eos = res.tokens[3]
    cut = gen.generate(prompt, 7, eos_token_id=eos)
    assert cut.tokens == res.tokens[:res.tokens.index(eos)]


def test_generator_rejects_prompts_that_do_not_fit(model, graphs):
    from irgen.hf_qwen import kv_mapping
    from npu_runtime.generation import GreedyGenerator

    dec, pre = graphs
    gen = GreedyGenerator(None, None, kv_mapping(pre, dec, 2, 16, S), pre, dec)
    with pytest.raises(ValueError):
        gen.generate([], 4)
    with pytest.raises(ValueError):
        gen.generate(list(range(17)), 4)
    with pytest.raises(ValueError):
        gen.generate(list(range(16)), S)


def test_prefill_mask_is_causal_and_keeps_padding_rows_open():
    """Real rows see no padding column; padding rows stay causal, so no row is fully
    closed (a softmax over an all ``-inf`` row is NaN in ATen)."""
    from npu_runtime.generation import decode_mask, prefill_mask

    m = torch.from_numpy(prefill_mask(6, 10, 4)).view(torch.bfloat16).float()[0, 0]
    for i in range(6):
        for j in range(10):
            assert m[i, j] == (0.0 if j <= i else float("-inf"))
    assert bool(torch.isfinite(m).any(dim=1).all())
    d = torch.from_numpy(decode_mask(10, 6)).view(torch.bfloat16).float().reshape(-1)
    assert d[:7].eq(0).all() and d[7:].eq(float("-inf")).all()
    with pytest.raises(ValueError):
        prefill_mask(6, 5, 4)


def test_full_size_qwen2_5_export_lowers_to_the_bench_launch_list():
    """Qwen2.5-1.5B's architecture (28 layers, vocab 151936) on the meta device: the
    exported decode graph over a 2048 cache lowers to the benchmark graph's 143 launches."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from hip_compiler import compile_subgraph
    from irgen.hf_qwen import export_qwen, to_dtype_keep_rotary
    from irgen.qwen import build_decode_ir

    cfg = Qwen2Config(hidden_size=1536, intermediate_size=8960, num_hidden_layers=28, num_attention_heads=12,
                      num_key_value_heads=2, head_dim=128, vocab_size=151936, rope_theta=1e6,
                      tie_word_embeddings=True, rms_norm_eps=1e-6, max_position_embeddings=32768)
    cfg._attn_implementation = "eager"
    with torch.device("meta"):
        m = to_dtype_keep_rotary(Qwen2ForCausalLM(cfg).eval())
    ea = export_qwen(m, 2048, tokens=1, argmax=True)
    a = compile_subgraph(ea, persistent=False)
    b = compile_subgraph(build_decode_ir(2048, argmax=True), persistent=False)
    assert len(a.steps) == 143
    assert [(s.kernel, s.grid, s.lds) for s in a.steps] == [(s.kernel, s.grid, s.lds) for s in b.steps]
    # and both become the same single persistent launch by default
    pa, pb = compile_subgraph(ea), compile_subgraph(build_decode_ir(2048, argmax=True))
    assert [s.kernel for s in pa.steps] == [s.kernel for s in pb.steps] == ["k_decode_step_k3_i3_e2"]


def test_safetensors_loader_theta_default_is_hfs(tmp_path, model):
    """No rope_theta in config.json: inv_freq is built with Qwen2Config's default (10000),
    as HF itself would build it."""
    import json as _json

    from npu_runtime.hf_weights import load_safetensors_weights
    from transformers import Qwen2Config

    model.save_pretrained(str(tmp_path), safe_serialization=True)
    cfgp = tmp_path / "config.json"
    c = _json.loads(cfgp.read_text())
    c.pop("rope_theta", None)
    c.pop("rope_parameters", None)
    cfgp.write_text(_json.dumps(c))
    ir = {"weights": [{"name": "model.rotary_emb.inv_freq", "shape": [64], "dtype": "float32"}]}
    got = load_safetensors_weights(str(tmp_path), ir)["model.rotary_emb.inv_freq"]
    theta = Qwen2Config().rope_parameters["rope_theta"] if hasattr(Qwen2Config(), "rope_parameters") \
        else Qwen2Config().rope_theta
    want = 1.0 / (theta ** (torch.arange(0, 128, 2, dtype=torch.int64).float() / 128))
    assert theta == 10000.0 and torch.equal(got, want)
