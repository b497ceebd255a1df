"""HF Qwen2 → exported IR → HIP path, on the GPU.

The model is this image's transformers ``Qwen2ForCausalLM`` (random init, eager
attention), exported with ``irgen.hf_qwen.export_qwen``, saved as safetensors and
loaded straight into device memory by ``npu_runtime.hf_weights``. The reference for
every comparison is HF's own eager forward on the CPU (ATen bf16). Tolerances:
rtol 2e-2 of the output's largest magnitude for floating point, bit-exact for cache
rows the step does not write, and the next token equal to HF's argmax unless HF's
top two logits are within that tolerance (a near tie).
"""

import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]
transformers = pytest.importorskip("transformers")

RTOL = 2e-2
S = 256


def tiny_model(layers=2, seed=0):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from irgen.hf_qwen import to_dtype_keep_rotary

    cfg = Qwen2Config(hidden_size=1536, intermediate_size=8960, num_hidden_layers=layers, num_attention_heads=12,
                      num_key_value_heads=2, head_dim=128, vocab_size=8192, rope_theta=1e6,
                      tie_word_embeddings=True, rms_norm_eps=1e-6, max_position_embeddings=4096)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    m = Qwen2ForCausalLM(cfg).eval()
    with torch.no_grad():   # HF's init gives near-constant logits at this size; widen them
        m.model.embed_tokens.weight.normal_(0, 0.5)
    return to_dtype_keep_rotary(m)


@pytest.fixture(scope="module")
def hf(tmp_path_factory):
    m = tiny_model()
    d = tmp_path_factory.mktemp("qwen2")
    m.save_pretrained(str(d), safe_serialization=True)
    return m, str(d)


def hip_executor(ir, model_dir, backend):
    from hip_compiler import compile_subgraph, is_hip_op_supported
    from npu_compiler import partition
    from npu_runtime import DAGExecutor
    from npu_runtime.hf_weights import load_safetensors_weights

    plan = partition(ir, is_hip_op_supported)
    assert [p.target for p in plan.steps] == ["npu"], "the exported graph must run as one device partition"
    ex = DAGExecutor(plan, backend, compile_fn=compile_subgraph)
    ex.load_weights(load_safetensors_weights(model_dir, ir, device="cuda"))
    return ex


def f32(t):
    return t.float().cpu()


def close(got, ref, rtol=RTOL):
    g, r = f32(got), f32(ref)
    assert g.shape == r.shape
    err = (g - r).abs().max().item()
    scale = max(r.abs().max().item(), 1e-6)
    assert err <= rtol * scale, f"max abs err {err} vs scale {scale}"
    return err / scale


def token_ok(tok, logits_row):
    r = logits_row.float()
    best = r.max().item()
    return int(tok) == int(r.argmax()) or r[int(tok)].item() >= best - RTOL * r.abs().max().item()


def test_exported_decode_step_on_hip_matches_hf(hf, backend):
    from irgen.hf_qwen import QwenStaticWrapper, export_qwen

    m, d = hf
    ir = export_qwen(m, S, tokens=1, argmax=True)
    ex = hip_executor(ir, d, backend)
    pos = 200
    g = torch.Generator().manual_seed(1)
    kv = [torch.randn(1, 2, S, 128, generator=g).to(torch.bfloat16) for _ in range(4)]
    mask = torch.zeros(1, 1, 1, S, dtype=torch.bfloat16)
    mask[..., pos + 1:] = float("-inf")
    args = (torch.tensor([[4321]]), mask, torch.tensor([[pos]]), torch.tensor([pos]), *kv)
    with torch.no_grad():
        ref = QwenStaticWrapper(m, 2, argmax=True)(*args)
    print(f"[case] exported decode, S={S}, pos={pos}", flush=True)
    out = ex.execute({s["name"]: backend.allocate_buffer(a.clone()) for s, a in zip(ir["graph_inputs"], args)})
    names = [o["name"] for o in ir["graph_outputs"]]
    logits = out[names[0]].to_torch()
    close(logits, ref[0])
    assert token_ok(out[names[-1]].to_torch().reshape(-1)[0].item(), ref[0].reshape(-1))
    for name, r in zip(names[1:-1], ref[1:-1]):
        got = f32(out[name].to_torch())
        rr = f32(r)
        keep = torch.ones(S, dtype=torch.bool)
        keep[pos] = False
        assert torch.equal(got[:, :, keep], rr[:, :, keep]), name
        close(got[:, :, pos], rr[:, :, pos])


def test_exported_prefill_on_hip_matches_hf(hf, backend):
    from irgen.hf_qwen import QwenStaticWrapper, export_qwen

    m, d = hf
    T = 64
    ir = export_qwen(m, S, tokens=T, argmax=True)
    ex = hip_executor(ir, d, backend)
    g = torch.Generator().manual_seed(2)
    mask = torch.full((T, S), float("-inf"))
    mask[:, :T] = torch.triu(torch.full((T, T), float("-inf")), diagonal=1)
    ar = torch.arange(T)
    kv = [torch.zeros(1, 2, S, 128, dtype=torch.bfloat16) for _ in range(4)]
    args = (torch.randint(0, 8192, (1, T), generator=g), mask.to(torch.bfloat16).reshape(1, 1, T, S),
            ar.reshape(1, T), ar, *kv)
    with torch.no_grad():
        ref = QwenStaticWrapper(m, 2, argmax=True)(*args)
    print(f"[case] exported prefill, T={T}, S={S}", flush=True)
    out = ex.execute({s["name"]: backend.allocate_buffer(a.clone()) for s, a in zip(ir["graph_inputs"], args)})
    names = [o["name"] for o in ir["graph_outputs"]]
    close(out[names[0]].to_torch(), ref[0])
    toks = out[names[-1]].to_torch().reshape(-1).cpu()
    rl = ref[0].reshape(T, -1)
    assert all(token_ok(toks[i], rl[i]) for i in range(T))
    for name, r in zip(names[1:-1], ref[1:-1]):
        got = f32(out[name].to_torch())
        close(got[:, :, :T], f32(r)[:, :, :T])
        assert got[:, :, T:].eq(0).all()


def test_generation_on_hip_follows_hf_teacher_forced(hf, backend):
    """Padded 32-token prefill graph, a 23-token prompt, then 12 device-resident decode
    steps. Every generated token must be HF's argmax (or a near tie) given the tokens
    before it, from one uncached HF forward over the whole sequence."""
    from irgen.hf_qwen import export_qwen, kv_mapping
    from npu_runtime.generation import GreedyGenerator

    m, d = hf
    T = 32
    pre = export_qwen(m, S, tokens=T, argmax=True)
    dec = export_qwen(m, S, tokens=1, argmax=True)
    gen = GreedyGenerator(hip_executor(pre, d, backend), hip_executor(dec, d, backend),
                          kv_mapping(pre, dec, 2, T, S), pre, dec, backend=backend)
    prompt = [int(t) for t in torch.randint(0, 8192, (23,), generator=torch.Generator().manual_seed(7))]
    print("[case] generation, prompt 23 / prefill 32 / 13 tokens", flush=True)
    res = gen.generate(prompt, 13)
    assert len(res.tokens) == 13
    seq = torch.tensor([prompt + res.tokens[:-1]])
    with torch.no_grad():
        logits = m(seq).logits[0]
    for i, tok in enumerate(res.tokens):
        assert token_ok(tok, logits[len(prompt) - 1 + i]), f"step {i}: token {tok}"
    again = gen.generate(prompt, 13)        # caches are fresh per call: same tokens
    assert again.tokens == res.tokens
    eos = res.tokens[5]
    cut = gen.generate(prompt, 13, eos_token_id=eos)
    assert cut.tokens == res.tokens[:res.tokens.index(eos)]


def test_generator_raises_when_the_decode_step_timed_out(hf, backend):
    """A persistent decode step's timeout word (set from the host, as a timed-out workgroup sets
    it) makes GreedyGenerator.generate raise instead of returning the step's tokens."""
    import torch as _t

    from irgen.hf_qwen import export_qwen, kv_mapping
    from npu_runtime.generation import GreedyGenerator

    m, d = hf
    T = 32
    pre = export_qwen(m, S, tokens=T, argmax=True)
    dec = export_qwen(m, S, tokens=1, argmax=True)
    dex = hip_executor(dec, d, backend)
    gen = GreedyGenerator(hip_executor(pre, d, backend), dex, kv_mapping(pre, dec, 2, T, S), pre, dec,
                          backend=backend)
    (h,) = dex.npu_executors.values()
    assert h.program.steps[0].kind == "decode_step"
    prompt = [3, 14, 15, 92, 65]
    print("[case] generator timeout report", flush=True)
    ok = gen.generate(prompt, 4)
    st = h.program.steps[0]
    off = h.program.storages[st.args["ll"].storage].offset + (int(st.params["exchange_words"]) - 1) * 4
    h.arena[off:off + 4].view(_t.int32).fill_(1)
    with pytest.raises(RuntimeError, match="timed out"):
        gen.generate(prompt, 4)
    assert gen.generate(prompt, 4).tokens == ok.tokens   # cleared by the report


def test_program_from_hipbin_runs_bit_identical(backend, tmp_path):
    """A decode program written to and read back from a ``.hipbin`` file produces the same
    bits as the freshly compiled one, and matches the CPU fallback (ATen) on the same
    inputs: logits within 2e-2 of the largest, the same next token, the cache rows the step
    does not write bit-exact and the one it writes within 2e-2."""
    from hip_compiler import compile_subgraph, is_hip_op_supported
    from hip_compiler.program_io import compile_cached
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights, to_host
    from npu_compiler import partition
    from npu_runtime import DAGExecutor
    from oracle.numpy_ref import bf16_bits_to_f32

    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    ir = build_decode_ir(256, cfg, argmax=True)
    w = make_weights(ir, cfg, device="cuda")
    x = decode_inputs(256, 100, cfg)
    compile_cached(ir, str(tmp_path))                       # writes the file
    outs = []
    for fn in (compile_subgraph, lambda sub: compile_cached(sub, str(tmp_path))):
        ex = DAGExecutor(partition(ir, is_hip_op_supported), backend, compile_fn=fn)
        ex.load_weights(w)
        print("[case] hipbin vs fresh compile", flush=True)
        o = ex.execute({k: backend.allocate_buffer(v.clone()) for k, v in x.items()})
        outs.append({k: v.to_torch().cpu() for k, v in o.items()})
    assert outs[0].keys() == outs[1].keys()
    for k in outs[0]:
        assert torch.equal(outs[0][k], outs[1][k]), k
    print("[case] hipbin program vs CPU fallback", flush=True)
    cpu = DAGExecutor(partition(ir, lambda *_: False), None)
    cpu.load_weights({k: to_host(v) for k, v in w.items()})
    ref = cpu.execute({k: to_host(v) for k, v in x.items()})

    def as_f32(a):
        a = np.asarray(a)
        return bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)

    got = outs[1]
    lg = ir["graph_outputs"][0]["name"]
    g, r = got[lg].float().numpy(), as_f32(ref[lg])
    assert float(np.abs(g - r).max()) <= RTOL * float(np.abs(r).max())
    assert int(got["next_token"].reshape(-1)[0]) == int(np.argmax(r.reshape(-1)))
    for o in ir["graph_outputs"][1:-1]:
        gc, rc = got[o["name"]].float().numpy(), as_f32(ref[o["name"]])
        keep = np.ones(gc.shape[2], bool)
        keep[100] = False
        assert np.array_equal(gc[:, :, keep], rc[:, :, keep]), o["name"]
        err = float(np.abs(gc[:, :, 100] - rc[:, :, 100]).max())
        assert err <= RTOL * max(float(np.abs(rc[:, :, 100]).max()), 1e-6), o["name"]


def test_executor_keeps_one_graph_per_pointer_set(backend):
    """Two input_ids buffers used in turn: A, B, A. The third run relaunches the graph
    captured for A and must reproduce A's first run bit for bit (a graph holds its own
    kernel arguments), and B's run must differ from it."""
    from hip_compiler import compile_subgraph, is_hip_op_supported
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    ir = build_decode_ir(256, cfg, argmax=True)
    ex = DAGExecutor(partition(ir, is_hip_op_supported), backend, compile_fn=compile_subgraph)
    ex.load_weights(make_weights(ir, cfg, device="cuda"))
    (hexec,) = ex._npu_executors.values()
    hexec.use_graph = True   # (a one-launch program is launched directly by default)
    st = {k: backend.allocate_buffer(v.clone()) for k, v in decode_inputs(256, 100, cfg).items()}
    a = backend.allocate_buffer(torch.tensor([[11]]))
    b = backend.allocate_buffer(torch.tensor([[3000]]))
    lname = ir["graph_outputs"][0]["name"]
    runs = []
    for ids in (a, b, a):
        print("[case] graph per pointer set", flush=True)
        out = ex.execute({**st, "input_ids": ids})
        runs.append(out[lname].to_torch().clone())
    assert len(hexec._graphs) == 2
    assert torch.equal(runs[0], runs[2])
    assert not torch.equal(runs[0], runs[1])


def test_long_generation_across_attention_splits(hf, backend):
    """A 32-token prompt filling the prefill graph (no padding), then 120 device-resident
    decode steps at positions 32..151: the in-place mask / position updates and the split-S
    attention cross several 64- and 128-position split boundaries. Every token must be HF's
    argmax (or a near tie) given the tokens before it."""
    from irgen.hf_qwen import export_qwen, kv_mapping
    from npu_runtime.generation import GreedyGenerator

    m, d = hf
    T = 32
    pre = export_qwen(m, S, tokens=T, argmax=True)
    dec = export_qwen(m, S, tokens=1, argmax=True)
    gen = GreedyGenerator(hip_executor(pre, d, backend), hip_executor(dec, d, backend),
                          kv_mapping(pre, dec, 2, T, S), pre, dec, backend=backend)
    prompt = [int(t) for t in torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(9))]
    print("[case] generation, prompt 32 / prefill 32 / 121 tokens", flush=True)
    res = gen.generate(prompt, 121)
    assert len(res.tokens) == 121 and res.decode_tok_s > 0
    seq = torch.tensor([prompt + res.tokens[:-1]])
    with torch.no_grad():
        logits = m(seq).logits[0]
    bad = [i for i, tok in enumerate(res.tokens) if not token_ok(tok, logits[T - 1 + i])]
    assert not bad, f"steps {bad[:5]} differ from HF beyond a near tie"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_decode_advance_moves_positions_and_opens_one_mask_entry(backend, dt):
    """k_decode_advance: p = cache_position + 1 written to both position inputs, mask[p] = 0,
    every other mask entry untouched; at the last cache position it changes nothing."""
    S = 16
    mask = torch.full((1, 1, 1, S), float("-inf"))
    mask[..., :4] = 0.0
    mb = backend.allocate_buffer(mask.to(dt))
    pb = backend.allocate_buffer(torch.tensor([[3]]))
    cb = backend.allocate_buffer(torch.tensor([3]))
    adv = backend.decode_advance(mb, pb, cb)
    for p in range(4, S):
        print(f"[case] decode advance to {p} ({dt})", flush=True)
        adv()
        torch.cuda.synchronize()
        m = mb.to_torch().float().reshape(-1).cpu()
        assert int(pb.to_torch().item()) == p and int(cb.to_torch().item()) == p
        assert m[:p + 1].eq(0).all() and m[p + 1:].eq(float("-inf")).all()
    adv.check()   # every step so far stayed inside the cache
    adv()   # at S - 1: no position past the cache; the overflow flag is raised instead
    torch.cuda.synchronize()
    assert int(cb.to_torch().item()) == S - 1 and int(pb.to_torch().item()) == S - 1
    with pytest.raises(RuntimeError, match="past the end"):
        adv.check()
    adv.clear()
    adv.check()
