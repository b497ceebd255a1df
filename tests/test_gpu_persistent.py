"""The persistent decode step (one launch per step, csrc/kernels/decode.hip) against the CPU
fallback (ATen) and against the multi-kernel launch list it replaces, on the GPU.

Tolerances: logits and the K/V rows written within 2e-2 of the largest magnitude (the
north-star bound), the next token equal to the argmax of the CPU path's logits, the cache rows
the step does not write bit-exact. The full 28-layer model is covered by
test_gpu_parity.py::test_full_model_logits_as_close_to_fp32_as_the_cpu_path, which compiles
the default (persistent) program.
"""

import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

RTOL = 2e-2


def _f32(a):
    from oracle.numpy_ref import bf16_bits_to_f32

    a = np.asarray(a)
    return bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)


def _close(got, ref, rtol=RTOL):
    g, r = _f32(got), _f32(ref)
    err = float(np.abs(g - r).max())
    scale = max(float(np.abs(r).max()), 1e-6)
    assert err <= rtol * scale, f"max abs err {err} vs scale {scale}"
    return err / scale


def _host(d):
    from irgen.workloads import to_host

    return {k: to_host(v) for k, v in d.items()}


def _executor(ir, backend, persistent):
    from hip_compiler import compile_subgraph, is_hip_op_supported
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    ex = DAGExecutor(partition(ir, is_hip_op_supported), backend,
                     compile_fn=lambda sub: compile_subgraph(sub, persistent=persistent))
    (prog,) = ex.npu_programs.values()
    kernels = [s.kernel for s in prog.steps]
    if persistent:
        assert len(kernels) == 1 and kernels[0].startswith("k_decode_step_"), kernels
        import hip_compiler.persistent as P

        S = int(prog.steps[0].args["S"])
        assert kernels[0].endswith("_kv") == (S >= P.KV_MAJOR_MIN_S), kernels   # KV-head-major for long caches
    else:
        assert len(kernels) > 1
    return ex


def _hexec(ex):
    (h,) = ex._npu_executors.values()
    return h


def _cpu(ir, x, w):
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    ex = DAGExecutor(partition(ir, lambda *_: False), None)
    ex.load_weights(w)
    return ex.execute(x)


CASES = {
    "mini_s128": (dict(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096), 128, 100),
    "mini_s256_last": (dict(hidden=512, intermediate=1024, layers=3, heads=4, kv_heads=2, head_dim=128, vocab=4096), 256, 255),
    "real_dims_2l": (dict(layers=2), 2048, 1984),
    "real_dims_pos0": (dict(layers=1), 2048, 0),
    # attention slots whose every chunk is closed (positions 0..100 open: slot 0 only)
    "real_dims_pos100": (dict(layers=1), 2048, 100),
    # a cache that is not a multiple of the 128-position chunk (the last chunk is partial)
    "real_s1000_last": (dict(layers=1), 1000, 999),
    # 32 chunks over 16 slots: every slot folds two chunks
    "real_s4096_pos4000": (dict(layers=2), 4096, 4000),
    # the reference's benchmark cache length: 17 open chunks of 256 (slot 0 folds two)
    "real_s32768_pos2048": (dict(layers=2), 32768, 2048),
    "real_s128": (dict(layers=1), 128, 77),
    # KV-head-major attention (taken by default from 12,288 positions; these cases lower the
    # threshold): 64 chunks over 96 slots per KV head (slots 64..95 hold none), the position in
    # the last chunk
    "real_s8192_pos8000_kv": (dict(layers=2), 8192, 8000),
    # ragged: 40 chunks, the last one partial, the last position
    "real_s5000_last_kv": (dict(layers=1), 5000, 4999),
    # G = 2: 32 slots per KV head, 2 chunks each
    "mini_s8192_pos6000_kv": (dict(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096), 8192, 6000),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_persistent_step_vs_cpu_fallback_and_launch_list(backend, case, monkeypatch):
    import hip_compiler.persistent as P
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    kw, S, pos = CASES[case]
    if case.endswith("_kv"):
        monkeypatch.setattr(P, "KV_MAJOR_MIN_S", 4097)
    cfg = QwenConfig(**kw)
    ir = build_decode_ir(S, cfg, argmax=True)
    w = _host(make_weights(ir, cfg, device="cuda"))
    x = _host(decode_inputs(S, pos, cfg))
    print(f"[case] persistent decode step {case}", flush=True)
    outs = {}
    for persistent in (True, False):
        ex = _executor(ir, backend, persistent)
        ex.load_weights(w)
        o = ex.execute({k: v.copy() for k, v in x.items()})
        outs[persistent] = {k: (v if isinstance(v, np.ndarray) else v.to_numpy()) for k, v in o.items()}
        _hexec(ex).check()   # no workgroup timed out
    ref = _cpu(ir, x, w)
    got, multi = outs[True], outs[False]
    lg = ir["graph_outputs"][0]["name"]
    _close(got[lg], ref[lg])
    _close(got[lg], multi[lg])
    assert int(np.asarray(got["next_token"]).reshape(-1)[0]) == int(np.argmax(_f32(got[lg]).reshape(-1)))
    assert int(np.asarray(got["next_token"]).reshape(-1)[0]) == int(np.argmax(_f32(ref[lg]).reshape(-1)))
    for o in ir["graph_outputs"][1:-1]:
        g, r = np.asarray(got[o["name"]]), np.asarray(ref[o["name"]])
        keep = np.ones(g.shape[2], bool)
        keep[pos] = False
        assert np.array_equal(g[:, :, keep], r[:, :, keep])      # untouched rows: bit-exact
        _close(g[:, :, pos], r[:, :, pos])                          # the row written at `pos`


def test_persistent_greedy_loop_follows_launch_list_and_wraps_step_tags(backend):
    """A device-resident greedy loop on the persistent program (graph relaunched each step, inputs
    advanced on the device): teacher-forced with the launch-list program's tokens, every step's
    logits match within 2e-2 and the tokens agree. The step tag starts near its wrap (65534), so
    the loop crosses 65535 -> 1."""
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    S, start, n = 256, 60, 12
    ir = build_decode_ir(S, cfg, argmax=True)
    w = make_weights(ir, cfg, device="cuda")
    kv_in = [g["name"] for g in ir["graph_inputs"][4:]]
    kv_out = [o["name"] for o in ir["graph_outputs"][1:-1]]
    lg = ir["graph_outputs"][0]["name"]
    runs = {}
    for persistent in (False, True):
        ex = _executor(ir, backend, persistent)
        ex.load_weights(w)
        if persistent:
            h = _hexec(ex)
            st = h.program.steps[0]
            xs = h.program.storages[st.args["ll"].storage]
            ctl = xs.offset + (int(st.params["exchange_words"]) - 2) * 4
            h.arena[ctl:ctl + 4].view(torch.int32).fill_(65534)
        state = {k: backend.allocate_buffer(v) for k, v in decode_inputs(S, start, cfg, device="cuda").items()}
        adv = backend.decode_advance(state["attention_mask"], state["position_ids"], state["cache_position"])
        toks, logits = [], []
        feed = runs.get(False, {}).get("toks")
        for s in range(n):
            print(f"[case] greedy loop persistent={persistent} step {s}", flush=True)
            if feed is not None and s > 0:
                state["input_ids"] = backend.allocate_buffer(torch.tensor([[feed[s - 1]]], device="cuda"))
            out = ex.execute(state)
            toks.append(int(out["next_token"].native_handle.reshape(-1)[0].item()))
            logits.append(out[lg].native_handle.float().cpu().numpy().reshape(-1))
            state["input_ids"] = out["next_token"]
            for i, o in zip(kv_in, kv_out):
                state[i] = out[o]
            if s < n - 1:
                adv()
        torch.cuda.synchronize()
        adv.check()
        if persistent:
            _hexec(ex).check()
            tag = int(h.arena[ctl:ctl + 4].view(torch.int32).item())
            assert tag == ((65534 + n - 1) % 65535) + 1   # 65535, then 1, 2, ... (0 is never a tag)
        runs[persistent] = {"toks": toks, "logits": logits}
    for s in range(n):
        _close(runs[True]["logits"][s], runs[False]["logits"][s])
    assert runs[True]["toks"] == runs[False]["toks"]


def test_one_launch_program_runs_without_a_graph_and_matches_the_graph_launch(backend):
    """A one-launch program (the persistent step) is launched directly by default; the same
    device-resident greedy loop, its inputs advanced inside the step, launched through a captured
    HIP graph instead, gives the same tokens and bit-identical logits at every step."""
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    S, start, n = 256, 30, 8
    ir = build_decode_ir(S, cfg, argmax=True)
    w = make_weights(ir, cfg, device="cuda")
    kv_in = [g["name"] for g in ir["graph_inputs"][4:]]
    kv_out = [o["name"] for o in ir["graph_outputs"][1:-1]]
    lg = ir["graph_outputs"][0]["name"]
    runs = {}
    for graph in (False, True):
        ex = _executor(ir, backend, True)
        ex.load_weights(w)
        h = _hexec(ex)
        assert h.use_graph is False   # the default for one launch
        h.use_graph = graph
        state = {k: backend.allocate_buffer(v) for k, v in decode_inputs(S, start, cfg, device="cuda").items()}
        adv = backend.decode_advance(state["attention_mask"], state["position_ids"], state["cache_position"])
        assert h.fold_advance(adv)
        toks, logits = [], []
        for s in range(n):
            print(f"[case] one-launch loop graph={graph} step {s}", flush=True)
            out = ex.execute(state)
            toks.append(int(out["next_token"].native_handle.reshape(-1)[0].item()))
            logits.append(out[lg].native_handle.clone())
            state["input_ids"] = out["next_token"]
            for i, o in zip(kv_in, kv_out):
                state[i] = out[o]
        torch.cuda.synchronize()
        adv.check()
        h.check()
        assert (len(h._graphs) > 0) == graph   # graphs captured only when asked for
        runs[graph] = (toks, logits)
    assert runs[True][0] == runs[False][0]
    for a, b in zip(runs[True][1], runs[False][1]):
        assert torch.equal(a, b)


def test_folded_advance_matches_separate_launches_and_reports_the_cache_end(backend):
    """``HIPExecutor.fold_advance``: the persistent step moves its own position inputs after each
    step. A greedy loop run that way gives the same tokens and bit-identical logits as the same
    loop with a ``k_decode_advance`` launch after each step; after the step at the last cache
    position the inputs stand at S (mask untouched past the cache), ``check()`` stays quiet, and
    the step launched there sets the flag."""
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    S, start = 256, 244
    n = S - start
    ir = build_decode_ir(S, cfg, argmax=True)
    w = make_weights(ir, cfg, device="cuda")
    kv_in = [g["name"] for g in ir["graph_inputs"][4:]]
    kv_out = [o["name"] for o in ir["graph_outputs"][1:-1]]
    lg = ir["graph_outputs"][0]["name"]
    ex = _executor(ir, backend, True)
    ex.load_weights(w)
    h = _hexec(ex)
    runs = {}
    for fold in (False, True):
        state = {k: backend.allocate_buffer(v) for k, v in decode_inputs(S, start, cfg, device="cuda").items()}
        adv = backend.decode_advance(state["attention_mask"], state["position_ids"], state["cache_position"])
        assert h.fold_advance(adv if fold else None)
        toks, logits = [], []
        for s in range(n):
            print(f"[case] folded advance={fold} step {s}", flush=True)
            out = ex.execute(state)
            toks.append(int(out["next_token"].native_handle.reshape(-1)[0].item()))
            logits.append(out[lg].native_handle.view(torch.int16).cpu().numpy().reshape(-1).copy())
            state["input_ids"] = out["next_token"]
            for i, o in zip(kv_in, kv_out):
                state[i] = out[o]
            if not fold and s < n - 1:
                adv()
        torch.cuda.synchronize()
        adv.check()
        h.check()
        mask = state["attention_mask"].native_handle.float().cpu().numpy().reshape(-1)
        assert np.all(mask[:S] == 0.0)                     # every position of the cache opened
        runs[fold] = (toks, logits)
        if fold:
            assert int(state["cache_position"].native_handle.item()) == S
            assert int(state["position_ids"].native_handle.item()) == S
            print("[case] folded advance: one step past the cache end", flush=True)
            ex.execute(state)
            torch.cuda.synchronize()
            with pytest.raises(RuntimeError):
                adv.check()
            h.fold_advance(None)
    assert runs[True][0] == runs[False][0]
    for a, b in zip(runs[True][1], runs[False][1]):
        assert np.array_equal(a, b)


def test_executor_sees_a_weight_replaced_in_its_dict_and_alternating_inputs(backend):
    """The executor checks a weights dict once, but a buffer replaced inside the same dict (same
    key, new object) is picked up on the next call; two alternating input-buffer sets each keep
    their own pointers. Checked against a fresh executor built with the replaced weight."""
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    S, pos = 128, 40
    ir = build_decode_ir(S, cfg, argmax=True)
    w = make_weights(ir, cfg, device="cuda")
    lg = ir["graph_outputs"][0]["name"]
    ex = _executor(ir, backend, True)
    ex.load_weights(w)
    xa = {k: backend.allocate_buffer(v) for k, v in decode_inputs(S, pos, cfg, device="cuda").items()}
    xb = {k: backend.allocate_buffer(v) for k, v in decode_inputs(S, pos, cfg, device="cuda").items()}
    xb["input_ids"] = backend.allocate_buffer(torch.tensor([[7]], device="cuda"))

    def logits(e, x):
        return e.execute(x)[lg].native_handle.view(torch.int16).cpu().numpy().copy()

    print("[case] alternating input sets", flush=True)
    la, lb = logits(ex, xa), logits(ex, xb)
    assert np.array_equal(logits(ex, xa), la) and np.array_equal(logits(ex, xb), lb)
    assert not np.array_equal(la, lb)
    print("[case] weight replaced in place", flush=True)
    ((pid, prog),) = ex.npu_programs.items()
    wd = ex._npu_weight_cache[pid]
    wmap = getattr(prog, "weight_name_mapping", {})
    name = next(k for k in wd if wmap.get(k, k) == "model.norm.weight")
    old = wd[name].native_handle
    wd[name] = backend.allocate_buffer(old * 2)
    got = logits(ex, xa)
    w2 = dict(w)
    w2["model.norm.weight"] = old * 2
    fresh = _executor(ir, backend, True)
    fresh.load_weights(w2)
    ref = logits(fresh, xa)
    assert np.array_equal(got, ref)
    assert not np.array_equal(got, la)


def test_persistent_step_reads_chunks_the_mask_opens_beyond_the_position(backend):
    """A mask that also opens positions far past cache_position (chunks other slots hold, and a
    chunk of slot 0's second round): those chunks are read and weigh in as on the CPU."""
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    cfg = QwenConfig(layers=1)
    S, pos = 32768, 1500
    ir = build_decode_ir(S, cfg, argmax=True)
    w = _host(make_weights(ir, cfg, device="cuda"))
    xt = decode_inputs(S, pos, cfg)
    m = xt["attention_mask"]
    for p in (2048, 2100, 20000, 31000, 32767):   # chunk 16 (slot 0's second chunk), 156, 242, 255
        m[..., p] = 0.0
    x = _host(xt)
    print("[case] persistent decode step, S 32768, open positions past cache_position", flush=True)
    ex = _executor(ir, backend, True)
    ex.load_weights(w)
    o = ex.execute({k: v.copy() for k, v in x.items()})
    _hexec(ex).check()
    got = {k: (v if isinstance(v, np.ndarray) else v.to_numpy()) for k, v in o.items()}
    ref = _cpu(ir, x, w)
    lg = ir["graph_outputs"][0]["name"]
    _close(got[lg], ref[lg])
    assert int(np.asarray(got["next_token"]).reshape(-1)[0]) == int(np.argmax(_f32(ref[lg]).reshape(-1)))


def test_timeout_flags_raise_on_the_product_path(backend):
    """The step's timeout words, set from the host after a normal step as a timed-out workgroup
    would set them: the host-visible word makes the next execute() raise before launching, the
    device word makes check() raise; both are cleared by the report."""
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    cfg = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)
    ir = build_decode_ir(128, cfg, argmax=True)
    ex = _executor(ir, backend, True)
    ex.load_weights(_host(make_weights(ir, cfg, device="cuda")))
    x = _host(decode_inputs(128, 10, cfg))
    print("[case] timeout flags", flush=True)
    ex.execute({k: v.copy() for k, v in x.items()})
    h = _hexec(ex)
    h.check()
    h._hflag.value = 1
    with pytest.raises(RuntimeError, match="timed out"):
        ex.execute({k: v.copy() for k, v in x.items()})
    ex.execute({k: v.copy() for k, v in x.items()})   # reported once, then cleared
    st = h.program.steps[0]
    off = h.program.storages[st.args["ll"].storage].offset + (int(st.params["exchange_words"]) - 1) * 4
    h.arena[off:off + 4].view(torch.int32).fill_(1)
    with pytest.raises(RuntimeError, match="timed out"):
        h.check()
    h.check()


@pytest.mark.parametrize("persistent", [True, False])
def test_rotary_attention_scaling_on_the_device(backend, persistent):
    """A rotary node with ``attention_scaling`` (0.5): the kernels scale their cos / sin the way the
    CPU fallback does (k_qkv_rope in the launch list, the persistent step's rotary factors)."""
    from irgen.qwen import QwenConfig, build_decode_ir
    from irgen.workloads import decode_inputs, make_weights

    cfg = QwenConfig(layers=2)
    S, pos = 2048, 1500
    ir = build_decode_ir(S, cfg, argmax=True)
    rot = [n for n in ir["nodes"] if n["op_type"] == "wrap_with_set_grad_enabled"]
    assert rot
    for n in rot:
        n.setdefault("attrs", {})["attention_scaling"] = 0.5
    w = _host(make_weights(ir, cfg, device="cuda"))
    x = _host(decode_inputs(S, pos, cfg))
    print(f"[case] rotary attention_scaling, persistent={persistent}", flush=True)
    ex = _executor(ir, backend, persistent)
    (prog,) = ex.npu_programs.values()
    assert any(float(st.args.get("rope_scaling", 1.0)) == 0.5 for st in prog.steps)
    ex.load_weights(w)
    o = ex.execute({k: v.copy() for k, v in x.items()})
    _hexec(ex).check()
    got = {k: (v if isinstance(v, np.ndarray) else v.to_numpy()) for k, v in o.items()}
    ref = _cpu(ir, x, w)
    plain = _cpu(build_decode_ir(S, cfg, argmax=True), x, w)
    lg = ir["graph_outputs"][0]["name"]
    _close(got[lg], ref[lg])
    for o_ in ir["graph_outputs"][1:-1]:   # the K rows written carry the scaled rotation
        _close(np.asarray(got[o_["name"]])[:, :, pos], np.asarray(ref[o_["name"]])[:, :, pos])
    k0 = ir["graph_outputs"][1]["name"]
    assert not np.array_equal(np.asarray(ref[k0])[:, :, pos], np.asarray(plain[k0])[:, :, pos])
