"""``.hipbin`` program files and the on-disk program cache (CPU only: no launches)."""

import json
import os

import pytest

from hip_compiler import compile_subgraph
from hip_compiler.program_io import (cache_key, compile_cached, load_program, program_from_dict, program_to_dict,
                                     save_program)
from irgen.qwen import QwenConfig, build_decode_ir

MINI = QwenConfig(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)


def graphs():
    from irgen.resnet import build_resnet50_ir

    return {"decode": build_decode_ir(256, MINI, argmax=True),
            "prefill": build_decode_ir(64, MINI, argmax=True, tokens=64),
            "resnet": build_resnet50_ir(2, 64)}


@pytest.mark.parametrize("name", ["decode", "prefill", "resnet"])
def test_hipbin_round_trip_is_exact(name, tmp_path):
    prog = compile_subgraph(graphs()[name])
    path = str(tmp_path / f"{name}.hipbin")
    save_program(prog, path)
    back = load_program(path)
    assert back == prog
    assert back.steps[0].grid == prog.steps[0].grid and isinstance(back.steps[0].grid, tuple)


def test_hipbin_rejects_other_formats_and_unknown_records(tmp_path):
    prog = compile_subgraph(graphs()["decode"])
    d = program_to_dict(prog)
    with pytest.raises(ValueError):
        program_from_dict({**d, "version": 2})
    with pytest.raises(ValueError):
        program_from_dict({**d, "format": "npubin"})
    bad = json.loads(json.dumps(d))
    bad["program"]["steps"][0]["__t"] = "Popen"
    with pytest.raises(ValueError):
        program_from_dict(bad)


def test_program_cache_hits_and_keys(tmp_path):
    ir = graphs()["decode"]
    a = compile_cached(ir, str(tmp_path))
    files = os.listdir(tmp_path)
    assert len(files) == 1 and files[0].endswith(".hipbin")
    b = compile_cached(ir, str(tmp_path))
    assert a == b == compile_subgraph(ir)
    assert os.listdir(tmp_path) == files
    # other options or another graph get their own entry
    c = compile_cached(ir, str(tmp_path), fold_attention=False)
    assert c != a and len(os.listdir(tmp_path)) == 2
    assert cache_key(ir, {}) != cache_key(build_decode_ir(128, MINI, argmax=True), {})
    # a damaged entry is rebuilt, not trusted
    path = os.path.join(tmp_path, files[0])
    with open(path, "w") as f:
        f.write("{\"format\": \"hipbin\", \"version\": 1, \"program\": {}}")
    assert compile_cached(ir, str(tmp_path)) == a
    assert load_program(path) == a


def test_program_cache_serves_dag_executor_as_compile_fn(tmp_path):
    """``compile_cached`` has the ``compile_fn`` signature: DAGExecutor compiles each device
    partition through it (a stand-in backend records the programs; nothing launches)."""
    from hip_compiler import is_hip_op_supported
    from npu_compiler import partition
    from npu_runtime.dag_executor import DAGExecutor, _build_sub_ir_dict

    ir = graphs()["decode"]
    plan = partition(ir, is_hip_op_supported)

    class _Recorder:
        def __init__(self):
            self.programs = []

        def create_executor(self, program):
            self.programs.append(program)

    rec = _Recorder()
    DAGExecutor(plan, rec, compile_fn=lambda sub: compile_cached(sub, str(tmp_path)))
    assert len(rec.programs) == 1 and len(os.listdir(tmp_path)) == 1
    assert rec.programs[0] == compile_subgraph(_build_sub_ir_dict(plan.steps[0], ir))


def test_cache_key_covers_lowering_switches(monkeypatch):
    """Environment and module switches that change the lowering change the key, so a cached
    program built under other settings is never returned."""
    from hip_compiler import patterns, subgraph_analyzer

    ir = graphs()["decode"]
    base = cache_key(ir, {})
    monkeypatch.setenv("HIPRT_FOLD_ATTN", "0")
    assert cache_key(ir, {}) != base
    assert cache_key(ir, {"fold_attention": True}) == cache_key(ir, {"fold_attention": True}) != base
    monkeypatch.delenv("HIPRT_FOLD_ATTN")
    monkeypatch.setenv("HIPRT_CONV_NHWC", "0")
    assert cache_key(ir, {}) != base
    monkeypatch.delenv("HIPRT_CONV_NHWC")
    monkeypatch.setattr(patterns, "FUSE_REDUCE_NORM", False)
    assert cache_key(ir, {}) != base
    monkeypatch.setattr(patterns, "FUSE_REDUCE_NORM", True)
    d2 = subgraph_analyzer.CONV_D2_MAX_K
    monkeypatch.setattr(subgraph_analyzer, "CONV_D2_MAX_K", 256)
    assert cache_key(ir, {}) != base
    monkeypatch.setattr(subgraph_analyzer, "CONV_D2_MAX_K", d2)
    assert cache_key(ir, {}) == base
    monkeypatch.setattr(subgraph_analyzer, "CONV_NFAST", not subgraph_analyzer.CONV_NFAST)
    assert cache_key(ir, {}) != base
