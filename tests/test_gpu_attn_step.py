"""The one-launch attention block (k_attn_step, csrc/kernels/decode.hip) against the CPU fallback
(ATen) and against the three-launch list it replaces (q/k/v + RoPE + cache rows, split
attention, combine + o_proj), on the GPU.

Tolerances as for the persistent decode step: outputs and the K/V rows written within 2e-2 of
the largest magnitude, the cache rows the block does not write bit-exact.
Relaunching the block on the same inputs (the step tag advances) reproduces its outputs
bit for bit.
"""

import numpy as np
import pytest

from conftest import gpu_available
from test_gpu_persistent import _close, _cpu, _host

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

MINI = dict(hidden=512, intermediate=1024, heads=4, kv_heads=2, head_dim=128, vocab=4096)

# name: (config, cache length, position, input RMSNorm + residual)
CASES = {
    # cfg2 itself: 9 slots of one chunk, the last chunk holding one position
    "cfg2_s1025": (dict(), 1025, 1024, False),
    # a decoder layer's first half at the decode bench's shape: chunks past the position closed
    "layer_s2048_pos1984": (dict(), 2048, 1984, True),
    # position 0: one open chunk, 15 slots publish empty partials
    "s2048_pos0": (dict(), 2048, 0, False),
    # a cache that is not a multiple of 128 positions
    "s1000_last": (dict(), 1000, 999, True),
    # the reference's benchmark cache length: 16 slots over 256 chunks, 17 of them open
    "s32768_pos2048": (dict(), 32768, 2048, False),
    # hidden 512 (the KC = 1 instance), 4 query heads over 2 KV heads
    "mini_s256_last": (MINI, 256, 255, True),
}


def _inputs(S, pos, cfg):
    from irgen.workloads import attention_inputs, decode_mask

    x = attention_inputs(S, cfg=cfg)
    x["attention_mask"] = decode_mask(S, pos)
    x["position_ids"][:] = pos
    x["cache_position"][:] = pos
    return _host(x)


def _run(ir, backend, w, x, persistent, times=1):
    from hip_compiler import compile_subgraph, is_hip_op_supported
    from npu_compiler import partition
    from npu_runtime import DAGExecutor

    ex = DAGExecutor(partition(ir, is_hip_op_supported), backend,
                     compile_fn=lambda sub: compile_subgraph(sub, persistent=persistent))
    (prog,) = ex.npu_programs.values()
    kernels = [s.kernel for s in prog.steps]
    if persistent:
        assert len(kernels) == 1 and kernels[0].startswith("k_attn_step_k"), kernels
    else:
        assert len(kernels) > 1
    ex.load_weights(w)
    outs = []
    for _ in range(times):
        o = ex.execute({k: v.copy() for k, v in x.items()})
        outs.append({k: (v if isinstance(v, np.ndarray) else v.to_numpy()).copy() for k, v in o.items()})
    (h,) = ex._npu_executors.values()
    h.check()   # no workgroup timed out
    return outs


@pytest.mark.parametrize("case", sorted(CASES))
def test_attention_step_vs_cpu_fallback_and_launch_list(backend, case):
    from irgen.qwen import QwenConfig, build_attention_ir
    from irgen.workloads import make_weights

    kw, S, pos, resid = CASES[case]
    cfg = QwenConfig(**kw)
    ir = build_attention_ir(S, cfg, residual=resid)
    w = _host(make_weights(ir, cfg, device="cuda"))
    x = _inputs(S, pos, cfg)
    print(f"[case] attention step {case}", flush=True)
    runs = _run(ir, backend, w, x, True, times=3)
    (multi,) = _run(ir, backend, w, x, False)
    ref = _cpu(ir, x, w)
    got = runs[0]
    for r in runs[1:]:   # relaunched (new step tag): the same bits
        for k in got:
            assert np.array_equal(r[k], got[k]), k
    out = ir["graph_outputs"][0]["name"]
    _close(got[out], ref[out])
    _close(got[out], multi[out])
    for o, src in zip(ir["graph_outputs"][1:], ("past_key_0", "past_value_0")):
        g, r = np.asarray(got[o["name"]]), np.asarray(ref[o["name"]])
        keep = np.ones(g.shape[2], bool)
        keep[pos] = False
        assert np.array_equal(g[:, :, keep], x[src][:, :, keep])   # untouched rows: bit-exact
        _close(g[:, :, pos], r[:, :, pos])                         # the row written at `pos`
