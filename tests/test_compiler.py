"""Structure of compiled HIP programs (no GPU): step lists, fusion decisions, views, arena,
codegen and the op support table. Counterpart of the reference's CPU-only compiler tests
(tests/test_cuda_compiler.py:53-530)."""

import numpy as np
import pytest

from hip_compiler import compile_subgraph, get_hip_supported_ops, is_hip_op_supported
from hip_compiler import persistent
from hip_compiler import views as V
from hip_compiler.program import ELEM_SIZE, Ref, TView, contiguous_strides
from irgen.qwen import QwenConfig, build_attention_ir, build_decode_ir, build_mlp_ir
from npu_compiler import partition


def kernels(p):
    return [s.kernel for s in p.steps]


def test_mlp_block_fused_and_generic_step_lists():
    fused = compile_subgraph(build_mlp_ir(1))
    assert kernels(fused) == ["k_gemv_norm_silu_r1", "k_gemv_resid_ks_r2"]
    gen = compile_subgraph(build_mlp_ir(1), fuse=False)
    kinds = [s.kind for s in gen.steps]
    # the reference's expected list: [RMSNorm, gemm gate, gemm up, fused(silu, mul), gemm down, fused(add)]
    assert kinds.count("gemv") == 3 and kinds.count("fused") >= 2
    # 2 .. 15 rows: the same list with the skinny MFMA kernels for the linears
    gen4 = compile_subgraph(build_mlp_ir(4), fuse=False)
    assert [s.kernel for s in gen4.steps if s.kind == "gemm"] == ["k_skinny_bias_mt1"] * 2 + ["k_skinny_bias_mt1_r8"]
    assert "rmsnorm" not in kinds  # generic lowering: the norm becomes a chain + mean reduction
    chains = [s.params["ops"] for s in gen.steps if s.kind == "fused"]
    assert ["aten.silu.default", "aten.mul.Tensor"] in chains
    assert ["aten.add.Tensor"] in chains
    # prefill-shaped rows: the linears go to the MFMA GEMM (gate, up, down), fused or not
    gen16 = compile_subgraph(build_mlp_ir(16), fuse=False)
    assert sum(1 for s in gen16.steps if s.kind == "gemm" and not s.params.get("reduce")) == 3


def test_mlp_33_to_128_rows_take_the_wide_silu_kernel():
    # 33-128 rows: the norm's launch, the wide SiLU kernel (4 waves, 5 tiles of 8 pairs per
    # workgroup: 224 tile groups for 8960 pairs; past 64 rows two workgroups of 64 rows per
    # group, 448 in all), then the down GEMM; 129 rows: the GEMM
    from hip_compiler.subgraph_analyzer import WIDE_HALVES, WIDE_TA
    assert -(-8960 // (8 * WIDE_TA)) == 224
    for T, kn, g in ((33, "mt4", 224), (64, "mt4", 224), (65, "mt4x2" if WIDE_HALVES else "mt8", 448 if WIDE_HALVES else 224),
                     (128, "mt4x2" if WIDE_HALVES else "mt8", 448 if WIDE_HALVES else 224)):
        p = compile_subgraph(build_mlp_ir(T))
        ks = kernels(p)
        assert ks[0] == "k_rmsnorm_w" and ks[1] == f"k_wide_silu_{kn}", (T, ks)
        st = p.steps[1]
        assert st.grid == (g, 1, 1) and st.block == (256, 1, 1)
        assert st.args["M"] == T and st.args["K"] == 1536 and st.args["w2"] is not None
    assert not any(k.startswith("k_wide") for k in kernels(compile_subgraph(build_mlp_ir(129))))


def test_prefill_mlp_is_norm_plus_two_mfma_gemms():
    p = compile_subgraph(build_mlp_ir(512))
    main = [s for s in p.steps if s.kind == "gemm" and not s.params.get("reduce")]
    assert kernels(p)[0] == "k_rmsnorm_w" and abs(p.steps[0].args["eps"] - 1e-6) < 1e-12   # wave per row
    assert [s.params["epilogue"] for s in main] == ["silu", "resid"]
    assert main[0].params["weights"] == 2 and main[0].args["w2"] is not None
    # K % 64 == 0 and a tile grid below 1024: operands staged straight into LDS (the _k64d kernels)
    assert all(s.params["lds_direct"] and s.kernel.endswith("_k64d") for s in main)
    from irgen.qwen import QwenConfig
    odd = [s for s in compile_subgraph(build_mlp_ir(512, QwenConfig(hidden=96, intermediate=160))).steps
           if s.kind == "gemm" and not s.params.get("reduce")]
    assert odd and not any(s.params["lds_direct"] for s in odd)   # K = 96 or 160: not a multiple of 64
    for s in main:   # every workgroup covers a whole K range; splits tile K exactly
        g = s.grid
        assert g[2] == s.args["ksplit"] and s.args["kchunk"] % 32 == 0
        assert (g[2] - 1) * s.args["kchunk"] < s.args["K"] <= g[2] * s.args["kchunk"]
        bm, bn = s.params["tile"]
        assert g[0] * bn >= s.args["N"] and g[1] * bm >= s.args["M"]
    # split-K launches are followed by their reduction, which applies the epilogue
    for i, s in enumerate(p.steps):
        if s.kind == "gemm" and s.args["ksplit"] > 1 and not s.params.get("reduce"):
            assert p.steps[i + 1].kernel.startswith("k_gemm_reduce_")
            assert p.steps[i + 1].args["part"] == s.args["part"]


def test_rmsnorm_pattern_alone_is_one_kernel():
    # the RMSNorm folded into the first projection: the GEMV prologue (1 row) or the skinny SiLU
    # kernel (2-16 rows); no launch of its own either way
    for T in (1, 4, 16):
        p = compile_subgraph(build_mlp_ir(T))
        first = p.steps[0]
        assert first.params.get("norm") is True and "rmsnorm" not in [s.kind for s in p.steps], T
        assert abs(first.args["eps"] - 1e-6) < 1e-12


def test_attention_block_is_one_launch_by_default():
    # the one-launch block: 9 slots of one 128-position chunk each for 12 heads (108 attention
    # workgroups); 12 of the other 148 combine a head's partials, and 140 take 11 o_proj rows each
    p = compile_subgraph(build_attention_ir(1025))
    assert kernels(p) == ["k_attn_step_k3"]
    st = p.steps[0]
    assert st.kind == "attn_step" and st.grid == (256, 1, 1) and st.block == (512, 1, 1)
    assert st.params["nsplit"] == 9 and st.args["nchunk"] == 9 and st.args["rows"] == 11 and st.args["resid"] is None
    assert st.params["replaces"] == ["k_qkv_rope_k1536", "k_attn_flash_w8", "k_gemv_attn16_bias_r2"]
    assert st.params["exchange_words"] == 12 * 3 * 128 + 12 * 9 * 132 + 12 * 128 + 2
    assert set(p.stats["mutated_inputs"]) == {"past_key_0", "past_value_0"}
    assert p.output_views["index_copy"].storage == "past_key_0"
    # long caches: 16 slots walking up to 32 chunks each; the separate-combine list is fused too
    long = compile_subgraph(build_attention_ir(40000))
    assert kernels(long) == ["k_attn_step_k3"] and long.steps[0].params["nsplit"] == 16
    assert long.steps[0].params["replaces"][2:] == ["k_attn_combine", "k_gemv_bias_r1"]
    # past 16 x 32 chunks, or off the kernel's shapes (hidden 2048), the launch list stays
    assert len(compile_subgraph(build_attention_ir(65537)).steps) > 1
    assert len(compile_subgraph(build_attention_ir(700, QwenConfig(hidden=2048, heads=16, kv_heads=2))).steps) == 3


def test_attention_slots_leave_room_for_the_combine_and_o_proj():
    for S in (1, 128, 129, 1025, 2048, 4096, 65536):
        n = persistent.attention_slots(S, 1536, 12)
        nchunk = -(-S // 128)
        assert n == min(nchunk, 16) and -(-nchunk // n) <= 32
        nd = 256 - 12 * n
        assert nd > 12 and -(-1536 // nd) <= persistent.AST_ROWS
    assert persistent.attention_slots(65537, 1536, 12) is None
    # 20 heads, hidden 2560: 12 slots leave 16 workgroups (fewer than the 20 combines), 9 leave 76
    # (34 o_proj rows each, more than 32); 8 leave 96 (27 rows)
    assert persistent.attention_slots(4096, 2560, 20) == 8


def test_attention_block_is_three_launches_with_inplace_cache():
    # the launch list: 128-position splits (8 waves), combined in the o_proj prologue
    p = compile_subgraph(build_attention_ir(1025), persistent=False)
    assert kernels(p) == ["k_qkv_rope_k1536", "k_attn_flash_w8", "k_gemv_attn16_bias_r2"]
    flash = p.steps[1]
    assert flash.args["nsplit"] == 9 and flash.block == (512, 1, 1) and flash.grid == (9, 2, 6)
    assert p.steps[2].args["attn_splits"] == 9 and p.steps[2].args["attn_heads"] == 12
    # up to 8 splits: the 8-split prologue
    short = compile_subgraph(build_attention_ir(256), persistent=False)
    assert kernels(short) == ["k_qkv_rope_k1536", "k_attn_flash_w8", "k_gemv_attn_bias_r2"]
    # 2048 < S <= 4096: 256-position splits (16 waves), at most 16 of them
    mid = compile_subgraph(build_attention_ir(4096), persistent=False)
    assert kernels(mid) == ["k_qkv_rope_k1536", "k_attn_flash_w16", "k_gemv_attn16_bias_r2"]
    assert mid.steps[1].args["nsplit"] == 16 and mid.steps[1].block == (1024, 1, 1)
    # separate combine kernel: 64-position splits
    sep = compile_subgraph(build_attention_ir(1025), fold_attention=False, persistent=False)
    assert kernels(sep) == ["k_qkv_rope_k1536", "k_attn_flash", "k_attn_combine", "k_gemv_bias_r1"]
    assert sep.steps[1].args["nsplit"] == 17
    # more than 16 splits of 256 do not fit the prologue: the separate combine is kept, and
    # beyond 32 splits each split checks its mask before reading K / V
    long = compile_subgraph(build_attention_ir(4097), persistent=False)
    assert kernels(long) == ["k_qkv_rope_k1536", "k_attn_flash_chk", "k_attn_combine", "k_gemv_bias_r1"]
    assert set(p.stats["mutated_inputs"]) == {"past_key_0", "past_value_0"}
    assert p.output_views["index_copy"].storage == "past_key_0"
    exact = compile_subgraph(build_attention_ir(1025), exact_attention=True)
    assert kernels(exact) == ["k_qkv_rope_k1536", "k_attn_scores", "k_attn_out", "k_gemv_bias_r1"]
    gen = compile_subgraph(build_attention_ir(1025), fuse=False)
    assert "k_index_copy" in kernels(gen) and "k_bmm" in kernels(gen)


def test_decode_step_launch_count_and_cache_aliasing():
    cfg = QwenConfig(layers=3)
    p = compile_subgraph(build_decode_ir(256, cfg, argmax=True), persistent=False)
    assert len(p.steps) == 1 + 5 * cfg.layers + 2      # embedding, 5 per layer, lm_head+argmax, finalize
    assert kernels(p)[0] == "k_embedding" and kernels(p)[-2:] == ["k_gemv_norm_argmax_r4", "k_argmax_finalize"]
    assert len(p.stats["mutated_inputs"]) == 2 * cfg.layers
    assert not any(s.kernel in ("k_rope_table", "k_rmsnorm", "k_rmsnorm_w", "k_copy") for s in p.steps)


def test_not_inplace_when_cache_input_has_another_reader():
    ir = build_attention_ir(64)
    # make the K cache also a graph output read directly: in-place update is no longer allowed
    ir["graph_outputs"].append({"name": "past_key_0", "shape": [1, 2, 64, 128], "dtype": "bfloat16"})
    p = compile_subgraph(ir)
    assert "past_key_0" not in p.stats["mutated_inputs"]


def test_every_decode_op_is_supported_and_partitions_to_one_device_partition():
    ir = build_decode_ir(128, QwenConfig(layers=2), argmax=True)
    assert all(is_hip_op_supported(n["op_type"], n.get("attrs")) for n in ir["nodes"])
    plan = partition(ir, is_hip_op_supported)
    assert len(plan.steps) == 1 and plan.steps[0].target == "npu"
    assert is_hip_op_supported("aten.conv2d.default", {"groups": 1, "dilation": [1, 1]})
    assert not is_hip_op_supported("aten.conv2d.default", {"groups": 32})       # grouped conv -> CPU
    assert not is_hip_op_supported("aten.batch_norm.default", {"training": True})
    assert not is_hip_op_supported("aten.adaptive_avg_pool2d.default", {"output_size": [7, 7]})
    assert not is_hip_op_supported("aten.dropout.default", {"p": 0.1, "train": True})
    assert "aten.index_copy.default" in get_hip_supported_ops()


def _intervals(p):
    out = []
    for s in p.storages.values():
        if s.kind in ("arena", "persistent") and s.first >= 0:
            size = (s.nbytes + 255) // 256 * 256
            out.append((s.first, s.last, s.offset, s.offset + size, s.kind))
    return out


@pytest.mark.parametrize("build", [lambda: build_decode_ir(256, QwenConfig(layers=2), argmax=True),
                                   lambda: build_mlp_ir(16), lambda: build_attention_ir(300)])
@pytest.mark.parametrize("fuse", [True, False])
def test_arena_live_ranges_never_share_bytes(build, fuse):
    p = compile_subgraph(build(), fuse=fuse)
    iv = _intervals(p)
    for i, a in enumerate(iv):
        assert a[3] <= p.arena_bytes
        for b in iv[i + 1:]:
            live_overlap = not (a[1] < b[0] or b[1] < a[0]) or "persistent" in (a[4], b[4])
            if live_overlap:
                assert a[3] <= b[2] or b[3] <= a[2]


@pytest.mark.parametrize("fuse", [True, False])
def test_steps_read_only_already_written_arena_storage(fuse):
    p = compile_subgraph(build_decode_ir(128, QwenConfig(layers=2), argmax=True), fuse=fuse, persistent=False)
    out_fields = {"dst", "out", "c", "cos_out", "sin_out", "q_out", "k_dst", "v_dst", "part_o", "part_ml",
                  "scores", "stats", "argmax_slot", "part", "slot"}
    written = set()
    for s in p.steps:
        outs = {v.storage for k, v in s.args.items() if k in out_fields and isinstance(v, Ref)}
        for k, v in s.args.items():
            refs = [v] if isinstance(v, Ref) else [x for x in v if isinstance(x, Ref)] if isinstance(v, (list, tuple)) \
                else []
            for r in refs:
                if k in out_fields or p.storages[r.storage].kind != "arena":
                    continue
                assert r.storage in written or r.storage in outs, (s.kernel, k, r)
        written |= outs


def test_view_arithmetic():
    v = TView("s", 0, (1, 12, 1, 128), contiguous_strides((1, 12, 1, 128)), "bfloat16")
    t = V.transpose(v, 1, 2)
    assert t.shape == (1, 1, 12, 128)
    r = V.restride(t, (1, 1, 1536))
    assert r is not None and r.is_contiguous()
    m = TView("m", 0, (4, 6), contiguous_strides((4, 6)), "float32")
    assert V.restride(V.transpose(m, 0, 1), (24,)) is None        # needs a copy
    e = V.expand(TView("c", 0, (1, 1, 1, 128), (128, 128, 128, 1), "bfloat16"), (1, 12, 1, 128))
    assert e.strides[1] == 0
    s = V.slice_(m, 1, 2, 5)
    assert s.offset == 2 and s.shape == (4, 3) and s.strides == (6, 1)
    assert V.slice_(m, 1, 3, 9223372036854775807).shape == (4, 3)


def test_generated_chain_reads_broadcast_operands_with_zero_stride():
    from hip_compiler.codegen import ChainOp, generate_chain

    out = (1, 12, 1, 128)
    x = TView("x", 0, out, contiguous_strides(out), "bfloat16")
    c = V.broadcast_to(TView("c", 0, (1, 1, 1, 128), contiguous_strides((1, 1, 1, 128)), "bfloat16"), out)
    name, src = generate_chain([ChainOp("aten.mul.Tensor", [("ext", 0), ("ext", 1)], "bfloat16")], [x, c], out,
                               "bfloat16")
    assert "c1 * 128LL" in src                     # x walks heads
    # 8 outputs per thread (last dim 128): 16-byte loads; cos broadcast over heads: only the dim term
    assert "ld8_f(a.in[1], c3 * 1LL, 2" in src and "st8_f(a.out, i * 8, 2" in src
    assert name.startswith("fused_ew_")
    # a last dimension that is not a multiple of 8 keeps one element per thread
    out = (1, 12, 1, 100)
    x = TView("x", 0, out, contiguous_strides(out), "bfloat16")
    c = V.broadcast_to(TView("c", 0, (1, 1, 1, 100), contiguous_strides((1, 1, 1, 100)), "bfloat16"), out)
    _, src = generate_chain([ChainOp("aten.mul.Tensor", [("ext", 0), ("ext", 1)], "bfloat16")], [x, c], out,
                            "bfloat16")
    assert "ld_f(a.in[1], c3 * 1LL, 2)" in src and "st8_f" not in src
    # an operand broadcast along the last dimension is one load per 8 outputs
    out = (4, 64)
    x = TView("x", 0, out, contiguous_strides(out), "float32")
    s_ = V.broadcast_to(TView("s", 0, (4, 1), contiguous_strides((4, 1)), "float32"), out)
    _, src = generate_chain([ChainOp("aten.mul.Tensor", [("ext", 0), ("ext", 1)], "float32")], [x, s_], out,
                            "float32")
    assert "ld1x8_f(a.in[1], c0 * 1LL, 0" in src and "ld8_f(a.in[0]" in src


def test_output_views_are_whole_contiguous_storages():
    p = compile_subgraph(build_decode_ir(128, QwenConfig(layers=2), argmax=True))
    for name, v in p.output_views.items():
        st = p.storages[v.storage]
        assert v.offset == 0 and v.is_contiguous() and v.numel * ELEM_SIZE[v.dtype] == st.nbytes


def test_resnet50_compiles_to_fused_convs():
    from irgen.resnet import build_resnet50_ir

    ir = build_resnet50_ir(32, 224)
    plan = partition(ir, is_hip_op_supported)
    assert len(plan.steps) == 1 and plan.steps[0].target == "npu"
    p = compile_subgraph(ir)
    convs = [s for s in p.steps if s.kind == "conv" and not s.params.get("reduce")]
    reduces = [s for s in p.steps if s.kind == "conv" and s.params.get("reduce")]
    # every BN / add / ReLU folded into a conv (or into the split-K reduce that finishes it); the 16
    # convs with a kernel wider than 1 x 1 read their weights as OHWI, copied by one launch that
    # opens every run
    perm = [s for s in p.steps if s.kernel == "k_permute_ohwi"]
    assert len(convs) == 53 and len(perm) == 1 and perm[0].params["tensors"] == 17 and p.steps[0] is perm[0]
    assert len(p.steps) <= 57 + len(reduces) + 2 and not any(s.kernel == "k_copy" for s in p.steps)
    assert all(s.kernel.startswith("k_gemm_reduce_f16_conv") for s in reduces)
    assert len(reduces) == sum(1 for s in convs if s.params["ksplit"] > 1)
    assert sum(1 for s in convs if s.args["flags"] & 4) == 16 and all(s.args["flags"] & 2 for s in convs)
    # the 3-channel stem reads a zero-bordered 4-channel NHWC copy of the image: 8 x 8 x 4 taps, K = 256
    assert p.steps[1].kernel == "k_pad_nhwc4" and p.steps[1].params["padded"] == [230, 230]
    assert convs[0].kernel.startswith("k_gemm_f16_convp_") and convs[0].args["K"] == 256
    # channels-last from the stem on: all 53 convs are MFMA GEMMs over NHWC (1 x 1 stride 1: the image
    # rows as they are; else tap gathers), pools read NHWC
    assert all(s.params.get("nhwc") for s in convs)
    assert all(s.kernel.startswith(("k_gemm_f16_conv_", "k_gemm_f16_convg_")) for s in convs[1:])
    assert sum(1 for s in convs[1:] if "_convg_" in s.kernel) == 16 + 3   # 3 x 3 and the stride-2 1 x 1
    ks = [s.kernel for s in p.steps]
    assert "k_maxpool2d_nhwc_f16" in ks and "k_mean_nhwc_f16" in ks
    # scheduling: tiles N-fastest (GEMM flag 16) exactly where the input outweighs the weights; short-K
    # convs over >= 1,024 tiles on 64 x 64 tiles; K = 64 1 x 1 convs on the one-stage kernels
    # (_k64d1), K <= 1,024 on two stages
    for s in convs[1:]:
        a = s.args
        x_elems = a["M"] // (a["cHo"] * a["cWo"]) * a["cH"] * a["cW"] * a["cCin"]
        assert bool(a["flags"] & 16) == (x_elems > a["N"] * a["K"]), s.params["nodes"]
        tiles64 = -(-a["M"] // 64) * -(-a["N"] // 64)
        if a["K"] <= 512 and tiles64 >= 1024:
            assert s.params["tile"] == (64, 64), s.params["nodes"]
        plain = "_conv_" in s.kernel
        if plain and a["K"] == 64 and s.params["tile"] == (64, 64):
            assert s.kernel.endswith("_k64d1")
        elif a["K"] <= 1024:
            assert s.kernel.endswith("_k64d2")
    assert sum(1 for s in convs if s.kernel.endswith("_k64d1")) == 5   # the 56 x 56 64-channel 1 x 1 convs
    # HIPRT_CONV_NHWC=0 keeps every conv on the NCHW kernels
    import os
    os.environ["HIPRT_CONV_NHWC"] = "0"
    try:
        q = compile_subgraph(ir)
    finally:
        del os.environ["HIPRT_CONV_NHWC"]
    assert all(s.kernel.startswith("k_conv_") for s in q.steps if s.kind == "conv")


@pytest.mark.parametrize("fuse", [True, False])
def test_graph_outputs_share_no_arena_bytes(fuse):
    """A greedy loop feeds ``next_token`` (an arena output) back as the next run's ``input_ids``;
    no step of a run may write bytes of an output storage other than the output itself, so the
    embedding that reads input_ids first never races with a write into the same bytes."""
    p = compile_subgraph(build_decode_ir(128, QwenConfig(layers=2), argmax=True), fuse=fuse)
    out_storages = {p.output_views[spec.name].storage for spec in p.output_specs if spec.name in p.output_views}
    assert {"next_token"} <= {spec.name for spec in p.output_specs} and out_storages
    placed = [s for s in p.storages.values() if s.kind in ("arena", "persistent") and s.offset >= 0]
    for o in placed:
        if o.name not in out_storages:
            continue
        lo, hi = o.offset, o.offset + (o.nbytes + 255) // 256 * 256
        assert o.first == 0 and o.last >= len(p.steps) - 1
        for s in placed:
            if s is o:
                continue
            s_hi = s.offset + (s.nbytes + 255) // 256 * 256
            assert s_hi <= lo or hi <= s.offset, (o.name, s.name)


def test_decode_step_becomes_one_persistent_launch():
    """The fused decode lowering is replaced by one launch of the persistent kernel, whose pointer
    table holds 14 tensors per layer; the launch list stays available with persistent=False, and
    graphs that are not a decode step (prefill, an unfused lowering) are left alone."""
    from hip_compiler.persistent import TABLE_FIELDS, exchange_words

    cfg = QwenConfig(layers=3)
    ir = build_decode_ir(2048, cfg, argmax=True)
    p = compile_subgraph(ir)
    assert [s.kernel for s in p.steps] == ["k_decode_step_k3_i3_e2"]
    st = p.steps[0]
    assert st.grid == (256, 1, 1) and st.block == (512, 1, 1)
    entries = st.params["table"]["entries"]
    assert len(entries) == len(TABLE_FIELDS) * cfg.layers
    assert entries[TABLE_FIELDS.index("kc")].storage == "past_key_0"
    assert entries[TABLE_FIELDS.index("wd") + 14 * 2].storage == "p_model_layers_2_mlp_down_proj_weight"
    xs = p.storages[st.args["ll"].storage]
    assert xs.kind == "persistent" and xs.nbytes == 4 * exchange_words(3, 1536, 8960, 12, 2, 16)
    assert st.args["logits"].storage == p.output_views[ir["graph_outputs"][0]["name"]].storage
    assert len(compile_subgraph(ir, persistent=False).steps) == 2 + 5 * cfg.layers + 1
    assert len(compile_subgraph(ir, fuse=False).steps) > 20
    pre = compile_subgraph(build_decode_ir(64, QwenConfig(layers=1), argmax=True, tokens=64))
    assert not any(s.kind == "decode_step" for s in pre.steps)


def test_persistent_step_needs_every_workgroup_resident(monkeypatch):
    """A device that holds fewer than the step's 256 workgroups at once keeps the launch list
    (the step's workgroups wait for each other's data)."""
    import hip_compiler.persistent as P
    from hip_compiler import compile_subgraph
    from irgen.qwen import QwenConfig, build_decode_ir

    ir = build_decode_ir(2048, QwenConfig(layers=2), argmax=True)
    monkeypatch.setattr(P, "resident_workgroups", lambda kernel: 128)
    assert len(compile_subgraph(ir).steps) > 1
    monkeypatch.setattr(P, "resident_workgroups", lambda kernel: 256)
    assert [s.kind for s in compile_subgraph(ir).steps] == ["decode_step"]


@pytest.mark.parametrize("S", [128, 1000, 2048, 2176, 4096, 32768, 65536])
def test_persistent_step_covers_long_and_ragged_caches(S):
    """One launch for caches up to 32 chunks per slot; the work split covers every gate/up row
    exactly once (the kernel's e0 / ecnt arithmetic) and fits the kernel's LDS staging."""
    import hip_compiler.persistent as P
    from hip_compiler import compile_subgraph
    from irgen.qwen import QwenConfig, build_decode_ir

    cfg = QwenConfig(layers=1)
    prog = compile_subgraph(build_decode_ir(S, cfg, argmax=True))
    (st,) = prog.steps
    ws, ns = st.params["work_split"], st.params["nsplit"]
    assert st.args["nchunk"] == -(-S // 128) and -(-st.args["nchunk"] // ns) <= 32
    NB, ND, NE, NEO, H = ws["NB"], ws["ND"], ws["NE"], ws["NEO"], cfg.heads
    rows = []
    for b in range(P.NWG):
        att, comb = b < NB, NB <= b < NB + H and not st.params["slot_combine"]
        e0 = (b * (NE + ws["RBA"]) if att else
              NB * (NE + ws["RBA"]) + min(b - NB, H) * ws["RBC"] + max(b - NB - H, 0) * (ws["RBO"] + NEO))
        nlc = NE if att else (0 if comb else NEO)
        ecnt = max(min(nlc + (ws["RBA"] if att else (ws["RBC"] if comb else ws["RBO"])), cfg.intermediate - e0), 0)
        rows += range(e0, e0 + ecnt)
        assert ecnt - min(nlc, ecnt) <= 8 * ws["EM"]
    assert sorted(rows) == list(range(cfg.intermediate))


def test_long_caches_take_the_kv_head_major_attention():
    """From KV_MAJOR_MIN_S positions the step scores the G query heads of a KV head in one workgroup:
    G times the slots (the same attention workgroups), G times the partials in the exchange area."""
    import hip_compiler.persistent as P
    from hip_compiler import compile_subgraph
    from irgen.qwen import QwenConfig, build_decode_ir

    cfg = QwenConfig(layers=1)
    G = cfg.heads // cfg.kv_heads
    steps = {S: compile_subgraph(build_decode_ir(S, cfg, argmax=True)).steps for S in (8192, 32768)}
    (short,), (long_,) = steps[8192], steps[32768]
    assert not short.kernel.endswith("_kv") and long_.kernel.endswith("_kv") and long_.params["kv_major"]
    assert 8192 < P.KV_MAJOR_MIN_S <= 32768
    ns = int(long_.args["nsplit"])
    assert ns == G * P.MAX_SLOTS and cfg.kv_heads * ns == long_.params["work_split"]["NB"]
    assert -(-int(long_.args["nchunk"]) // ns) <= P.MAX_CHUNKS_PER_SLOT
    assert long_.params["exchange_words"] == P.exchange_words(1, cfg.hidden, cfg.intermediate, cfg.heads,
                                                              cfg.kv_heads, ns)


def test_persistent_step_rejects_caches_past_its_chunk_word():
    from hip_compiler import compile_subgraph
    from irgen.qwen import QwenConfig, build_decode_ir

    prog = compile_subgraph(build_decode_ir(65536 + 128, QwenConfig(layers=1), argmax=True))
    assert len(prog.steps) > 1
