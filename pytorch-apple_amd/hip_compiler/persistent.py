"""Persistent decode step: a decoder step's launch list replaced by one launch.

The fused lowering of a Qwen2-style decode step (one token, static KV caches) is a fixed
sequence of launches: ``k_embedding``, then per layer ``k_qkv_rope*`` (RMSNorm, q/k/v, RoPE,
K/V cache rows), ``k_attn_flash*`` (split-S attention), ``k_gemv_attn*_resid_r2`` (combine,
o_proj, residual), ``k_gemv_norm_silu_r1`` (RMSNorm, gate/up, SiLU * up) and
``k_gemv_resid_ks_r2`` / ``k_gemv_resid_r1`` (down_proj, residual), then ``k_gemv_norm_argmax_r4`` (final RMSNorm,
lm_head, argmax keys) and ``k_argmax_finalize``. When the launch list is exactly that, with
every layer reading what the previous launch wrote and dimensions the persistent kernel
covers, ``fuse_decode_step`` replaces it with one launch of ``k_decode_step_k<KC>_i<IC>_e<EM>``
(``csrc/kernels/decode.hip``), which runs every layer with one workgroup per CU and hands
activations between the parts of a layer through tagged exchange words instead of launch
boundaries. Anything else keeps the launch list unchanged.

The launch reads the layers' tensors from a pointer table (``params["table"]``): 14 entries
per layer (``TABLE_FIELDS``), resolved by the executor for each set of bound buffers.

The reference runs this step as one Python dispatch per IR op
(`cuda_runtime/cuda_executor.py:136-176`); here the same IR ops become one launch.
"""

from __future__ import annotations

import os

from hip_compiler.program import DTYPE_CODE, LaunchStep, Ref, Storage

NWG = 256            # workgroups of the launch: one per CU of an MI355X (all resident together)
THREADS = 512
D = 128
SPL = 128            # positions per attention split
MAX_G = 8            # query heads per KV head
MAX_SPLITS = 32
VARIANTS = {1, 2, 3}     # hidden / 512 with a kernel instance (inter <= 4096 * that)
E_LDS_ROWS = {1: 48, 2: 32, 3: 24}   # gate/up rows an attention workgroup holds in LDS (decode.hip DEC_NE)
RING_ROWS = {1: (1, 2), 2: (4,), 3: (2, 3, 4, 6)}
O_RING_MAX = 11     # gate/up rows an o_proj workgroup streams, at most (decode.hip DEC_RBO)   # instances: gate/up rows per wave streamed through registers

TABLE_FIELDS = ("norm1", "wq", "bq", "wk", "bk", "wv", "bv", "kc", "vc", "wo", "norm2", "wg", "wu", "wd")

QKV = ("k_qkv_rope_k1536", "k_qkv_rope")
FLASH = ("k_attn_flash_w8", "k_attn_flash", "k_attn_flash_w16")
OPROJ = ("k_gemv_attn16_resid_r2", "k_gemv_attn_resid_r2")
DOWN = ("k_gemv_resid_ks_r2", "k_gemv_resid_r1")


def enabled() -> bool:
    return os.environ.get("HIPRT_PERSISTENT", "1") == "1"


def exchange_words(L: int, hidden: int, inter: int, H: int, KVH: int, nsplit: int) -> int:
    """32-bit words of the exchange area (decode.hip ``xlayout``): per layer the input row, each
    query head's q row with its KV head's k and v rows, the attention partials (o[D] plus m and l as four half-words per split and
    head), the combined attention row, the o_proj output and the SiLU * up row; then the final
    row, one 64-bit argmax key per workgroup and two control words (step tag, timeout flag)."""
    stride = hidden + H * 3 * D + H * nsplit * (D + 4) + H * D + hidden + inter
    stride += stride & 1
    return stride * L + hidden + 2 * NWG + 2


def _same(a, b) -> bool:
    return isinstance(a, Ref) and isinstance(b, Ref) and a == b


def fuse_decode_step(steps: list[LaunchStep], storages: dict[str, Storage]) -> list[LaunchStep] | None:
    """The one-launch form of ``steps``, or None when they are not a decode step it covers."""
    n = len(steps)
    if n < 8 or (n - 3) % 5 != 0:
        return None
    L = (n - 3) // 5
    emb, lm, fin = steps[0], steps[-2], steps[-1]
    if emb.kernel != "k_embedding" or lm.kernel != "k_gemv_norm_argmax_r4" or fin.kernel != "k_argmax_finalize":
        return None
    layers = [steps[1 + 5 * i: 6 + 5 * i] for i in range(L)]
    for q, f, o, g, d in layers:
        if (q.kernel not in QKV or f.kernel not in FLASH or o.kernel not in OPROJ or
                g.kernel != "k_gemv_norm_silu_r1" or d.kernel not in DOWN):
            return None
    ea, la, fa = emb.args, lm.args, fin.args
    q0, f0, g0 = layers[0][0].args, layers[0][1].args, layers[0][3].args
    hidden, H, KVH = int(q0["K"]), int(q0["H"]), int(q0["KVH"])
    inter, vocab, S = int(g0["N"]), int(la["N"]), int(f0["S"])
    if int(ea["n_ids"]) != 1 or int(ea["row_bytes"]) != 2 * hidden or int(ea["vocab"]) != vocab:
        return None
    if int(q0["D"]) != D or H * D != hidden or hidden % 512 or hidden // 512 not in VARIANTS:
        return None
    KC = hidden // 512
    if H % KVH or H // KVH > MAX_G or inter % 8 or inter > 4096 * KC or (H + 2 * KVH) * D > 8 * NWG:
        return None
    # attention runs one workgroup per (query head, split), the combine one per query head
    if S % SPL or S // SPL > MAX_SPLITS or H * (S // SPL) + H > NWG or vocab >= 2 ** 32:
        return None
    nsplit = S // SPL
    # the work split of decode.hip: NB attention workgroups (each also holds NE gate/up rows in
    # LDS), ND o_proj workgroups of RD rows (those that run no combine also hold NEO gate/up rows
    # in LDS); an o_proj workgroup streams RBO gate/up rows, an attention workgroup RBA
    NB, NE = H * nsplit, E_LDS_ROWS[KC]
    ND = NWG - NB
    RD = -(-hidden // ND)
    NEO = max(2 * NE - RD, 0) // 2
    ring = max(inter - NB * NE - (ND - H) * NEO, 0)
    RBO = min(-(-ring // NWG), O_RING_MAX)
    RBA = -(-max(ring - ND * RBO, 0) // NB)
    RB = max(RBA, RBO)
    em = [e for e in RING_ROWS[KC] if 8 * e >= RB]
    if RD > 2 * NE or not em or NE + RB > 128:   # decode.hip DEC_OSTAGE: a workgroup's rows, staged
        return None
    if nsplit * (D + 4) * 2 > 8192 * KC:   # the combine stages a head's partials in LDS
        return None
    shared = ("pos_ids", "cache_pos", "inv_freq")
    x = ea["out"]
    table: list = []
    for q, f, o, g, d in layers:
        qa, fl, oa, ga, da = q.args, f.args, o.args, g.args, d.args
        ok = (
            _same(qa["x"], x) and _same(fl["q"], qa["q_out"]) and _same(fl["k"], qa["k_dst"])
            and _same(fl["v"], qa["v_dst"]) and _same(oa["resid"], x) and _same(oa["attn_o"], fl["part_o"])
            and _same(ga["x"], oa["out"]) and _same(da["x"], ga["out"]) and _same(da["resid"], oa["out"])
            and all(_same(qa[k], q0[k]) for k in shared)
            and (int(qa["flags"]) | 2) == 63 and int(qa["flags"]) & 2 == int(q0["flags"]) & 2
            and int(qa["K"]) == hidden and int(qa["H"]) == H and int(qa["KVH"]) == KVH and int(qa["D"]) == D
            and int(qa["cache_len"]) == S and int(qa["kv_head_stride"]) == int(fl["kv_head_stride"])
            and int(qa["kv_head_stride"]) == int(q0["kv_head_stride"]) and float(qa["rope_scaling"]) == float(q0["rope_scaling"])
            and int(fl["S"]) == S and int(fl["H"]) == H and int(fl["KVH"]) == KVH and int(fl["dtype"]) == DTYPE_CODE["bfloat16"]
            and int(fl["q_head_stride"]) == D and float(fl["scale"]) == float(f0["scale"])
            and (fl["mask"] is None or (_same(fl["mask"], f0["mask"]) and int(fl["mask_stride"]) == 1
                                        and int(fl["mask_dtype"]) in (0, 2)))
            and int(fl.get("add_dtype", 2)) == int(f0.get("add_dtype", 2))
            and int(oa["N"]) == hidden and int(oa["K"]) == hidden and int(oa["M"]) == 1 and int(oa["flags"]) == 0
            and int(ga["N"]) == inter and int(ga["K"]) == hidden and int(ga["M"]) == 1 and int(ga["flags"]) == 0
            and ga["bias"] is None and ga["bias2"] is None and float(ga["eps"]) == float(qa["eps"])
            and int(ga["n_dtype"]) == int(qa["n_dtype"]) == int(q0["n_dtype"])
            and int(da["N"]) == hidden and int(da["K"]) == inter and int(da["M"]) == 1 and int(da["flags"]) == 0
            and float(qa["eps"]) == float(q0["eps"])
        )
        if not ok:
            return None
        bias = int(qa["flags"]) & 2
        table += [qa["norm_w"], qa["wq"], qa["bq"] if bias else None, qa["wk"], qa["bk"] if bias else None,
                  qa["wv"], qa["bv"] if bias else None, qa["k_dst"], qa["v_dst"], oa["w"], ga["norm_w"], ga["w"],
                  ga["w2"], da["w"]]
        x = da["out"]
    if not (_same(la["x"], x) and _same(fa["slot"], la["argmax_slot"]) and int(la["K"]) == hidden
            and int(la["M"]) == 1 and int(la["flags"]) == 0 and int(fa["rows"]) == 1
            and int(fa["out_dtype"]) in (DTYPE_CODE["int64"], DTYPE_CODE["int32"])
            and int(la["n_dtype"]) == int(q0["n_dtype"])):
        return None
    words = exchange_words(L, hidden, inter, H, KVH, nsplit)
    xname = "decode_step.exchange"
    storages[xname] = Storage(xname, "persistent", words * 4, "uint8", zero_init=True)
    mask = f0["mask"]
    args = dict(
        layers=None, emb=ea["w"], ids=ea["ids"], pos_ids=q0["pos_ids"], cache_pos=q0["cache_pos"], mask=mask,
        inv_freq=q0["inv_freq"], norm_f=la["norm_w"], lm_w=la["w"], logits=la["out"], next_token=fa["out"],
        ll=Ref(xname, 0), trace=None, S=S, kv_head_stride=int(q0["kv_head_stride"]), vocab=vocab, L=L, hidden=hidden,
        inter=inter, H=H, KVH=KVH, D=D, nsplit=nsplit, nwg=NWG, ids_dtype=int(ea["ids_dtype"]),
        pos_dtype=int(q0["pos_dtype"]), cpos_dtype=int(q0["cpos_dtype"]),
        mask_dtype=int(f0["mask_dtype"]) if mask is not None else -1, add_dtype=int(f0.get("add_dtype", 2)),
        n_dtype=int(q0["n_dtype"]), out_dtype=int(fa["out_dtype"]), flags=1 if int(q0["flags"]) & 2 else 0,
        eps=float(q0["eps"]), eps_f=float(la["eps"]), scale=float(f0["scale"]),
        rope_scaling=float(q0["rope_scaling"]))
    inputs = sorted({t for st in steps for t in st.inputs})
    outputs = [t for st in steps for t in st.outputs]
    step = LaunchStep(
        kind="decode_step", kernel=f"k_decode_step_k{KC}_i{KC}_e{em[0]}", module="decode", arg_struct="PersistArgs",
        args=args, grid=(NWG, 1, 1), block=(THREADS, 1, 1), inputs=inputs, outputs=outputs,
        params={"table": {"field": "layers", "entries": table}, "layers": L, "nsplit": nsplit,
                "replaces": [st.kernel for st in steps], "exchange_words": words})
    return [step]
