"""Persistent decode step: a decoder step's launch list replaced by one launch.

The fused lowering of a Qwen2-style decode step (one token, static KV caches) is a fixed
sequence of launches: ``k_embedding``, then per layer ``k_qkv_rope*`` (RMSNorm, q/k/v, RoPE,
K/V cache rows), ``k_attn_flash*`` (split-S attention), ``k_gemv_attn*_resid_r2`` (combine,
o_proj, residual; for long caches ``k_attn_combine`` then ``k_gemv_resid_r*``),
``k_gemv_norm_silu_r1`` (RMSNorm, gate/up, SiLU * up) and
``k_gemv_resid_ks_r2`` / ``k_gemv_resid_r1`` (down_proj, residual), then ``k_gemv_norm_argmax_r4`` (final RMSNorm,
lm_head, argmax keys) and ``k_argmax_finalize``. When the launch list is exactly that, with
every layer reading what the previous launch wrote and dimensions the persistent kernel
covers, ``fuse_decode_step`` replaces it with one launch of ``k_decode_step_k<KC>_i<IC>_e<EM>``
(``csrc/kernels/decode.hip``), which runs every layer with one workgroup per CU and hands
activations between the parts of a layer through tagged exchange words instead of launch
boundaries. Anything else keeps the launch list unchanged.

The launch reads the layers' tensors from a pointer table (``params["table"]``): 14 entries
per layer (``TABLE_FIELDS``), resolved by the executor for each set of bound buffers.

Attention runs on ``nsplit`` workgroups (slots) per query head, at most ``MAX_SLOTS``; slot j
reads the cache's 128-position chunks j, j + nsplit, ... that the step's mask leaves open, so a
cache of up to 32 * 128 * nsplit positions is one launch and the K/V rows read follow the open
positions, not the cache length.

The step is correct only when all ``NWG`` workgroups are resident at once (they wait for each
other's data). ``fuse_decode_step`` asks ``resident_workgroups`` how many fit on the device and
keeps the launch list when that is fewer; the executor checks again before it launches.

``fuse_attention_step`` does the same for a graph that is one decode-token attention block
(the cfg2 block: q/k/v + RoPE + cache rows, split attention, combine + o_proj, optionally with
the input RMSNorm and a residual): one launch of ``k_attn_step_k<KC>``, the decode step's
attention parts for a single layer.

The reference runs this step as one Python dispatch per IR op
(`cuda_runtime/cuda_executor.py:136-176`, GQA attention at :226-273); here the same IR ops
become one launch.
"""

from __future__ import annotations

import os

from hip_compiler.program import DTYPE_CODE, LaunchStep, Ref, Storage

NWG = 256            # workgroups of the launch: one per CU of an MI355X (all resident together)
THREADS = 512
D = 128
SPL = 128            # positions per attention chunk
MAX_G = 8            # query heads per KV head
MAX_SLOTS = 16       # attention workgroups per query head
MAX_CHUNKS_PER_SLOT = 32   # the kernel's open-chunk word (decode.hip ``ob``)
VARIANTS = {1, 2, 3}     # hidden / 512 with a kernel instance (inter <= 4096 * that)
E_LDS_ROWS = {1: 48, 2: 32, 3: 24}   # gate/up rows an attention workgroup holds in LDS (decode.hip DEC_NE)
RING_ROWS = {1: (1, 2), 2: (4,), 3: (2, 3, 4, 6)}   # kernel instances: gate/up rows per wave in registers
# gate/up rows an o_proj workgroup streams, at most, while the attention workgroups can take the
# rest (Qwen2.5-1.5B at 2048 positions: 11, and 16 per attention workgroup, 0.724 ms per step; the
# even split, 15 and 15: 0.733; 12: 0.725; 13-14: 0.734)
O_RING_MAX = 11
# caches from this length on take the KV-head-major attention (decode.hip dec_attend_kv): one
# workgroup per (KV head, slot) scores all G query heads of the K / V rows it reads on MFMA, G times
# fewer bytes per workgroup than one workgroup per (query head, slot), at a combine of G times more
# partials. Measured (Qwen2.5-1.5B, positions 128 before the cache end, tok/s KV-major /
# head-major): 8,192: 1,141 / 1,214; 10,240: 1,134 / 1,146; 12,288: 1,117 / 1,087; 14,336:
# 1,034 / 1,035; 16,384: 1,026 / 987; 24,576: 1,005 / 827. The kernel instances that have it, by
# (KC, EM)
KV_MAJOR_MIN_S = int(os.environ.get("HIPRT_DECODE_KV_MIN_S", "12288"))
KV_MAJOR = {(3, 2), (1, 1)}
MAX_KV_SLOTS = 128    # decode.hip DecShared::cwk (the combine's slot weights)
# query heads per KV head, at most, whose q / k / v rows, rotated rows and the 8 waves' chunk
# weights fit the attention staging (decode.hip DEC_SMEM, 8,448 bytes: 1,024 G + 768)
KV_MAX_G = 7
# gate/up rows a combine workgroup streams fewer than an o_proj workgroup: it waits for its head's
# partials and runs the combine before its o_proj, so with the o_proj workgroups' share its h and
# the next layer's rows were the last published (Qwen2.5-1.5B at 2048 positions: 11 - 4 = 7,
# 0.670 ms per step against 0.673 with 11; 5 or 3 with one row more per o_proj workgroup: 0.674)
C_RING_LESS = 4
# the head-major attention without combine workgroups: slot j of a head, once its partial is out,
# gathers dims j D / nsplit .. of all the head's partials and publishes them (decode.hip
# dec_combine_slot). Off: measured slower (Qwen2.5-1.5B at 2048 positions, 0.713 ms per step
# against 0.666: the attention row is out sooner, but o_proj's poll for it returns no sooner and
# the attention workgroups' gate / up rows, issued after the combine, land later)
SLOT_COMBINE = os.environ.get("HIPRT_DECODE_SLOT_COMBINE", "0") == "1"
OSTAGE = 128         # decode.hip DEC_OSTAGE: a workgroup's gate/up rows, staged

TABLE_FIELDS = ("norm1", "wq", "bq", "wk", "bk", "wv", "bv", "kc", "vc", "wo", "norm2", "wg", "wu", "wd")

QKV = ("k_qkv_rope_k1536", "k_qkv_rope")
FLASH = ("k_attn_flash_w8", "k_attn_flash", "k_attn_flash_w16", "k_attn_flash_chk")
OPROJ = ("k_gemv_attn16_resid_r2", "k_gemv_attn_resid_r2")    # the combine folded in
PLAIN = ("k_gemv_resid_r1", "k_gemv_resid_r2")                # after a k_attn_combine
DOWN = ("k_gemv_resid_ks_r2", "k_gemv_resid_r1")


def enabled() -> bool:
    return os.environ.get("HIPRT_PERSISTENT", "1") == "1"


def _device_resident(kernel: str) -> int | None:
    """Workgroups of ``kernel`` (``THREADS`` threads) that the current device holds at once: CUs x
    workgroups per CU. None when no GPU is visible (compiling on a CPU-only host)."""
    try:
        import torch

        if not torch.cuda.is_available():
            return None
    except ImportError:
        return None
    from hip_runtime.hip_executor import resident_workgroups

    return resident_workgroups(torch.cuda.current_device(), "decode", kernel, THREADS)


# Replaceable hook (tests fake a smaller device through it).
resident_workgroups = _device_resident


def work_split(hidden: int, inter: int, H: int, nslot: int, comb: bool = True) -> dict | None:
    """The kernel's division of a layer among the NWG workgroups (decode.hip ``decode_body``): NB
    attention workgroups (each also holds NE gate/up rows in LDS), ND o_proj workgroups of RD rows
    (those that run no combine also hold NEO gate/up rows in LDS); the gate/up rows left over are
    streamed through registers, RBO by each o_proj workgroup that runs no combine, RBC by each of
    the H combine workgroups and RBA by each attention workgroup; EM is the kernel instance's
    register rows per wave. ``comb`` False: the attention workgroups run the combine, the first H
    o_proj workgroups are like the others (RBC is then their stride in the gate/up rows, RBO +
    NEO). None when no instance fits."""
    KC = hidden // 512
    NB, NE = H * nslot, E_LDS_ROWS[KC]
    ND = NWG - NB
    if ND <= H:
        return None
    RD = -(-hidden // ND)
    if RD > 2 * NE:   # the o_proj rows of one workgroup must fit its LDS
        return None
    NEO = max(2 * NE - RD, 0) // 2
    HC = H if comb else 0
    ring = max(inter - NB * NE - (ND - HC) * NEO, 0)
    cap = 8 * max(RING_ROWS[KC])
    RBO = min(-(-ring // NWG), O_RING_MAX)
    RBO = max(RBO, -(-max(ring - NB * cap, 0) // ND))   # what the attention workgroups cannot take
    RBC = max(RBO - C_RING_LESS, 0) if comb else RBO + NEO
    RBA = -(-max(ring - (ND - HC) * RBO - HC * RBC, 0) // NB)
    RB = max(RBA, RBO)
    em = [e for e in RING_ROWS[KC] if 8 * e >= RB]
    if not em or max(NE, NEO) + RB > OSTAGE:
        return None
    return dict(NB=NB, NE=NE, ND=ND, RD=RD, NEO=NEO, RBO=RBO, RBC=RBC, RBA=RBA, EM=em[0])


def _parse_layers(steps: list[LaunchStep]):
    """Per layer (qkv, flash, combine or None, o_proj, gate/up, down), or None."""
    n = len(steps)
    layers, i = [], 1
    while i < n - 2:
        if i + 4 >= n - 2 or steps[i].kernel not in QKV or steps[i + 1].kernel not in FLASH:
            return None
        j, c = i + 2, None
        if steps[j].kernel == "k_attn_combine":
            c, j = steps[j], j + 1
        if j + 2 >= n - 2:
            return None
        o, g, d = steps[j], steps[j + 1], steps[j + 2]
        if c is None and o.kernel not in OPROJ or c is not None and o.kernel not in PLAIN:
            return None
        if g.kernel != "k_gemv_norm_silu_r1" or d.kernel not in DOWN:
            return None
        layers.append((steps[i], steps[i + 1], c, o, g, d))
        i = j + 3
    return layers if i == n - 2 and layers else None


def exchange_words(L: int, hidden: int, inter: int, H: int, KVH: int, nsplit: int) -> int:
    """32-bit words of the exchange area (decode.hip ``xlayout``): per layer the input row, each
    query head's q row with its KV head's k and v rows, the attention partials (o[D] plus m and l
    as four half-words per slot and head), the combined attention row, the o_proj output and the
    SiLU * up row; then the final row, one 64-bit argmax key per workgroup and two control words
    (step tag, timeout flag)."""
    stride = hidden + H * 3 * D + H * nsplit * (D + 4) + H * D + hidden + inter
    stride += stride & 1
    return stride * L + hidden + 2 * NWG + 2


def _same(a, b) -> bool:
    return isinstance(a, Ref) and isinstance(b, Ref) and a == b


def slots_for(S: int, hidden: int, inter: int, H: int) -> tuple[int, dict] | None:
    """Attention slots per query head for an S-position cache (as many as fit, up to MAX_SLOTS and
    one per chunk) with their work split, or None."""
    nchunk = -(-S // SPL)
    for nslot in range(min(nchunk, MAX_SLOTS), 0, -1):
        if -(-nchunk // nslot) > MAX_CHUNKS_PER_SLOT:
            return None
        ws = work_split(hidden, inter, H, nslot)
        if ws is not None:
            return nslot, ws
    return None


def fuse_decode_step(steps: list[LaunchStep], storages: dict[str, Storage]) -> list[LaunchStep] | None:
    """The one-launch form of ``steps``, or None when they are not a decode step it covers (or the
    device cannot hold all of its workgroups at once)."""
    n = len(steps)
    if n < 8:
        return None
    emb, lm, fin = steps[0], steps[-2], steps[-1]
    if emb.kernel != "k_embedding" or lm.kernel != "k_gemv_norm_argmax_r4" or fin.kernel != "k_argmax_finalize":
        return None
    layers = _parse_layers(steps)
    if layers is None:
        return None
    L = len(layers)
    ea, la, fa = emb.args, lm.args, fin.args
    q0, f0, g0 = layers[0][0].args, layers[0][1].args, layers[0][4].args
    hidden, H, KVH = int(q0["K"]), int(q0["H"]), int(q0["KVH"])
    inter, vocab, S = int(g0["N"]), int(la["N"]), int(f0["S"])
    if int(ea["n_ids"]) != 1 or int(ea["row_bytes"]) != 2 * hidden or int(ea["vocab"]) != vocab:
        return None
    if int(q0["D"]) != D or H * D != hidden or hidden % 512 or hidden // 512 not in VARIANTS:
        return None
    KC = hidden // 512
    if H % KVH or H // KVH > MAX_G or inter % 8 or inter > 4096 * KC or (H + 2 * KVH) * D > 8 * NWG:
        return None
    if vocab >= 2 ** 32:
        return None
    sl = slots_for(S, hidden, inter, H)
    if sl is None:
        return None
    nsplit, ws = sl
    # KV-head-major: the same NB attention workgroups as G nsplit slots per KV head
    G = H // KVH
    kvm = (S >= KV_MAJOR_MIN_S and (KC, ws["EM"]) in KV_MAJOR and G <= KV_MAX_G
           and G * nsplit <= MAX_KV_SLOTS
           and -(-(-(-S // SPL)) // (G * nsplit)) <= MAX_CHUNKS_PER_SLOT)
    if kvm:
        nsplit = G * nsplit
    # the head-major attention's workgroups combine their head's partials themselves
    scomb = not kvm and SLOT_COMBINE and work_split(hidden, inter, H, nsplit, comb=False) is not None
    if scomb:
        ws = work_split(hidden, inter, H, nsplit, comb=False)
    shared = ("pos_ids", "cache_pos", "inv_freq")
    x = ea["out"]
    table: list = []
    for q, f, c, o, g, d in layers:
        qa, fl, oa, ga, da = q.args, f.args, o.args, g.args, d.args
        if c is None:
            attn_ok = _same(oa["attn_o"], fl["part_o"])
        else:
            ca = c.args
            attn_ok = (_same(ca["part_o"], fl["part_o"]) and _same(ca["part_ml"], fl["part_ml"])
                       and _same(oa["x"], ca["out"]) and oa.get("bias") is None)
        ok = (
            attn_ok and _same(qa["x"], x) and _same(fl["q"], qa["q_out"]) and _same(fl["k"], qa["k_dst"])
            and _same(fl["v"], qa["v_dst"]) and _same(oa["resid"], x)
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
            and all(int(d) in (DTYPE_CODE["int64"], DTYPE_CODE["int32"])   # the kernel's branch-free loads
                    for d in (ea["ids_dtype"], q0["pos_dtype"], q0["cpos_dtype"]))
            and int(la["n_dtype"]) == int(q0["n_dtype"])):
        return None
    # the table holds graph inputs (caches) and weights only: the executor resolves it per set of
    # bound buffers, and arena storages get no offset of their own for it
    for r in table:
        if r is not None and storages[r.storage].kind not in ("input", "weight"):
            return None
    kernel = f"k_decode_step_k{KC}_i{KC}_e{ws['EM']}" + ("_kv" if kvm else "")
    fit = resident_workgroups(kernel)
    if fit is not None and fit < NWG:
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
        n_dtype=int(q0["n_dtype"]), out_dtype=int(fa["out_dtype"]),
        flags=(1 if int(q0["flags"]) & 2 else 0) | (2 if scomb else 0),
        eps=float(q0["eps"]), eps_f=float(la["eps"]), scale=float(f0["scale"]),
        rope_scaling=float(q0["rope_scaling"]), nchunk=-(-S // SPL), rbo=ws["RBO"], rba=ws["RBA"], rbc=ws["RBC"])
    inputs = sorted({t for st in steps for t in st.inputs})
    outputs = [t for st in steps for t in st.outputs]
    step = LaunchStep(
        kind="decode_step", kernel=kernel, module="decode", arg_struct="PersistArgs",
        args=args, grid=(NWG, 1, 1), block=(THREADS, 1, 1), inputs=inputs, outputs=outputs,
        params={"table": {"field": "layers", "entries": table}, "layers": L, "nsplit": nsplit,
                "replaces": [st.kernel for st in steps], "exchange_words": words, "work_split": ws,
                "kv_major": kvm, "slot_combine": scomb})
    return [step]


# ---------------------------------------------------------------- one attention block, one launch

AST_ROWS = 32        # decode.hip AST_ROWS: o_proj rows per workgroup, at most
OPROJ_ATT = OPROJ + ("k_gemv_attn16_bias_r2", "k_gemv_attn_bias_r2")   # combine folded in, [+ residual]
OPROJ_PLAIN = ("k_gemv_bias_r1", "k_gemv_bias_r4", "k_gemv_resid_r1", "k_gemv_resid_r2")


def attention_slots(S: int, hidden: int, H: int) -> int | None:
    """Attention slots per query head for ``k_attn_step`` over an S-position cache (as many as
    fit, up to MAX_SLOTS and one per chunk), or None: the H nslot attention workgroups, the H
    combine workgroups among the rest, and at most AST_ROWS o_proj rows for each of those."""
    nchunk = -(-S // SPL)
    for nslot in range(min(nchunk, MAX_SLOTS), 0, -1):
        if -(-nchunk // nslot) > MAX_CHUNKS_PER_SLOT:
            return None
        nd = NWG - H * nslot
        if nd > H and -(-hidden // nd) <= AST_ROWS:
            return nslot
    return None


def attention_step_words(H: int, nsplit: int) -> int:
    """32-bit words of ``k_attn_step``'s exchange area: per query head its q row with its KV head's
    k and v rows, the slot partials (o[D], m, l as four half-words), the attention row, then the
    step tag and the timeout flag."""
    return H * 3 * D + H * nsplit * (D + 4) + H * D + 2


def fuse_attention_step(steps: list[LaunchStep], storages: dict[str, Storage]) -> list[LaunchStep] | None:
    """The one-launch form (``k_attn_step_k<KC>``, csrc/kernels/decode.hip) of a launch list that is
    exactly one decode-token attention block: ``k_qkv_rope*`` (optional RMSNorm and biases, RoPE on
    q and k, both cache rows), ``k_attn_flash*`` and the o_proj GEMV with the combine folded in
    (or ``k_attn_combine`` then a plain GEMV), with or without a residual. None otherwise, or when
    the device cannot hold all of its workgroups at once."""
    if len(steps) == 3:
        q, f, o = steps
        c = None
        if o.kernel not in OPROJ_ATT:
            return None
    elif len(steps) == 4:
        q, f, c, o = steps
        if c.kernel != "k_attn_combine" or o.kernel not in OPROJ_PLAIN:
            return None
    else:
        return None
    if q.kernel not in QKV or f.kernel not in FLASH:
        return None
    qa, fl, oa = q.args, f.args, o.args
    hidden, H, KVH, S = int(qa["K"]), int(qa["H"]), int(qa["KVH"]), int(fl["S"])
    flags = int(qa["flags"])
    if int(qa["D"]) != D or H * D != hidden or hidden % 512 or hidden // 512 not in VARIANTS:
        return None
    if H % KVH or H // KVH > MAX_G or (H + 2 * KVH) * D > 8 * NWG or flags & 60 != 60:
        return None
    if c is None:
        attn_ok = _same(oa["attn_o"], fl["part_o"]) and _same(oa["attn_ml"], fl["part_ml"])
    else:
        ca = c.args
        attn_ok = (_same(ca["part_o"], fl["part_o"]) and _same(ca["part_ml"], fl["part_ml"])
                   and _same(oa["x"], ca["out"]))
    resid = oa.get("resid")
    ok = (
        attn_ok and _same(fl["q"], qa["q_out"]) and _same(fl["k"], qa["k_dst"]) and _same(fl["v"], qa["v_dst"])
        and isinstance(qa["x"], Ref) and isinstance(oa["out"], Ref) and (resid is None or isinstance(resid, Ref))
        and ((flags & 1) == 0 or isinstance(qa["norm_w"], Ref))
        and int(qa["cache_len"]) == S and int(qa["kv_head_stride"]) == int(fl["kv_head_stride"])
        and int(fl["H"]) == H and int(fl["KVH"]) == KVH and int(fl["dtype"]) == DTYPE_CODE["bfloat16"]
        and int(fl["q_head_stride"]) == D
        and (fl["mask"] is None or (int(fl["mask_stride"]) == 1 and int(fl["mask_dtype"]) in (0, 2)))
        and int(oa["N"]) == hidden and int(oa["K"]) == hidden and int(oa["M"]) == 1 and int(oa["flags"]) == 0
        and oa.get("bias") is None and oa.get("w2") is None and oa.get("norm_w") is None
        and all(int(d) in (DTYPE_CODE["int64"], DTYPE_CODE["int32"])   # the kernel's branch-free loads
                for d in (qa["pos_dtype"], qa["cpos_dtype"]))
    )
    if not ok:
        return None
    nsplit = attention_slots(S, hidden, H)
    if nsplit is None:
        return None
    bias = flags & 2
    table = [qa["norm_w"] if flags & 1 else None, qa["wq"], qa["bq"] if bias else None, qa["wk"],
             qa["bk"] if bias else None, qa["wv"], qa["bv"] if bias else None, qa["k_dst"], qa["v_dst"], oa["w"],
             None, None, None, None]
    for r in table:
        if r is not None and storages[r.storage].kind not in ("input", "weight"):
            return None
    KC = hidden // 512
    kernel = f"k_attn_step_k{KC}"
    fit = resident_workgroups(kernel)
    if fit is not None and fit < NWG:
        return None
    words = attention_step_words(H, nsplit)
    xname = "attn_step.exchange"
    storages[xname] = Storage(xname, "persistent", words * 4, "uint8", zero_init=True)
    mask = fl["mask"]
    args = dict(
        layers=None, pos_ids=qa["pos_ids"], cache_pos=qa["cache_pos"], mask=mask, inv_freq=qa["inv_freq"],
        ll=Ref(xname, 0), trace=None, S=S, kv_head_stride=int(qa["kv_head_stride"]), L=1, hidden=hidden, H=H,
        KVH=KVH, D=D, nsplit=nsplit, nwg=NWG, pos_dtype=int(qa["pos_dtype"]), cpos_dtype=int(qa["cpos_dtype"]),
        mask_dtype=int(fl["mask_dtype"]) if mask is not None else -1, add_dtype=int(fl.get("add_dtype", 2)),
        n_dtype=int(qa["n_dtype"]), flags=1 if bias else 0, eps=float(qa["eps"]), scale=float(fl["scale"]),
        rope_scaling=float(qa["rope_scaling"]), nchunk=-(-S // SPL), rows=-(-hidden // (NWG - H * nsplit)),
        xin=qa["x"], out=oa["out"], resid=resid)
    inputs = sorted({t for st in steps for t in st.inputs})
    outputs = [t for st in steps for t in st.outputs]
    step = LaunchStep(
        kind="attn_step", kernel=kernel, module="decode", arg_struct="PersistArgs",
        args=args, grid=(NWG, 1, 1), block=(THREADS, 1, 1), inputs=inputs, outputs=outputs,
        params={"table": {"field": "layers", "entries": table}, "layers": 1, "nsplit": nsplit,
                "replaces": [st.kernel for st in steps], "exchange_words": words})
    return [step]
