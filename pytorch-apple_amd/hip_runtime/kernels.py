"""Kernel registry: ctypes mirrors of the argument structs and code-object loading.

Each ``csrc/kernels/*.hip`` file is compiled ahead of time into ``<name>.hsaco``
(``csrc/build.py``); generated elementwise chains are compiled with hiprtc and
cached on disk by source hash (the reference keeps an in-process md5 → RawKernel
cache, `cuda_runtime/cuda_executor.py:38-51`; this cache also survives processes
and travels with the tree). The ctypes structs below mirror
``csrc/kernels/common.h`` field for field; ``check_layouts()`` compares their sizes
with ``hs_argsize`` from the shim.
"""

from __future__ import annotations

import ctypes as C
import hashlib
import os

from hip_runtime import _shim

P = C.c_void_p
LL = C.c_longlong
I = C.c_int
F = C.c_float

STRUCTS: dict[str, type] = {}


def _struct(name: str, fields: list):
    cls = type(name, (C.Structure,), {"_fields_": fields})
    STRUCTS[name] = cls
    return cls


_struct("PersistArgs", [("layers", P), ("emb", P), ("ids", P), ("pos_ids", P), ("cache_pos", P), ("mask", P),
                        ("inv_freq", P), ("norm_f", P), ("lm_w", P), ("logits", P), ("next_token", P), ("ll", P),
                        ("trace", P), ("S", LL), ("kv_head_stride", LL), ("vocab", LL), ("L", I), ("hidden", I), ("inter", I),
                        ("H", I), ("KVH", I), ("D", I), ("nsplit", I), ("nwg", I), ("ids_dtype", I),
                        ("pos_dtype", I), ("cpos_dtype", I), ("mask_dtype", I), ("add_dtype", I), ("n_dtype", I),
                        ("out_dtype", I), ("flags", I), ("eps", F), ("eps_f", F), ("scale", F),
                        ("rope_scaling", F), ("adv_mask", P), ("adv_pos", P), ("adv_cpos", P), ("adv_flag", P),
                        ("adv_mask_bytes", I), ("adv_pad", I), ("nchunk", I), ("rbo", I), ("rba", I),
                        ("rbc", I), ("rows", I), ("host_err", P), ("xin", P), ("out", P), ("resid", P)])
_struct("CopyArgs", [("dst", P), ("src", P), ("n", LL), ("shape", LL * 6), ("sstride", LL * 6),
                     ("dstride", LL * 6), ("ndim", I), ("sdtype", I), ("ddtype", I), ("pad", I)])
_struct("FillArgs", [("out", P), ("n", LL), ("value", C.c_double), ("dtype", I), ("pad", I)])
_struct("AdvanceArgs", [("mask", P), ("pos", P), ("cpos", P), ("overflow", P), ("S", LL), ("mask_bytes", I),
                        ("pad", I)])
_struct("RMSNormArgs", [("x", P), ("w", P), ("out", P), ("rows", LL), ("ldx", LL), ("ldo", LL), ("cols", I),
                        ("eps", F), ("x_dtype", I), ("w_dtype", I), ("n_dtype", I), ("out_dtype", I)])
_struct("EmbeddingArgs", [("w", P), ("ids", P), ("out", P), ("n_ids", LL), ("vocab", LL), ("row_bytes", LL),
                          ("ids_dtype", I), ("pad", I)])
_struct("RopeTableArgs", [("inv_freq", P), ("pos", P), ("cos_out", P), ("sin_out", P), ("S", LL), ("half", I),
                          ("pos_dtype", I), ("out_dtype", I), ("scaling", F)])
_struct("IndexCopyArgs", [("dst", P), ("src", P), ("index", P), ("outer", LL), ("dim_size", LL), ("inner", LL),
                          ("nidx", LL), ("src_so", LL), ("src_sj", LL), ("src_si", LL), ("idx_dtype", I),
                          ("elem_bytes", I)])
_struct("SoftmaxArgs", [("x", P), ("mask", P), ("out", P), ("rows", LL), ("cols", LL), ("lead_shape", LL * 5),
                        ("x_lead_stride", LL * 5), ("mask_lead_stride", LL * 5), ("mask_col_stride", LL),
                        ("nlead", I), ("x_dtype", I), ("mask_dtype", I), ("add_dtype", I), ("out_dtype", I),
                        ("has_mask", I)])
_struct("ReduceLastArgs", [("x", P), ("out", P), ("rows", LL), ("cols", LL), ("x_dtype", I), ("out_dtype", I)])
_struct("BmmArgs", [("a", P), ("b", P), ("c", P), ("batch_shape", LL * 4), ("a_bstride", LL * 4),
                    ("b_bstride", LL * 4), ("M", LL), ("N", LL), ("K", LL), ("a_sm", LL), ("a_sk", LL),
                    ("b_sk", LL), ("b_sn", LL), ("nbatch", I), ("a_dtype", I), ("b_dtype", I), ("c_dtype", I)])
_struct("LinearArgs", [("x", P), ("w", P), ("bias", P), ("out", P), ("resid", P), ("M", LL), ("ldx", LL),
                       ("ldo", LL), ("ldr", LL), ("N", I), ("K", I), ("dtype", I), ("has_bias", I),
                       ("has_resid", I), ("pad", I)])
_struct("GemmArgs", [("x", P), ("w", P), ("w2", P), ("bias", P), ("bias2", P), ("resid", P), ("out", P),
                     ("part", P), ("w3", P), ("bias3", P), ("M", LL), ("ldx", LL), ("ldw", LL), ("ldo", LL),
                     ("ldr", LL), ("sx", LL), ("sw", LL), ("so", LL), ("batch", I), ("bdiv", I), ("N", I), ("K", I),
                     ("flags", I), ("ksplit", I), ("kchunk", I), ("nw", I), ("n1", I), ("n2", I), ("bn_w", P),
                     ("bn_b", P), ("bn_mean", P), ("bn_var", P), ("zero", P), ("eps", F), ("cH", I), ("cW", I),
                     ("cCin", I), ("cHo", I), ("cWo", I), ("cKW", I), ("csh", I), ("csw", I), ("cph", I), ("cpw", I)])
_struct("ConvArgs", [("x", P), ("w", P), ("bias", P), ("bn_w", P), ("bn_b", P), ("bn_mean", P), ("bn_var", P),
                     ("resid", P), ("out", P), ("part", P), ("M", LL), ("N", I), ("Cin", I), ("H", I), ("W", I),
                     ("Cout", I), ("Ho", I), ("Wo", I), ("KH", I), ("KW", I), ("sh", I), ("sw", I), ("ph", I),
                     ("pw", I), ("K", I), ("eps", F), ("flags", I), ("ksplit", I), ("kchunk", I)])
_struct("PoolArgs", [("x", P), ("out", P), ("planes", LL), ("H", I), ("W", I), ("Ho", I), ("Wo", I), ("kh", I),
                     ("kw", I), ("sh", I), ("sw", I), ("ph", I), ("pw", I), ("dtype", I), ("C", I)])
OHWI_MAX = 24   # HS_OHWI_MAX
_struct("PermuteOHWIArgs", [("src", P * OHWI_MAX), ("dst", P * OHWI_MAX), ("start", LL * (OHWI_MAX + 1)),
                            ("cin", I * OHWI_MAX), ("kh", I * OHWI_MAX), ("kw", I * OHWI_MAX), ("cp", I * OHWI_MAX),
                            ("khp", I * OHWI_MAX), ("kwp", I * OHWI_MAX), ("n", I), ("pad", I)])
_struct("PadNHWCArgs", [("x", P), ("out", P), ("n", LL), ("C", I), ("H", I), ("W", I), ("Hp", I), ("Wp", I),
                        ("top", I), ("left", I), ("pad", I)])
_struct("MeanNHWCArgs", [("x", P), ("out", P), ("n", LL), ("hw", I), ("c", I)])
_struct("BatchNormArgs", [("x", P), ("w", P), ("b", P), ("mean", P), ("var", P), ("out", P), ("n", LL),
                          ("hw", LL), ("C", I), ("eps", F), ("dtype", I), ("relu", I), ("p_dtype", I), ("pad", I)])
_struct("RopeCacheArgs", [("y", P), ("inv_freq", P), ("pos_ids", P), ("cache_pos", P), ("q_out", P), ("k_dst", P),
                          ("v_dst", P), ("ldy", LL), ("kv_head_stride", LL), ("cache_len", LL), ("T", I), ("H", I),
                          ("KVH", I), ("D", I), ("flags", I), ("pos_dtype", I), ("cpos_dtype", I), ("dtype", I),
                          ("rope_scaling", F)])
_struct("PrefillAttnArgs", [("q", P), ("k", P), ("v", P), ("mask", P), ("out", P), ("T", LL), ("S", LL),
                            ("q_head_stride", LL), ("kv_head_stride", LL), ("mask_row_stride", LL),
                            ("mask_col_stride", LL), ("H", I), ("KVH", I), ("scale", F), ("mask_dtype", I),
                            ("add_dtype", I), ("dtype", I), ("blk_limit", P)])
_struct("ReduceNormArgs", [("part", P), ("bias", P), ("resid", P), ("out", P), ("norm_w", P), ("norm_out", P),
                           ("M", LL), ("ldr", LL), ("ldo", LL), ("ldn", LL), ("N", I), ("ksplit", I), ("eps", F),
                           ("n_dtype", I), ("flags", I)])
_struct("MaskExtentArgs", [("mask", P), ("nblk_out", P), ("T", LL), ("S", LL), ("row_stride", LL),
                           ("col_stride", LL), ("mask_dtype", I)])
_struct("ArgmaxPartArgs", [("x", P), ("slot", P), ("rows", LL), ("cols", LL), ("seg", LL), ("x_dtype", I),
                           ("parts", I)])
_struct("FusedArgs", [("out", P), ("in", P * 8), ("n", LL)])
_struct("GemvArgs", [("x", P), ("w", P), ("bias", P), ("out", P), ("resid", P), ("w2", P), ("bias2", P),
                     ("norm_w", P), ("argmax_slot", P), ("attn_o", P), ("attn_ml", P), ("M", LL), ("ldx", LL),
                     ("ldo", LL), ("ldr", LL), ("N", I), ("K", I), ("eps", F), ("n_dtype", I), ("flags", I),
                     ("attn_heads", I), ("attn_kvh", I), ("attn_splits", I)])
_struct("FlashArgs", [("q", P), ("k", P), ("v", P), ("mask", P), ("part_o", P), ("part_ml", P), ("S", LL),
                      ("q_head_stride", LL), ("kv_head_stride", LL), ("mask_stride", LL), ("H", I), ("KVH", I),
                      ("nsplit", I), ("spl", I), ("scale", F), ("mask_dtype", I), ("add_dtype", I), ("dtype", I)])
_struct("CombineArgs", [("part_o", P), ("part_ml", P), ("out", P), ("H", I), ("KVH", I), ("nsplit", I),
                        ("dtype", I)])
_struct("ArgmaxFinalizeArgs", [("slot", P), ("out", P), ("rows", LL), ("parts", I), ("out_dtype", I)])
_struct("QKVArgs", [("x", P), ("norm_w", P), ("wq", P), ("bq", P), ("wk", P), ("bk", P), ("wv", P), ("bv", P),
                    ("inv_freq", P), ("pos_ids", P), ("cache_pos", P), ("q_out", P), ("k_dst", P), ("v_dst", P),
                    ("kv_head_stride", LL), ("cache_len", LL), ("K", I), ("H", I), ("KVH", I), ("D", I),
                    ("eps", F), ("n_dtype", I), ("flags", I), ("pos_dtype", I), ("cpos_dtype", I),
                    ("rope_scaling", F)])
_struct("AttnOutArgs", [("scores", P), ("stats", P), ("v", P), ("mask", P), ("out", P), ("S", LL),
                        ("kv_head_stride", LL), ("mask_stride", LL), ("H", I), ("KVH", I), ("ntiles", I),
                        ("mask_dtype", I), ("dtype", I), ("pad", I)])
_struct("DecodeAttnArgs", [("q", P), ("k", P), ("v", P), ("mask", P), ("out", P), ("scores", P), ("stats", P),
                           ("S", LL), ("q_head_stride", LL), ("kv_head_stride", LL),
                           ("mask_stride", LL), ("H", I), ("KVH", I), ("D", I), ("ntiles", I), ("scale", F),
                           ("mask_dtype", I), ("add_dtype", I), ("dtype", I)])


def check_layouts() -> dict[str, tuple[int, int]]:
    """Return {struct: (ctypes size, C size)} for every mismatch (empty when all agree)."""
    bad = {}
    for name, cls in STRUCTS.items():
        c_size = _shim.lib().hs_argsize(name.encode())
        if c_size != C.sizeof(cls):
            bad[name] = (C.sizeof(cls), c_size)
    return bad


def kernel_cache_dir() -> str:
    d = os.environ.get("HIPRT_KCACHE", os.path.join(_shim.PKG, ".kcache"))
    os.makedirs(d, exist_ok=True)
    return d


class ModuleCache:
    """Loaded code objects and function handles for one device."""

    def __init__(self):
        self.modules: dict[str, C.c_void_p] = {}
        self.functions: dict[tuple[str, str], int] = {}
        self._images: dict[str, bytes] = {}

    def _load(self, key: str, image: bytes) -> None:
        self._images[key] = image
        h = C.c_void_p()
        _shim.check(_shim.lib().hs_module_load(image, len(image), C.byref(h)), f"load {key}")
        self.modules[key] = h

    def ensure_builtin(self, module: str) -> None:
        if module in self.modules:
            return
        path = os.path.join(_shim.KERNEL_DIR, module + ".hsaco")
        if not os.path.exists(path):
            raise _shim.HIPShimError(f"code object {path} not built (run csrc/build.py)")
        _shim.check_built_from(path, [path[:-6] + ".hip", os.path.join(_shim.KERNEL_DIR, "common.h")])
        if not self.modules:   # first code object: the packed structs must match the built ones
            bad = check_layouts()
            if bad:
                raise _shim.HIPShimError(f"argument struct sizes differ from the built code (ctypes, C): {bad}")
        with open(path, "rb") as f:
            self._load(module, f.read())

    def ensure_generated(self, name: str, source: str) -> None:
        if name in self.modules:
            return
        self._load(name, generated_image(name, source))

    def function(self, module: str, kernel: str) -> int:
        key = (module, kernel)
        fn = self.functions.get(key)
        if fn is None:
            h = C.c_void_p()
            _shim.check(_shim.lib().hs_module_function(self.modules[module], kernel.encode(), C.byref(h)),
                        f"function {kernel}")
            fn = h.value
            self.functions[key] = fn
        return fn


def _common_header_hash() -> str:
    with open(os.path.join(_shim.KERNEL_DIR, "common.h"), "rb") as f:
        return hashlib.sha1(f.read()).hexdigest()[:12]


def generated_image(name: str, source: str) -> bytes:
    """Code object for generated source, from the on-disk cache or compiled with hiprtc."""
    key = hashlib.sha1((source + _common_header_hash()).encode()).hexdigest()[:20]
    path = os.path.join(kernel_cache_dir(), f"{name}-{key}.hsaco")
    if os.path.exists(path):
        with open(path, "rb") as f:
            return f.read()
    image = _shim.rtc_compile(source, name)
    tmp = f"{path}.{os.getpid()}.tmp"
    with open(tmp, "wb") as f:
        f.write(image)
    os.replace(tmp, path)
    return image
