"""ctypes binding of the C-ABI shim (``include/hipshim.h``, ``csrc/libhipshim.so``).

The shim is required: there is no Python or CPU fallback behind these calls. If
the library is missing the import of ``hip_runtime`` still works (so CPU-only
code paths can run), but the first call raises ``HIPShimError``.
"""

from __future__ import annotations

import ctypes as C
import hashlib
import os

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG, "csrc", "libhipshim.so")
KERNEL_DIR = os.path.join(PKG, "csrc", "kernels")
# what libhipshim.so is built from (csrc/build.py SHIM_SOURCES)
SHIM_SOURCES = [os.path.join(PKG, "csrc", "shim.cpp"), os.path.join(KERNEL_DIR, "common.h"),
                os.path.join(os.path.dirname(PKG), "include", "hipshim.h")]


class HIPShimError(RuntimeError):
    pass


class LaunchRec(C.Structure):
    _fields_ = [("fn", C.c_void_p), ("grid", C.c_uint32 * 3), ("block", C.c_uint32 * 3),
                ("lds_bytes", C.c_uint32), ("kernarg_size", C.c_uint32), ("kernarg", C.c_void_p)]


_SIGS = {
    "hs_init": ([C.c_int], C.c_int),
    "hs_device_count": ([C.POINTER(C.c_int)], C.c_int),
    "hs_last_error": ([], C.c_char_p),
    "hs_module_load": ([C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)], C.c_int),
    "hs_module_unload": ([C.c_void_p], C.c_int),
    "hs_module_function": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p)], C.c_int),
    "hs_rtc_compile": ([C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, C.POINTER(C.c_void_p),
                        C.POINTER(C.c_size_t), C.POINTER(C.c_void_p)], C.c_int),
    "hs_free_host": ([C.c_void_p], None),
    "hs_launch": ([C.c_void_p] + [C.c_uint32] * 7 + [C.c_void_p, C.c_void_p, C.c_size_t], C.c_int),
    "hs_replay": ([C.POINTER(LaunchRec), C.c_size_t, C.c_void_p], C.c_int),
    "hs_graph_capture": ([C.POINTER(LaunchRec), C.c_size_t, C.c_void_p, C.POINTER(C.c_void_p)], C.c_int),
    "hs_graph_launch": ([C.c_void_p, C.c_void_p], C.c_int),
    "hs_graph_destroy": ([C.c_void_p], C.c_int),
    "hs_stream_create": ([C.POINTER(C.c_void_p)], C.c_int),
    "hs_stream_destroy": ([C.c_void_p], C.c_int),
    "hs_stream_sync": ([C.c_void_p], C.c_int),
    "hs_device_sync": ([], C.c_int),
    "hs_event_create": ([C.POINTER(C.c_void_p)], C.c_int),
    "hs_event_destroy": ([C.c_void_p], C.c_int),
    "hs_event_record": ([C.c_void_p, C.c_void_p], C.c_int),
    "hs_event_sync": ([C.c_void_p], C.c_int),
    "hs_event_elapsed_ms": ([C.c_void_p, C.c_void_p, C.POINTER(C.c_float)], C.c_int),
    "hs_memcpy_htod": ([C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "hs_memcpy_dtoh": ([C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "hs_memcpy_dtod": ([C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p], C.c_int),
    "hs_argmax_workspace_bytes": ([C.c_int64, C.c_int64], C.c_size_t),
    "hs_argmax_rows": ([C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p],
                       C.c_int),
    "hs_argmax_rows_noalloc": ([C.c_void_p, C.c_int, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p], C.c_int),
    "hs_device_cus": ([C.POINTER(C.c_int)], C.c_int),
    "hs_occupancy": ([C.c_void_p, C.c_uint32, C.c_size_t, C.POINTER(C.c_int)], C.c_int),
    "hs_host_alloc_mapped": ([C.c_size_t, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)], C.c_int),
    "hs_argsize": ([C.c_char_p], C.c_size_t),
}
EXPORTED = tuple(_SIGS)

_lib = None


def _source_hash(paths: list[str]) -> str:
    h = hashlib.sha1()
    for p in paths:
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def check_built_from(out: str, sources: list[str]) -> None:
    """Raise ``HIPShimError`` unless ``out`` was built from the current bytes of ``sources``
    (the ``<out>.srchash`` stamp written by ``csrc/build.py``). A code object or shim older
    than ``common.h`` disagrees with the argument structs the host packs, and a kernel that
    reads fields past the packed struct would take them from unrelated memory."""
    try:
        with open(out + ".srchash") as f:
            stamp = f.read().strip()
    except OSError:
        raise HIPShimError(f"{out} has no build stamp; rebuild (`python -c 'import __graft_entry__ as g; g.build()'`)")
    if stamp != _source_hash(sources):
        raise HIPShimError(f"{out} is older than its sources; rebuild (`python -c 'import __graft_entry__ as g; "
                           f"g.build()'`)")


def lib():
    """Load ``libhipshim.so`` once; raise ``HIPShimError`` when it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HIPShimError(f"{LIB_PATH} not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        check_built_from(LIB_PATH, SHIM_SOURCES)
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().hs_last_error().decode(errors="replace")
        raise HIPShimError(f"{what}: rc={rc}: {msg}")


def rtc_compile(source: str, name: str, arch: str = "gfx950", include_dir: str = KERNEL_DIR) -> bytes:
    """Compile generated HIP source to a code object with hiprtc (through the shim)."""
    img = C.c_void_p()
    n = C.c_size_t()
    log = C.c_void_p()
    rc = lib().hs_rtc_compile(source.encode(), (name + ".hip").encode(), arch.encode(), include_dir.encode(),
                              C.byref(img), C.byref(n), C.byref(log))
    text = C.string_at(log.value).decode(errors="replace") if log.value else ""
    if log.value:
        lib().hs_free_host(log)
    if rc != 0:
        raise HIPShimError(f"hiprtc failed for {name}: {lib().hs_last_error().decode()}\n{text}")
    data = C.string_at(img.value, n.value)
    lib().hs_free_host(img)
    return data
