"""The C-ABI library: it loads, exports every entry point include/hipshim.h declares, agrees
with the host's ctypes mirrors on every kernel-argument struct, and reports errors instead
of aborting. No kernel is launched here."""

import ctypes as C
import os
import re

import pytest
import torch

from hip_runtime import _shim
from hip_runtime.kernels import STRUCTS, check_layouts

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "hipshim.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(hs_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    lib = _shim.lib()
    names = declared_symbols()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_shim.EXPORTED)


def test_kernel_argument_layouts_match():
    assert check_layouts() == {}
    assert _shim.lib().hs_argsize(b"NoSuchStruct") == 0
    assert C.sizeof(STRUCTS["GemvArgs"]) % 8 == 0


def test_built_code_matches_its_sources():
    """Every code object and the shim carry the hash of the sources they were built from, and
    the tree's built files are current (a stale code object reads argument fields the host no
    longer packs)."""
    kdir = _shim.KERNEL_DIR
    _shim.check_built_from(_shim.LIB_PATH, _shim.SHIM_SOURCES)
    built = [f for f in os.listdir(kdir) if f.endswith(".hsaco")]
    assert len(built) >= 6
    for f in built:
        _shim.check_built_from(os.path.join(kdir, f), [os.path.join(kdir, f[:-6] + ".hip"),
                                                      os.path.join(kdir, "common.h")])


def test_stale_build_is_refused(tmp_path):
    src, hdr, out = tmp_path / "k.hip", tmp_path / "common.h", tmp_path / "k.hsaco"
    src.write_text("kernel v1")
    hdr.write_text("struct A { int x; };")
    out.write_bytes(b"code")
    with pytest.raises(_shim.HIPShimError, match="no build stamp"):
        _shim.check_built_from(str(out), [str(src), str(hdr)])
    (tmp_path / "k.hsaco.srchash").write_text(_shim._source_hash([str(src), str(hdr)]) + "\n")
    _shim.check_built_from(str(out), [str(src), str(hdr)])
    hdr.write_text("struct A { int x; void* pf; };")
    with pytest.raises(_shim.HIPShimError, match="older than its sources"):
        _shim.check_built_from(str(out), [str(src), str(hdr)])


def test_init_reports_errors_without_aborting():
    lib = _shim.lib()
    rc = lib.hs_init(12345)
    assert rc != 0
    assert b"out of range" in lib.hs_last_error() or lib.hs_last_error()
    if not torch.cuda.is_available():
        assert lib.hs_init(0) != 0


def test_runtime_compile_of_a_generated_kernel_without_a_device():
    from hip_compiler import compile_subgraph
    from irgen.qwen import build_mlp_ir

    p = compile_subgraph(build_mlp_ir(4), fuse=False)
    ks = p.kernel_sources[0]
    image = _shim.rtc_compile(ks.source_code, ks.kernel_name)
    assert image[:4] == b"\x7fELF" or image[:24].startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    with pytest.raises(_shim.HIPShimError):
        _shim.rtc_compile("this is not C++", "broken")


def test_backend_fails_loudly_without_a_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from hip_runtime import HIPBackend

    with pytest.raises(RuntimeError, match="ROCm GPU"):
        HIPBackend().allocate_zeros((2, 2))


def test_argmax_entry_point_sizes_and_rejects_bad_operands_without_launching():
    """hs_argmax_rows validates before any HIP call, so these run without a device."""
    lib = _shim.lib()
    assert lib.hs_argmax_workspace_bytes(1, 151936) == 19 * 8          # 8192-column parts
    assert lib.hs_argmax_workspace_bytes(512, 151936) == 512 * 19 * 8
    assert lib.hs_argmax_workspace_bytes(3, 8) == 3 * 8
    assert lib.hs_argmax_workspace_bytes(0, 100) == 0
    buf = (C.c_uint16 * 64)()
    out = (C.c_int64 * 4)()
    ws = (C.c_uint64 * 8)()
    base = C.addressof(buf)
    aligned = base + (-base) % 16
    cases = [
        (aligned, 2, 1, 12, "multiple of 8"),       # cols % 8 != 0
        (aligned, 0, 1, 16, "dtype"),               # fp32 not supported
        (aligned + 2, 2, 1, 16, "16-byte aligned"),
        (aligned, 2, 70000, 16, "rows"),
    ]
    for x, dt, rows, cols, msg in cases:
        rc = lib.hs_argmax_rows(x, dt, rows, cols, C.addressof(out), C.addressof(ws), C.sizeof(ws), None)
        assert rc != 0 and msg.encode() in lib.hs_last_error(), (msg, lib.hs_last_error())
    rc = lib.hs_argmax_rows(aligned, 2, 1, 16, C.addressof(out), C.addressof(ws), 4, None)
    assert rc != 0 and b"workspace" in lib.hs_last_error()
    assert lib.hs_argmax_rows(aligned, 2, 0, 16, C.addressof(out), None, 0, None) == 0   # no rows: nothing to do
