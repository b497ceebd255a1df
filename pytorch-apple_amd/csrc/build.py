"""Build the native parts: the C-ABI shim (libhipshim.so) and the gfx950 code objects.

``python csrc/build.py`` compiles, in-tree:
* ``csrc/libhipshim.so`` from ``shim.cpp`` (hipcc, host + HIP runtime + hiprtc);
* ``csrc/kernels/<name>.hsaco`` from each ``csrc/kernels/<name>.hip`` with
  ``hipcc --genco --offload-arch=gfx950``.
Every HIP compile carries ``-Xclang -target-feature -Xclang -packed-fp32-ops``
(packed FP32 instructions disabled). No GPU is needed.
"""

from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
NO_PK_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
KDIR = os.path.join(HERE, "kernels")


SHIM_SOURCES = [os.path.join(HERE, "shim.cpp"), os.path.join(KDIR, "common.h"), os.path.join(ROOT, "include", "hipshim.h")]


def source_hash(paths: list[str]) -> str:
    """sha1 over the files' bytes in order; stored beside each built file as ``<out>.srchash``
    so the loader (``hip_runtime/_shim.py``) refuses a build older than its sources."""
    h = hashlib.sha1()
    for p in paths:
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def _stamp(out: str, sources: list[str]) -> None:
    with open(out + ".srchash.tmp", "w") as f:
        f.write(source_hash(sources) + "\n")
    os.replace(out + ".srchash.tmp", out + ".srchash")


def _run(cmd: list[str]) -> None:
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{p.stdout}\n{p.stderr}")


def build_shim() -> str:
    out = os.path.join(HERE, "libhipshim.so")
    _run([HIPCC, "-O2", "-fPIC", "-shared", f"--offload-arch={ARCH}", *NO_PK_FP32, "-std=c++17",
          "-I", os.path.join(ROOT, "include"), os.path.join(HERE, "shim.cpp"), "-o", out + ".tmp",
          "-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(out + ".tmp", out)
    _stamp(out, SHIM_SOURCES)
    return out


def build_kernel(src: str) -> str:
    out = src[:-4] + ".hsaco"
    _run([HIPCC, "--genco", f"--offload-arch={ARCH}", "-O3", "-std=c++17", *NO_PK_FP32, "-I", KDIR, src,
          "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    _stamp(out, [src, os.path.join(KDIR, "common.h")])
    return out


def kernel_sources() -> list[str]:
    return sorted(os.path.join(KDIR, f) for f in os.listdir(KDIR) if f.endswith(".hip"))


def build_all(verbose: bool = True) -> list[str]:
    srcs = kernel_sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + 1)) as ex:
        futs = [ex.submit(build_shim)] + [ex.submit(build_kernel, s) for s in srcs]
        outs = [f.result() for f in futs]
    if verbose:
        for o in outs:
            print("built", os.path.relpath(o, ROOT))
    return outs


if __name__ == "__main__":
    build_all()
    sys.exit(0)
