"""The rotary sincos of the fused q/k/v kernel (``sincos_rot`` in csrc/kernels/common.h).

The reference forms the rotary tables as ``cos(inv_freq * position)`` in fp32
(Qwen2 rotary embedding: freqs = inv_freq @ positions, emb = cat(freqs, freqs),
cos/sin in fp32, then cast to the model dtype). The kernel computes the same fp32
angle and must return its sine and cosine to fp32 accuracy: here it is checked, on
the CPU (the same source built for the host), against the correctly rounded fp32
values of the float64 sine and cosine, for every angle a 128-dim head with
theta = 1e6 produces at positions 0..131071, plus reduction edge cases (multiples
of pi/2, large and negative angles). A wrong coefficient, quadrant or sign fails.
"""

import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
KERNELS = os.path.join(HERE, "..", "pytorch-apple_amd", "csrc", "kernels")


@pytest.fixture(scope="module")
def rot(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("needs g++")
    so = str(tmp_path_factory.mktemp("rot") / "librot.so")
    subprocess.run(["g++", "-O2", "-shared", "-fPIC", "-I", KERNELS, os.path.join(HERE, "rotary_host.cpp"),
                    "-o", so], check=True)
    lib = ctypes.CDLL(so)
    lib.rot_sincos.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_longlong]

    def f(x):
        x = np.ascontiguousarray(x, np.float32)
        s, c = np.empty_like(x), np.empty_like(x)
        lib.rot_sincos(x.ctypes.data, s.ctypes.data, c.ctypes.data, x.size)
        return s, c

    return f


def test_rotary_angles_are_correctly_rounded(rot):
    inv = (1.0 / (1e6 ** (np.arange(0, 128, 2, dtype=np.int64).astype(np.float32) / 128))).astype(np.float32)
    pos = np.arange(131072, dtype=np.float32)
    x = (inv[:, None] * pos[None, :]).astype(np.float32).ravel()   # fp32 products, as the reference forms them
    s, c = rot(x)
    xd = x.astype(np.float64)
    assert np.array_equal(s, np.sin(xd).astype(np.float32))
    assert np.array_equal(c, np.cos(xd).astype(np.float32))


def test_rotary_reduction_edge_cases(rot):
    k = np.arange(-4096, 4097, dtype=np.float64)
    near = np.concatenate([k * np.pi / 2, k * np.pi / 4, [0.0, 1e-30, -1e-30, 1e-8, 3.0e5, -3.0e5, 1.0e6]])
    x = near.astype(np.float32)
    x = np.concatenate([x, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(-np.inf))])
    s, c = rot(x)
    xd = x.astype(np.float64)
    assert np.array_equal(s, np.sin(xd).astype(np.float32))
    assert np.array_equal(c, np.cos(xd).astype(np.float32))
