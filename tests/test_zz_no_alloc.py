"""hs_argmax_rows_noalloc through the C-ABI: the same result as hs_argmax_rows (caller-provided
workspace) and np.argmax, bit for bit, on two calls in a row, the second with a smaller input
(the library's scratch array keeps the first call's keys; the second must not read them)."""

import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


def _logits(rows, cols, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g).bfloat16()
    x[0, cols // 3] = x[0].max() + 2
    return x


def _with_workspace(lib, _shim, x, stream):
    rows, cols = x.shape
    out = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
    ws = torch.empty(lib.hs_argmax_workspace_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    _shim.check(lib.hs_argmax_rows(x.data_ptr(), 2, rows, cols, out.data_ptr(), ws.data_ptr(), ws.numel(), stream),
                "hs_argmax_rows")
    return out


def test_noalloc_argmax_matches_the_workspace_entry_point_twice():
    from hip_runtime import _shim

    lib = _shim.lib()
    _shim.check(lib.hs_init(0), "hs_init")
    stream = torch.cuda.current_stream().cuda_stream
    for rows, cols, seed in ((512, 151936, 1), (3, 1000, 2)):   # the second call is smaller
        print(f"[case] hs_argmax_rows_noalloc rows={rows} cols={cols}", flush=True)
        x = _logits(rows, cols, seed).cuda()
        got = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
        _shim.check(lib.hs_argmax_rows_noalloc(x.data_ptr(), 2, rows, cols, got.data_ptr(), stream),
                    "hs_argmax_rows_noalloc")
        ref = _with_workspace(lib, _shim, x, stream)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        assert np.array_equal(got.cpu().numpy(), np.argmax(x.float().cpu().numpy(), axis=1))


def test_noalloc_argmax_rejects_inputs_beyond_its_scratch():
    from hip_runtime import _shim

    lib = _shim.lib()
    x = torch.zeros(8, 16, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(3500, dtype=torch.int64, device="cuda")
    rc = lib.hs_argmax_rows_noalloc(x.data_ptr(), 2, 3500, 151936, out.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"exceeds the no-alloc scratch" in lib.hs_last_error()
