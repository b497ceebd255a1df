"""hs_argmax_rows through the C-ABI on the GPU: the device argmax that replaces the host
np.argmax over logits in the reference's generation loops (examples/run_qwen.py:125,180),
bit-exact against np.argmax (first index on ties, NaN largest, -0.0 == +0.0)."""

import ctypes as C

import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]


def _rows(rows, cols, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    if rows > 1:
        x[1, 7] = x[1, cols - 9] = x[1].max() + 1      # tie: the first index wins
    if rows > 2:
        x[2, 100] = float("nan")                       # NaN is the largest
        x[2, 50] = float("nan")
    if rows > 3:
        x[3] = -0.0
        x[3, 9] = 0.0                                  # all zeros: index 0
    return x


def _expect(x):
    # np.argmax on float32 values: NaN counts as the maximum, first index on ties, -0 == +0
    return np.argmax(x.float().numpy(), axis=1)


@pytest.mark.parametrize("rows,cols,dtype", [(5, 151936, torch.bfloat16), (4, 1000, torch.float16),
                                             (1, 8, torch.bfloat16), (130, 8200, torch.bfloat16)])
def test_argmax_rows_through_the_c_abi(rows, cols, dtype):
    from hip_runtime import _shim

    lib = _shim.lib()
    x = _rows(rows, cols, dtype, seed=rows + cols).cuda()
    out = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
    ws = torch.empty(lib.hs_argmax_workspace_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    code = 2 if dtype == torch.bfloat16 else 1
    stream = torch.cuda.current_stream().cuda_stream
    print(f"[case] hs_argmax_rows rows={rows} cols={cols} {dtype}", flush=True)
    _shim.check(lib.hs_argmax_rows(x.data_ptr(), code, rows, cols, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                   stream), "hs_argmax_rows")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), _expect(x.cpu()))
