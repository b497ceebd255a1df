"""HIP backend: ``Backend`` / ``DeviceBuffer`` over PyTorch-ROCm device tensors.

Drop-in counterpart of the reference's ``CUDABackend`` / ``CUDABuffer``
(`cuda_runtime/cuda_backend.py:24-150`) with the same methods, including the two
extras ``DAGExecutor`` uses (``to_numpy(dtype=...)``, ``write_from_numpy(data,
spec=...)``). Unlike the reference, dtypes are preserved (the reference casts
every float to fp16 and stages integer inputs through fp16, D1/D2): bf16 stays
bf16 (host carrier: uint16 bits), int64 stays int64.

PyTorch is used only to own device memory and to order host↔device copies on
its current stream; kernels are launched through the C-ABI shim.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from npu_runtime.backend import Backend, DeviceBuffer
from npu_runtime.cpu_fallback import torch_to_numpy

_TORCH_OF_IR = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
                "int64": torch.int64, "int32": torch.int32, "bool": torch.bool, "float64": torch.float64,
                "uint8": torch.uint8, "int8": torch.int8}
_NP_CARRIER = {torch.float32: np.float32, torch.float16: np.float16, torch.bfloat16: np.uint16,
               torch.int64: np.int64, torch.int32: np.int32, torch.bool: np.bool_, torch.float64: np.float64,
               torch.uint8: np.uint8, torch.int8: np.int8}


def torch_dtype_for(np_dtype=None, ir_dtype: str | None = None) -> torch.dtype:
    if ir_dtype is not None:
        return _TORCH_OF_IR[ir_dtype]
    dt = np.dtype(np_dtype)
    if dt == np.uint16:
        return torch.bfloat16
    return torch.from_numpy(np.zeros(1, dtype=dt)).dtype


def host_to_tensor(data, dtype: torch.dtype) -> torch.Tensor:
    """numpy (or tensor) → CPU tensor of ``dtype``; uint16 input is taken as bf16 bits."""
    if isinstance(data, torch.Tensor):
        t = data
    else:
        arr = np.ascontiguousarray(data)
        if arr.dtype == np.uint16:
            t = torch.from_numpy(arr).view(torch.bfloat16)
        else:
            t = torch.from_numpy(arr)
    if t.dtype != dtype:
        t = t.to(dtype)
    return t


class HIPBuffer(DeviceBuffer):
    """A device tensor with a logical shape; bf16 is exported to numpy as uint16 bits."""

    def __init__(self, tensor: torch.Tensor, logical_shape: tuple[int, ...] | None = None):
        self._t = tensor
        self._shape = tuple(logical_shape) if logical_shape is not None else tuple(tensor.shape)
        self._stage: torch.Tensor | None = None
        self._stage_evt: torch.cuda.Event | None = None

    @property
    def shape(self) -> tuple[int, ...]:
        return self._shape

    @property
    def alloc_shape(self) -> tuple[int, ...]:
        return tuple(self._t.shape)

    @property
    def dtype(self) -> np.dtype:
        return np.dtype(_NP_CARRIER[self._t.dtype])

    @property
    def torch_dtype(self) -> torch.dtype:
        return self._t.dtype

    @property
    def size_bytes(self) -> int:
        return self._t.numel() * self._t.element_size()

    @property
    def native_handle(self) -> torch.Tensor:
        return self._t

    @property
    def data_ptr(self) -> int:
        return self._t.data_ptr()

    def to_numpy(self, spec=None, dtype=None) -> np.ndarray:
        t = self._t
        n = int(np.prod(self._shape)) if self._shape else 1
        if tuple(t.shape) != self._shape:
            t = t.reshape(-1)[:n].reshape(self._shape)
        arr = torch_to_numpy(t)
        if dtype is not None and np.dtype(dtype) != arr.dtype:
            arr = arr.astype(dtype)
        return arr

    def to_torch(self) -> torch.Tensor:
        """The device tensor with the logical shape (no copy)."""
        n = int(np.prod(self._shape)) if self._shape else 1
        if tuple(self._t.shape) == self._shape:
            return self._t
        return self._t.reshape(-1)[:n].reshape(self._shape)

    def write_from_numpy(self, data, spec=None) -> None:
        """In-place upload, ordered on torch's current stream through a pinned staging buffer."""
        src = host_to_tensor(data, self._t.dtype).reshape(-1)
        n = min(src.numel(), self._t.numel())
        if self._stage is None or self._stage.numel() < n:
            self._stage = torch.empty(max(n, 1), dtype=self._t.dtype, pin_memory=True)
            self._stage_evt = torch.cuda.Event()
        else:
            self._stage_evt.synchronize()
        self._stage[:n].copy_(src[:n])
        self._t.view(-1)[:n].copy_(self._stage[:n], non_blocking=True)
        self._stage_evt.record()
        self._shape = tuple(np.shape(data)) if not isinstance(data, torch.Tensor) else tuple(data.shape)

    @classmethod
    def from_numpy(cls, data, dtype: torch.dtype | None = None, device: torch.device | str = "cuda") -> "HIPBuffer":
        if isinstance(data, torch.Tensor):
            dt = dtype or data.dtype
        else:
            dt = dtype or torch_dtype_for(data.dtype)
        t = host_to_tensor(data, dt).to(device)
        return cls(t)

    @classmethod
    def zeros(cls, shape, dtype: torch.dtype = torch.float16, device: torch.device | str = "cuda") -> "HIPBuffer":
        return cls(torch.zeros(tuple(shape), dtype=dtype, device=device))


class HIPBackend(Backend):
    """MI355X execution backend (one device per backend)."""

    def __init__(self, device_id: int = 0):
        self._device_id = device_id
        self._device = torch.device("cuda", device_id)
        self._ready = False

    def _ensure(self) -> None:
        if self._ready:
            return
        if not torch.cuda.is_available():
            raise RuntimeError("HIPBackend needs a ROCm GPU (torch.cuda.is_available() is False)")
        from hip_runtime import _shim

        torch.cuda.set_device(self._device_id)
        _shim.check(_shim.lib().hs_init(self._device_id), "hs_init")
        self._ready = True

    @property
    def name(self) -> str:
        return "hip"

    @property
    def device(self) -> torch.device:
        return self._device

    def allocate_buffer(self, data, alloc_shape=None, spec=None) -> HIPBuffer:
        self._ensure()
        if isinstance(data, HIPBuffer):
            return data
        ir_dt = getattr(spec, "dtype", None) if spec is not None else (spec.get("dtype") if isinstance(spec, dict) else None)
        if isinstance(data, torch.Tensor):
            dt = _TORCH_OF_IR[ir_dt] if ir_dt else data.dtype
            t = data.detach()
            if t.device != self._device or t.dtype != dt:
                t = t.to(device=self._device, dtype=dt)
            return HIPBuffer(t.contiguous())
        dt = torch_dtype_for(data.dtype, ir_dt)
        t = host_to_tensor(data, dt).to(self._device)
        return HIPBuffer(t)

    def allocate_zeros(self, shape, dtype=np.dtype(np.float16), alloc_shape=None) -> HIPBuffer:
        self._ensure()
        tdt = dtype if isinstance(dtype, torch.dtype) else torch_dtype_for(dtype)
        return HIPBuffer(torch.zeros(tuple(alloc_shape or shape), dtype=tdt, device=self._device),
                         logical_shape=tuple(shape))

    def execute(self, program, inputs, weights) -> dict[str, HIPBuffer]:
        return self.create_executor(program).run(inputs, weights)

    def create_executor(self, program) -> Any:
        self._ensure()
        from hip_runtime.hip_executor import HIPExecutor

        return HIPExecutor(program, self)

    def decode_advance(self, mask: HIPBuffer, pos: HIPBuffer, cpos: HIPBuffer):
        """A callable that moves a decode loop's mask / position inputs to the next step on the
        device (one launch of ``k_decode_advance`` on the current stream)."""
        self._ensure()
        from hip_runtime.hip_executor import DecodeAdvance

        return DecodeAdvance(mask, pos, cpos)

    def synchronize(self):
        torch.cuda.synchronize(self._device)
