"""Abstract backend interfaces (`npu_runtime/backend.py:11-68`).

``DAGExecutor`` only talks to a device through these two ABCs plus two duck-typed
extras that the reference's executor also relies on: ``to_numpy(dtype=...)`` as a
keyword and ``write_from_numpy(data, spec=...)``.

bfloat16 has no numpy dtype in this environment (``ml_dtypes`` is absent), so a
bf16 tensor crosses the host boundary as a ``uint16`` array holding the raw bits,
the same carrier the reference accepts in ``cpu_fallback._numpy_to_torch``.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any

import numpy as np


class DeviceBuffer(ABC):
    @property
    @abstractmethod
    def shape(self) -> tuple[int, ...]: ...

    @property
    @abstractmethod
    def alloc_shape(self) -> tuple[int, ...]: ...

    @property
    @abstractmethod
    def dtype(self) -> np.dtype: ...

    @property
    @abstractmethod
    def size_bytes(self) -> int: ...

    @property
    @abstractmethod
    def native_handle(self) -> Any: ...

    @abstractmethod
    def to_numpy(self, spec=None) -> np.ndarray: ...


class Backend(ABC):
    @property
    @abstractmethod
    def name(self) -> str: ...

    @property
    @abstractmethod
    def device(self) -> Any: ...

    @abstractmethod
    def allocate_buffer(self, data: np.ndarray, alloc_shape=None, spec=None) -> DeviceBuffer: ...

    @abstractmethod
    def allocate_zeros(self, shape, dtype=np.dtype(np.float16), alloc_shape=None) -> DeviceBuffer: ...

    @abstractmethod
    def execute(self, program, inputs, weights) -> dict[str, DeviceBuffer]: ...

    @abstractmethod
    def create_executor(self, program) -> Any: ...

    @abstractmethod
    def synchronize(self): ...
