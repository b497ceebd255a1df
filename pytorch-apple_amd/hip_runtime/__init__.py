"""MI355X runtime: ``HIPBackend`` / ``HIPBuffer`` and the launch-list executor.

Drop-in counterpart of the reference's ``cuda_runtime`` package
(`cuda_runtime/__init__.py`, `cuda_backend.py`, `cuda_executor.py`).
"""

from hip_runtime.hip_backend import HIPBackend, HIPBuffer

__all__ = ["HIPBackend", "HIPBuffer", "HIPExecutor"]


def __getattr__(name):
    if name == "HIPExecutor":
        from hip_runtime.hip_executor import HIPExecutor

        return HIPExecutor
    raise AttributeError(name)
