from npu_runtime.backend import Backend, DeviceBuffer
from npu_runtime.cpu_fallback import execute_cpu_partition
from npu_runtime.dag_executor import DAGExecutor

__all__ = ["Backend", "DeviceBuffer", "DAGExecutor", "execute_cpu_partition"]
