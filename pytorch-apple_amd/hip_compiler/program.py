"""Program data model of the HIP backend: tensor views, launch steps, arena plan.

The reference's CUDA program (`cuda_compiler/cuda_program.py:15-111`) is a list of
typed steps (cuBLAS calls, fused kernels, reductions, specials, aliases) plus one
``BufferAllocation`` per intermediate. Here every step is already a concrete
kernel launch (kernel name, grid, block and a by-value argument record whose
pointer fields are symbolic references into storages), aliases are resolved at
compile time into strided views, and intermediates live at planned offsets of
one device arena. The attributes ``DAGExecutor`` reads (``input_specs``,
``output_specs``, ``weight_specs``, ``weight_name_mapping``, ``compute_dtype``)
keep the reference's names and meaning.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from npu_compiler.ir_reader import TensorSpec

ELEM_SIZE = {"float32": 4, "float16": 2, "bfloat16": 2, "int64": 8, "int32": 4, "bool": 1, "uint8": 1,
             "int8": 1, "float64": 8}
DTYPE_CODE = {"float32": 0, "float16": 1, "bfloat16": 2, "int64": 3, "int32": 4, "bool": 5, "uint8": 5,
              "float64": 6}
FLOAT_DTYPES = {"float32", "float16", "bfloat16", "float64"}


def contiguous_strides(shape) -> tuple[int, ...]:
    st, acc = [], 1
    for s in reversed(list(shape)):
        st.append(acc)
        acc *= max(int(s), 1)
    return tuple(reversed(st))


def numel(shape) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


@dataclass(frozen=True)
class TView:
    """A strided view (element offset and strides) of one storage."""

    storage: str
    offset: int
    shape: tuple[int, ...]
    strides: tuple[int, ...]
    dtype: str

    @property
    def numel(self) -> int:
        return numel(self.shape)

    @property
    def itemsize(self) -> int:
        return ELEM_SIZE[self.dtype]

    def is_contiguous(self) -> bool:
        exp = 1
        for s, st in zip(reversed(self.shape), reversed(self.strides)):
            if s != 1 and st != exp:
                return False
            exp *= s
        return True

    def with_(self, **kw) -> "TView":
        d = dict(storage=self.storage, offset=self.offset, shape=self.shape, strides=self.strides,
                 dtype=self.dtype)
        d.update(kw)
        return TView(**d)


@dataclass(frozen=True)
class Ref:
    """Byte address ``storage + byte_offset``, resolved to a pointer at launch-build time."""

    storage: str
    byte_offset: int = 0


@dataclass
class Storage:
    name: str
    kind: str            # "input" | "weight" | "arena"
    nbytes: int
    dtype: str = "uint8"
    offset: int = -1     # arena byte offset (arena kind only)
    first: int = -1      # first step index that writes it
    last: int = -1       # last step index that reads it
    zero_init: bool = False


@dataclass
class BufferAllocation:
    """One arena allocation (`cuda_compiler/cuda_program.py:15-22`) plus its arena offset."""

    name: str
    shape: list[int]
    dtype: str = "bfloat16"
    size_bytes: int = 0
    offset: int = 0


@dataclass
class LaunchStep:
    """One kernel launch. ``args`` maps argument-struct fields to values or ``Ref``s."""

    kind: str                    # step family, e.g. "gemm", "fused", "rmsnorm", "attention"
    kernel: str                  # kernel symbol
    module: str                  # code object name ("basic", "linear", ..., or a generated chain)
    arg_struct: str              # name of the argument struct in csrc/kernels/common.h
    args: dict
    grid: tuple[int, int, int]
    block: tuple[int, int, int] = (256, 1, 1)
    lds: int = 0
    inputs: list[str] = field(default_factory=list)    # IR tensors read (for ordering and tests)
    outputs: list[str] = field(default_factory=list)   # IR tensors written
    params: dict = field(default_factory=dict)          # descriptive parameters (M, N, K, rows, ...)


@dataclass
class KernelSource:
    """Generated HIP source compiled at program-load time (`cuda_program.py:25-29`)."""

    kernel_name: str
    source_code: str


@dataclass
class HIPProgram:
    steps: list[LaunchStep]
    buffer_allocations: list[BufferAllocation]
    input_specs: list[TensorSpec]
    output_specs: list[TensorSpec]
    weight_specs: list[TensorSpec]
    weight_name_mapping: dict[str, str]
    kernel_sources: list[KernelSource] = field(default_factory=list)
    compute_dtype: str = "bfloat16"
    storages: dict[str, Storage] = field(default_factory=dict)
    views: dict[str, TView] = field(default_factory=dict)
    output_views: dict[str, TView] = field(default_factory=dict)
    arena_bytes: int = 0
    stats: dict = field(default_factory=dict)

    @property
    def kernel_calls(self):
        return self.steps
