"""Compiled programs on disk: the ``.hipbin`` file and the program cache.

The reference serialises compiled programs as ``.npubin`` (JSON with a format tag
and a version, `npu_compiler/compiled_program.py:49-75`) and keeps NVRTC results in
a process-wide dictionary keyed by a source hash (`cuda_runtime/cuda_executor.py:38-51`).
Here:

* ``save_program`` / ``load_program`` write and read a ``HIPProgram`` as JSON
  (``"format": "hipbin"``, ``"version": 1``). Every value of the program is one of
  its own dataclasses (``LaunchStep``, ``TView``, ``Ref``, ``Storage``,
  ``BufferAllocation``, ``TensorSpec``, ``KernelSource``), a tuple, or plain JSON;
  dataclasses are written as ``{"__t": name, ...fields}``, tuples as
  ``{"__tuple": [...]}``, and only the listed classes can be rebuilt, so loading a
  file runs no code from it;
* ``compile_cached`` returns the program for an IR dict from ``cache_dir`` when a file
  for the same IR, the same compile options and the same compiler sources exists,
  and otherwise compiles and writes it. Generated elementwise kernels keep their
  own on-disk code-object cache (``hip_runtime.kernels``), so a cached program needs
  neither the lowering nor hiprtc.
"""

from __future__ import annotations

import dataclasses
import hashlib
import json
import os
import tempfile

from hip_compiler.program import BufferAllocation, HIPProgram, KernelSource, LaunchStep, Ref, Storage, TView
from npu_compiler.ir_reader import TensorSpec

FORMAT, VERSION = "hipbin", 1
_CLASSES = {c.__name__: c for c in (LaunchStep, TView, Ref, Storage, BufferAllocation, TensorSpec, KernelSource)}


def _enc(v):
    if dataclasses.is_dataclass(v) and not isinstance(v, type):
        name = type(v).__name__
        if name not in _CLASSES:
            raise TypeError(f"cannot serialise {name}")
        d = {"__t": name}
        for f in dataclasses.fields(v):
            d[f.name] = _enc(getattr(v, f.name))
        return d
    if isinstance(v, tuple):
        return {"__tuple": [_enc(x) for x in v]}
    if isinstance(v, list):
        return [_enc(x) for x in v]
    if isinstance(v, dict):
        if any(not isinstance(k, str) for k in v):
            raise TypeError("dict keys must be strings")
        return {k: _enc(x) for k, x in v.items()}
    if v is None or isinstance(v, (bool, int, float, str)):
        return v
    raise TypeError(f"cannot serialise {type(v).__name__}")


def _dec(v):
    if isinstance(v, list):
        return [_dec(x) for x in v]
    if isinstance(v, dict):
        if "__tuple" in v:
            return tuple(_dec(x) for x in v["__tuple"])
        if "__t" in v:
            cls = _CLASSES.get(v["__t"])
            if cls is None:
                raise ValueError(f"unknown record type {v['__t']!r}")
            return cls(**{k: _dec(x) for k, x in v.items() if k != "__t"})
        return {k: _dec(x) for k, x in v.items()}
    return v


def program_to_dict(prog: HIPProgram) -> dict:
    body = {f.name: _enc(getattr(prog, f.name)) for f in dataclasses.fields(prog)}
    return {"format": FORMAT, "version": VERSION, "program": body}


def program_from_dict(data: dict) -> HIPProgram:
    if data.get("format") != FORMAT or data.get("version") != VERSION:
        raise ValueError(f"not a {FORMAT} v{VERSION} file")
    body = data["program"]
    names = {f.name for f in dataclasses.fields(HIPProgram)}
    if set(body) != names:
        raise ValueError(f"program fields differ: {sorted(set(body) ^ names)}")
    return HIPProgram(**{k: _dec(v) for k, v in body.items()})


def save_program(prog: HIPProgram, path: str) -> None:
    """Write ``prog`` to ``path`` atomically (a temporary file renamed into place)."""
    d = os.path.dirname(os.path.abspath(path))
    os.makedirs(d, exist_ok=True)
    fd, tmp = tempfile.mkstemp(dir=d, suffix=".tmp")
    with os.fdopen(fd, "w") as f:
        json.dump(program_to_dict(prog), f, separators=(",", ":"))
    os.replace(tmp, path)


def load_program(path: str) -> HIPProgram:
    with open(path) as f:
        return program_from_dict(json.load(f))


def compiler_fingerprint() -> str:
    """Hash of every source the lowering depends on: the compiler itself, the IR reader and
    partitioner it imports (``npu_compiler``) and the kernel-argument layouts the launch records
    are packed against (``hip_runtime/kernels.py``). A cached program is reused only with the
    lowering that produced it."""
    h = hashlib.sha256()
    here = os.path.dirname(os.path.abspath(__file__))
    pkg = os.path.dirname(here)
    files = [os.path.join(here, n) for n in sorted(os.listdir(here)) if n.endswith(".py")]
    npu = os.path.join(pkg, "npu_compiler")
    files += [os.path.join(npu, n) for n in sorted(os.listdir(npu)) if n.endswith(".py")]
    files.append(os.path.join(pkg, "hip_runtime", "kernels.py"))
    for path in files:
        with open(path, "rb") as f:
            h.update(os.path.relpath(path, pkg).encode() + b"\0" + f.read())
    return h.hexdigest()


def lowering_settings(options: dict) -> dict:
    """The resolved values of every setting that changes the lowering besides the call's own
    options: environment switches read at compile time and module-level switches."""
    from hip_compiler import patterns, persistent, subgraph_analyzer

    fold = options.get("fold_attention")
    return {
        "fold_attention": (os.environ.get("HIPRT_FOLD_ATTN", "1") == "1") if fold is None else bool(fold),
        "conv_nhwc": os.environ.get("HIPRT_CONV_NHWC", "1") == "1",
        "conv_d2_max_k": subgraph_analyzer.CONV_D2_MAX_K,
        "conv_small_tile_max_k": subgraph_analyzer.CONV_SMALL_TILE_MAX_K,
        "conv_nfast": bool(subgraph_analyzer.CONV_NFAST),
        "conv_d1_max_k": subgraph_analyzer.CONV_D1_MAX_K,
        "fuse_reduce_norm": bool(patterns.FUSE_REDUCE_NORM),
        "persistent_decode": (os.environ.get("HIPRT_PERSISTENT", "1") == "1") if options.get("persistent") is None
        else bool(options["persistent"]),
        "decode_kv_major_min_s": int(persistent.KV_MAJOR_MIN_S),
        "decode_slot_combine": bool(persistent.SLOT_COMBINE),
        "skinny_min_m": int(subgraph_analyzer.SKINNY_MIN_M),
        "skinny_norm_max_k": int(subgraph_analyzer.SKINNY_NORM_MAX_K),
        "wide_max_m": int(subgraph_analyzer.WIDE_MAX_M),
        "wide_halves": bool(subgraph_analyzer.WIDE_HALVES),
    }


def cache_key(ir_dict: dict, options: dict) -> str:
    h = hashlib.sha256()
    h.update(json.dumps(ir_dict, sort_keys=True, separators=(",", ":")).encode())
    h.update(json.dumps(options, sort_keys=True).encode())
    h.update(json.dumps(lowering_settings(options), sort_keys=True).encode())
    h.update(compiler_fingerprint().encode())
    return h.hexdigest()[:32]


def default_cache_dir() -> str:
    return os.environ.get("HIPRT_PROGRAM_CACHE",
                          os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), ".pcache"))


def compile_cached(ir_dict: dict, cache_dir: str | None = None, **options) -> HIPProgram:
    """``compile_subgraph(ir_dict, **options)`` through the on-disk program cache."""
    from hip_compiler import compile_subgraph

    d = cache_dir or default_cache_dir()
    path = os.path.join(d, cache_key(ir_dict, options) + ".hipbin")
    if os.path.exists(path):
        try:
            return load_program(path)
        except (ValueError, TypeError, KeyError, json.JSONDecodeError):
            pass   # unreadable or from another format version: rebuild it
    prog = compile_subgraph(ir_dict, **options)
    save_program(prog, path)
    return prog
