"""Arena planner: liveness-based offsets for every intermediate storage.

The reference records one ``BufferAllocation`` per produced tensor and allocates
each separately at executor init (`cuda_compiler/buffer_planner.py:25-77`,
`cuda_runtime/cuda_executor.py:89-95`), allocating alias outputs too and
flattening fused outputs (D11). Here aliases own no storage at all, and every
real intermediate gets an offset in one device arena: storages whose live ranges
(first writing step .. last reading step) overlap never share bytes, graph
outputs are live for the whole program (no other storage ever shares their bytes,
so an output can be fed back as the next run's input), and "persistent" storages (tickets
of the split attention, which must read zero at every launch) are never shared.
"""

from __future__ import annotations

from hip_compiler.program import BufferAllocation, LaunchStep, Ref, Storage

ALIGN = 256


def _refs(step: LaunchStep):
    for v in step.args.values():
        if isinstance(v, Ref):
            yield v
        elif isinstance(v, (list, tuple)):
            for x in v:
                if isinstance(x, Ref):
                    yield x


def plan_arena(steps: list[LaunchStep], storages: dict[str, Storage], live_to_end: set[str]) -> int:
    """Assign ``Storage.offset`` for arena/persistent storages; returns the arena size in bytes."""
    for i, st in enumerate(steps):
        for r in _refs(st):
            s = storages[r.storage]
            if s.first < 0:
                s.first = i
            s.last = i
    end = len(steps)
    # graph outputs hold their bytes for the whole program: a caller may feed an output back as
    # the next run's input (the greedy loop's next token, KV caches), and no step of that run may
    # write those bytes before its last read of the input
    for name in live_to_end:
        if name in storages and storages[name].first >= 0:
            storages[name].first = 0
            storages[name].last = end
    off = 0
    for s in storages.values():
        if s.kind == "persistent" and s.first >= 0:
            s.offset = off
            off += (s.nbytes + ALIGN - 1) // ALIGN * ALIGN
    base = off
    arena = sorted((s for s in storages.values() if s.kind == "arena" and s.first >= 0),
                   key=lambda s: (-s.nbytes, s.first))
    placed: list[Storage] = []
    top = base
    for s in arena:
        size = (s.nbytes + ALIGN - 1) // ALIGN * ALIGN
        busy = sorted((p.offset, p.offset + (p.nbytes + ALIGN - 1) // ALIGN * ALIGN) for p in placed
                      if not (p.last < s.first or s.last < p.first))
        cand = base
        for lo, hi in busy:
            if cand + size <= lo:
                break
            cand = max(cand, hi)
        s.offset = cand
        placed.append(s)
        top = max(top, cand + size)
    return top


def buffer_allocations(storages: dict[str, Storage], views_by_storage: dict[str, tuple]) -> list[BufferAllocation]:
    out = []
    for s in storages.values():
        if s.kind in ("arena", "persistent") and s.offset >= 0:
            shape, dtype = views_by_storage.get(s.name, ([s.nbytes], "uint8"))
            out.append(BufferAllocation(name=s.name, shape=list(shape), dtype=dtype, size_bytes=s.nbytes,
                                        offset=s.offset))
    return out
