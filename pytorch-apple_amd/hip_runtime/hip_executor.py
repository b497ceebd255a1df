"""HIP executor: runs a HIPProgram as one prebuilt launch list (or one HIP graph).

Counterpart of the reference's ``CUDAExecutor`` (`cuda_runtime/cuda_executor.py:54-176`).
Init-time work: load code objects (AOT ``.hsaco`` and hiprtc-compiled chains),
allocate the arena (zero-filled once), pack every step's argument struct with
concrete arena pointers, and record where external buffers (graph inputs and
weights) must be patched in. ``run()`` resolves the external pointers; when they
match a set seen before, the HIP graph captured for that set is relaunched as-is
(one host call per step, instead of the reference's one Python dispatch per IR
step); a new set re-packs the affected kernargs and captures one more graph. Up to
``MAX_GRAPHS`` graphs are kept, least recently used first out, so a loop whose
first step reads one buffer and whose later steps read another (a decode loop
feeding its own argmax back as ``input_ids``) captures twice in total, not twice
per run. A captured graph holds its own copy of the kernel arguments.

Returned outputs alias executor-owned storage and stay valid until the next
``run()``, as in the reference (`cuda_executor.py:153-176`); outputs that are
graph inputs updated in place (KV caches) are the input buffers themselves.
"""

from __future__ import annotations

import ctypes as C
import operator
import os
from collections import OrderedDict

import torch

from hip_compiler.program import ELEM_SIZE, HIPProgram, Ref
from hip_runtime import _shim
from hip_runtime.hip_backend import _TORCH_OF_IR, HIPBuffer
from hip_runtime.kernels import STRUCTS, ModuleCache

_MODULES: dict[int, ModuleCache] = {}
MAX_GRAPHS = 8
MAX_TABLES = 8   # pointer tables kept per executor without graphs (with graphs: all)


def _current_stream(device: torch.device) -> int:
    """torch's current stream on ``device`` as a raw handle (the cheap accessor when present)."""
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def module_cache(device_index: int) -> ModuleCache:
    mc = _MODULES.get(device_index)
    if mc is None:
        mc = _MODULES[device_index] = ModuleCache()
    return mc


def resident_workgroups(device_index: int, module: str, kernel: str, threads: int, lds: int = 0) -> int:
    """How many workgroups of ``kernel`` (``threads`` threads, ``lds`` bytes of dynamic LDS) the
    device holds at once: its CU count times the kernel's workgroups per CU."""
    lib = _shim.lib()
    with torch.cuda.device(device_index):
        mc = module_cache(device_index)
        mc.ensure_builtin(module)
        fn = mc.function(module, kernel)
        cus, per = C.c_int(), C.c_int()
        _shim.check(lib.hs_device_cus(C.byref(cus)), "device CU count")
        _shim.check(lib.hs_occupancy(fn, threads, lds, C.byref(per)), f"occupancy of {kernel}")
    return cus.value * per.value


class _HostFlags:
    """Host-visible 32-bit words that kernels set on failure (one per executor that needs one),
    carved out of pinned, coherent, device-mapped pages that are never freed."""
    PAGE = 4096

    def __init__(self):
        self._host = self._dev = 0
        self._next = self.PAGE

    def take(self) -> tuple[C.c_int, int]:
        """(host view of the word, its device address)."""
        if self._next + 4 > self.PAGE:
            h, d = C.c_void_p(), C.c_void_p()
            _shim.check(_shim.lib().hs_host_alloc_mapped(self.PAGE, C.byref(h), C.byref(d)), "host flag page")
            self._host, self._dev, self._next = h.value, d.value, 0
        off = self._next
        self._next += 4
        return C.c_int.from_address(self._host + off), self._dev + off


_HOST_FLAGS: dict[int, _HostFlags] = {}


class HIPExecutor:
    def __init__(self, program: HIPProgram, backend=None, use_graph: bool | None = None):
        self.program = program
        self.device = backend.device if backend is not None else torch.device("cuda", torch.cuda.current_device())
        if use_graph is None:
            # a graph pays for a launch list; around one launch (the persistent decode step) it only
            # adds to the gap between launches (0.680 -> 0.677 ms per decode step launched directly)
            use_graph = os.environ.get("HIPRT_NO_GRAPH", "0") != "1" and len(program.steps) > 1
        self.use_graph = use_graph
        mods = module_cache(self.device.index or 0)
        gen = {ks.kernel_name: ks.source_code for ks in program.kernel_sources}
        for st in program.steps:
            if st.module in gen:
                mods.ensure_generated(st.module, gen[st.module])
            else:
                mods.ensure_builtin(st.module)
        self.arena = torch.zeros(max(program.arena_bytes, 256), dtype=torch.uint8, device=self.device)
        base = self.arena.data_ptr()
        storages = program.storages
        self._ext_names: list[str] = sorted({r.storage for st in program.steps
                                             for r in list(_refs(st.args)) + list(_table_refs(st))
                                             if storages[r.storage].kind in ("input", "weight")})
        self._structs = []
        self._tables: list[tuple[object, str, list]] = []   # (struct, pointer field, entries)
        # table values -> [(device table, its pinned host copy)]; pointer set -> table values
        self._table_bufs: OrderedDict[tuple, list] = OrderedDict()
        self._tkey_of: OrderedDict[tuple, tuple] = OrderedDict()
        self._fixups: list[tuple[object, str, int, str, int]] = []   # (struct, field, index, storage, byte_off)
        n = len(program.steps)
        self._recs = (_shim.LaunchRec * max(n, 1))()
        for i, st in enumerate(program.steps):
            s = STRUCTS[st.arg_struct]()
            for k, v in st.args.items():
                if isinstance(v, (list, tuple)):
                    arr = getattr(s, k)
                    for j, x in enumerate(v):
                        self._set(s, k, j, x, arr, base, storages)
                else:
                    self._set(s, k, -1, v, None, base, storages)
            self._structs.append(s)
            if "table" in st.params:
                self._tables.append((s, st.params["table"]["field"], st.params["table"]["entries"]))
            r = self._recs[i]
            r.fn = mods.function(st.module, st.kernel)
            r.grid[:] = [int(g) for g in st.grid]
            r.block[:] = [int(b) for b in st.block]
            r.lds_bytes = int(st.lds)
            r.kernarg_size = C.sizeof(s)
            r.kernarg = C.addressof(s)
        self._n = n
        self._ext_key: tuple | None = None        # external pointers packed into the kernargs now
        # external storages bound to weights (checked once per weights dict) and to graph inputs
        # (checked once per set of buffer objects)
        self._w_names = [n for n in self._ext_names if storages[n].kind == "weight"]
        self._in_names = [n for n in self._ext_names if storages[n].kind != "weight"]
        self._w_names_set = frozenset(self._w_names)
        # each fixup's pointer as a position in the pointer set (weights, inputs): a launch with a
        # new set patches its kernargs without building a name -> pointer map
        pos = {n: (0, i) for i, n in enumerate(self._w_names)} | {n: (1, i) for i, n in enumerate(self._in_names)}
        self._fix_pos = [(s, field, idx, *pos[storage], off) for s, field, idx, storage, off in self._fixups]
        self._w_src, self._w_snap, self._w_key = None, (), ()
        self._last_bufs: tuple | None = None      # input buffer objects of the previous launch
        self._last_in_key: tuple = ()
        self._in_cache: OrderedDict[tuple, tuple] = OrderedDict()
        self._graphs: OrderedDict[tuple, int] = OrderedDict()   # (pointer set, advance) -> captured graph
        self._adv_ptr = 0                         # flag word of a decode advance folded into the launch
        self._adv_bufs: tuple = ()                # its (mask, position, cache position, mask bytes)
        self._adv_checked: tuple | None = None    # the (pointer set, advance) last checked
        self._capture_stream = None
        # a persistent step (PERSISTENT_KINDS): every workgroup must be resident at once, and its
        # timeout flag is mirrored into host memory, read on every launch without a synchronisation
        self._hflag = None
        for st, s in zip(program.steps, self._structs):
            if st.kind not in PERSISTENT_KINDS:
                continue
            need = int(st.grid[0])
            fit = resident_workgroups(self.device.index or 0, st.module, st.kernel, int(st.block[0]), int(st.lds))
            if fit < need:
                raise RuntimeError(f"persistent step {st.kernel} needs {need} workgroups resident at once; "
                                   f"this device holds {fit} (compile with persistent=False, or HIPRT_PERSISTENT=0)")
            flags = _HOST_FLAGS.setdefault(self.device.index or 0, _HostFlags())
            self._hflag, s.host_err = flags.take()
        self._out_cache: dict[str, HIPBuffer] = {}
        for spec in program.output_specs:
            v = program.output_views[spec.name]
            st = storages[v.storage]
            if st.kind in ("arena", "persistent"):
                off = st.offset + v.offset * ELEM_SIZE[v.dtype]
                t = self.arena[off:off + v.numel * ELEM_SIZE[v.dtype]].view(_TORCH_OF_IR[v.dtype]).view(v.shape)
                self._out_cache[spec.name] = HIPBuffer(t, tuple(spec.shape))

    # ------------------------------------------------------------------ kernarg packing

    def _set(self, s, field, idx, v, arr, base, storages) -> None:
        if isinstance(v, Ref):
            st = storages[v.storage]
            if st.kind in ("arena", "persistent"):
                val = base + st.offset + v.byte_offset
            else:
                self._fixups.append((s, field, idx, v.storage, v.byte_offset))
                val = 0
        elif v is None:
            val = 0
        else:
            val = v
        if idx < 0:
            setattr(s, field, val)
        else:
            arr[idx] = val

    def _patch(self, key: tuple) -> None:
        for s, field, idx, part, i, off in self._fix_pos:
            val = key[part][i] + off
            if idx < 0:
                setattr(s, field, val)
            else:
                getattr(s, field)[idx] = val
        if self._tables:
            self._fill_tables(key)

    def _fill_tables(self, key: tuple) -> None:
        """Pointer tables of the launches that read one (the persistent decode step's per-layer
        tensors): one device array per set of table values. A table holds weights and caches
        only, so calls that differ in other inputs (a decode loop's first token, then its own
        argmax) share one and switch between them with no upload. A new set is uploaded from
        pinned memory on the launch stream without waiting for the device; without graphs the
        least recently used set beyond MAX_TABLES is freed after a synchronisation (a launch in
        flight may still read it), and with graphs none is freed (a captured graph keeps reading
        the table it was captured with)."""
        tkey = self._tkey_of.get(key)
        if tkey is None:
            ptrs = self._ptrs_of(key)
            base = self.arena.data_ptr()
            storages = self.program.storages
            vals = []
            for _, _, entries in self._tables:
                row = []
                for r in entries:
                    if r is None:
                        row.append(0)
                    elif storages[r.storage].kind in ("arena", "persistent"):
                        row.append(base + storages[r.storage].offset + r.byte_offset)
                    else:
                        row.append(ptrs[r.storage] + r.byte_offset)
                vals.append(tuple(row))
            tkey = self._tkey_of[key] = tuple(vals)
            while len(self._tkey_of) > 4 * MAX_TABLES:
                self._tkey_of.popitem(last=False)
        else:
            self._tkey_of.move_to_end(key)
        bufs = self._table_bufs.get(tkey)
        if bufs is None:
            bufs = []
            for row in tkey:
                host = torch.tensor([v - (1 << 64) if v >= (1 << 63) else v for v in row], dtype=torch.int64)
                host = host.pin_memory()
                bufs.append((host.to(self.device, non_blocking=True), host))
            self._table_bufs[tkey] = bufs
            if not self.use_graph and len(self._table_bufs) > MAX_TABLES:
                torch.cuda.current_stream(self.device).synchronize()
                self._table_bufs.popitem(last=False)
        else:
            self._table_bufs.move_to_end(tkey)
        for (s, field, _), (t, _) in zip(self._tables, bufs):
            setattr(s, field, t.data_ptr())

    # ------------------------------------------------------------------ execution

    def _check(self, name: str, buf) -> int:
        """The device pointer of ``buf`` after checking that it can back storage ``name``."""
        if buf is None:
            raise KeyError(f"HIPExecutor: no buffer for '{name}' (graph input or weight)")
        t = buf.native_handle if isinstance(buf, HIPBuffer) else buf
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise TypeError(f"HIPExecutor: '{name}' must be a device buffer, got {type(buf).__name__}")
        spec_st = self.program.storages[name]
        if t.numel() * t.element_size() < spec_st.nbytes:
            raise ValueError(f"HIPExecutor: '{name}' holds {t.numel() * t.element_size()} bytes, "
                             f"program needs {spec_st.nbytes}")
        return t.data_ptr()

    def _lookup(self, name: str, inputs: dict, weights: dict):
        buf = inputs.get(name)
        if buf is None:
            buf = weights.get(name)
        if buf is None and name in self.program.weight_name_mapping:
            buf = weights.get(self.program.weight_name_mapping[name])
        return buf

    def _pointer_key(self, inputs: dict, weights: dict) -> tuple:
        """The external pointer set of this call, as (weight pointers, input pointers).

        Weights are checked once per set of weight buffer objects (the DAGExecutor hands the same
        dict of the same buffers to every call; a new dict, or a dict whose entries were replaced,
        is checked again: an identity pass over its values, ≈ 10 µs). Inputs are checked once per
        set of buffer objects (a ``HIPBuffer`` never rebinds its tensor, so the same objects mean
        the same pointers); the last few sets are remembered, so a loop that alternates between two
        sets (the prompt's token buffer, then the previous step's argmax) checks each once."""
        snap = self._w_snap
        if (weights is not self._w_src or len(weights) != len(snap) or self._w_names_set & inputs.keys()
                or not all(map(operator.is_, weights.values(), snap))):
            self._w_src, self._w_snap = None, ()
            wk = tuple(self._check(n, self._lookup(n, inputs, weights)) for n in self._w_names)
            if not (self._w_names_set & inputs.keys()):   # an input shadowing a weight is not cached
                self._w_src, self._w_snap, self._w_key = weights, tuple(weights.values()), wk
        else:
            wk = self._w_key
        bufs = tuple(self._lookup(n, inputs, weights) for n in self._in_names)
        last = self._last_bufs
        if last is not None and all(b is c for b, c in zip(bufs, last)):
            return (wk, self._last_in_key)
        ids = tuple(map(id, bufs))
        hit = self._in_cache.get(ids)
        if hit is not None and all(b is c for b, c in zip(bufs, hit[0])):
            self._in_cache.move_to_end(ids)
            ik = hit[1]
        else:
            ik = tuple(self._check(n, b) for n, b in zip(self._in_names, bufs))
            if all(isinstance(b, HIPBuffer) for b in bufs):
                self._in_cache[ids] = (bufs, ik)
                while len(self._in_cache) > MAX_GRAPHS:
                    self._in_cache.popitem(last=False)
        if all(isinstance(b, HIPBuffer) for b in bufs):
            self._last_bufs, self._last_in_key = bufs, ik
        else:
            self._last_bufs = None
        return (wk, ik)

    def _ptrs_of(self, key: tuple) -> dict[str, int]:
        return dict(zip(self._w_names, key[0])) | dict(zip(self._in_names, key[1]))

    def launch(self, inputs: dict, weights: dict, stream: int | None = None) -> None:
        """Enqueue the whole program on ``stream`` (default: torch's current stream). Raises
        ``RuntimeError`` first when an earlier persistent step of this executor reported a
        timeout (its host-visible flag; no synchronisation needed)."""
        if self._hflag is not None and self._hflag.value:
            self._hflag.value = 0
            raise RuntimeError(_TIMEOUT_MSG)
        key = self._pointer_key(inputs, weights)
        if stream is None:
            stream = _current_stream(self.device)
        if self._n == 0:
            return
        lib = _shim.lib()
        gkey = (key, self._adv_ptr)
        graph = self._graphs.get(gkey) if self.use_graph else None
        if graph is not None:
            self._graphs.move_to_end(gkey)
        else:
            if key != self._ext_key:
                self._patch(key)
                self._ext_key = key
            if self._adv_ptr and self._adv_checked != (key, self._adv_bufs):   # once per pointer set
                self._check_advance(key, self._adv_bufs)
                self._adv_checked = (key, self._adv_bufs)
            if not self.use_graph:
                _shim.check(lib.hs_replay(self._recs, self._n, stream), "replay")
                return
            if self._capture_stream is None:
                cs = C.c_void_p()
                _shim.check(lib.hs_stream_create(C.byref(cs)), "stream create")
                self._capture_stream = cs.value
            g = C.c_void_p()
            _shim.check(lib.hs_graph_capture(self._recs, self._n, self._capture_stream, C.byref(g)), "graph capture")
            graph = self._graphs[gkey] = g.value
            while len(self._graphs) > MAX_GRAPHS:
                _, old = self._graphs.popitem(last=False)
                _shim.check(lib.hs_graph_destroy(old), "graph destroy")
        _shim.check(lib.hs_graph_launch(graph, stream), "graph launch")

    def _check_advance(self, key: tuple, bufs: tuple) -> None:
        """A folded advance moves the buffers this launch reads as its mask and positions, with the
        mask's element size: anything else would move other buffers, or write 2-byte zeros into
        a 4-byte mask."""
        args = self.program.steps[0].args
        ptrs = self._ptrs_of(key)
        mask, pos, cpos, mbytes = bufs
        want = {"mask": mask, "pos_ids": pos, "cache_pos": cpos}
        for field, ptr in want.items():
            ref = args[field]
            got = None if ref is None else ptrs.get(ref.storage, -1) + ref.byte_offset
            if got != ptr:
                raise ValueError(f"the folded decode advance moves another buffer than the step's {field}")
        if mbytes != {0: 4, 2: 2}.get(int(args["mask_dtype"]), -1):
            raise ValueError("the folded decode advance's mask element size differs from the step's mask")

    def fold_advance(self, advance: "DecodeAdvance | None") -> bool:
        """Fold ``advance`` into this program's launch: a persistent decode step then moves its
        loop's position inputs to the next step itself, after its argmax (no second launch, and
        also after a loop's last step). The step launched after the inputs have moved past the
        cache end sets ``advance``'s flag (``advance.check()`` raises) instead of re-running the
        last position. Returns False and changes nothing when the program is not a single
        persistent decode step (call ``advance()`` after each step then). ``None`` unfolds."""
        if len(self.program.steps) != 1 or self.program.steps[0].kind != "decode_step":
            return False
        s = self._structs[0]
        if advance is None:
            s.adv_mask = s.adv_pos = s.adv_cpos = s.adv_flag = None
            s.adv_mask_bytes = 0
            self._adv_ptr = 0
        else:
            a = advance._args
            if int(a.S) != int(self.program.steps[0].args["S"]):
                raise ValueError("the advance's mask length differs from the step's cache length")
            bufs = (int(a.mask), int(a.pos), int(a.cpos), int(a.mask_bytes))   # checked at launch
            s.adv_mask, s.adv_pos, s.adv_cpos, s.adv_flag = a.mask, a.pos, a.cpos, a.overflow
            s.adv_mask_bytes = a.mask_bytes
            self._adv_ptr = int(a.overflow)
            self._adv_bufs = bufs
        return True

    def check(self) -> None:
        """Raise ``RuntimeError`` if a persistent step has recorded a timeout (one of its
        workgroups waited past its time limit for data from another: its results are not valid).
        Synchronises with the device; clears the flags."""
        for st in self.program.steps:
            if st.kind not in PERSISTENT_KINDS:
                continue
            xs = self.program.storages[st.args["ll"].storage]
            off = xs.offset + (int(st.params["exchange_words"]) - 1) * 4
            flag = self.arena[off:off + 4].view(torch.int32)
            dev = int(flag.item())
            host = self._hflag is not None and self._hflag.value
            if dev or host:
                flag.zero_()
                if self._hflag is not None:
                    self._hflag.value = 0
                raise RuntimeError(_TIMEOUT_MSG)

    def run(self, inputs: dict, weights: dict) -> dict[str, HIPBuffer]:
        self.launch(inputs, weights)
        out: dict[str, HIPBuffer] = {}
        for spec in self.program.output_specs:
            b = self._out_cache.get(spec.name)
            if b is None:
                v = self.program.output_views[spec.name]
                src = inputs.get(v.storage)
                if isinstance(src, HIPBuffer) and tuple(src.shape) == tuple(spec.shape):
                    b = src
                else:
                    t = src.native_handle if isinstance(src, HIPBuffer) else src
                    b = HIPBuffer(t.reshape(-1)[:v.numel].view(tuple(spec.shape)), tuple(spec.shape))
            out[spec.name] = b
        return out

    def __del__(self):
        try:
            lib = _shim.lib()
            for g in self._graphs.values():
                lib.hs_graph_destroy(g)
            self._graphs.clear()
            if self._capture_stream is not None:
                lib.hs_stream_destroy(self._capture_stream)
        except Exception:
            pass


# launches whose workgroups wait for each other's data (all resident at once, bounded waits with
# a timeout flag in the last exchange word): the persistent decode step and the one-launch
# attention block
PERSISTENT_KINDS = ("decode_step", "attn_step")

_TIMEOUT_MSG = ("persistent step: a workgroup timed out waiting for another's data, so the step's "
                "outputs are not valid (the step needs every one of its workgroups resident at once: "
                "is another kernel sharing the GPU?)")


def _table_refs(step):
    return [r for r in step.params.get("table", {}).get("entries", []) if isinstance(r, Ref)]


def _refs(args: dict):
    for v in args.values():
        if isinstance(v, Ref):
            yield v
        elif isinstance(v, (list, tuple)):
            for x in v:
                if isinstance(x, Ref):
                    yield x


class DecodeAdvance:
    """Advances a decode loop's ``attention_mask`` / ``position_ids`` / ``cache_position``
    buffers to the next step on the device (``k_decode_advance``), ordered after the step on
    the same stream: the loop needs no host-side input preparation between steps.

    A call that would move past the cache end (position S) writes nothing and raises a flag on
    the device instead; ``check()`` (a synchronising read) raises ``RuntimeError`` once it is
    set, so a loop that ran too long is reported instead of re-running position S - 1."""

    def __init__(self, mask: HIPBuffer, pos: HIPBuffer, cpos: HIPBuffer):
        m, p, c = mask.native_handle, pos.native_handle, cpos.native_handle
        if m.element_size() not in (2, 4) or p.dtype != torch.int64 or c.dtype != torch.int64:
            raise TypeError("DecodeAdvance needs a 16- or 32-bit mask and int64 positions")
        self.device = m.device
        mods = module_cache(self.device.index or 0)
        mods.ensure_builtin("basic")
        self._fn = mods.function("basic", "k_decode_advance")
        self._flag = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.S = int(mask.shape[-1])
        self._args = STRUCTS["AdvanceArgs"](mask=m.data_ptr(), pos=p.data_ptr(), cpos=c.data_ptr(),
                                            overflow=self._flag.data_ptr(), S=self.S,
                                            mask_bytes=m.element_size(), pad=0)
        self._keep = (m, p, c)

    def __call__(self, stream: int | None = None) -> None:
        s = stream if stream is not None else _current_stream(self.device)
        _shim.check(_shim.lib().hs_launch(self._fn, 1, 1, 1, 64, 1, 1, 0, s, C.byref(self._args),
                                          C.sizeof(self._args)), "k_decode_advance")

    def check(self) -> None:
        """Raise if any call since construction (or ``clear()``) tried to step past the cache end."""
        if int(self._flag.item()):
            raise RuntimeError(f"decode loop stepped past the end of the {self.S}-position cache "
                               "(k_decode_advance left the inputs at the last position)")

    def clear(self) -> None:
        self._flag.zero_()
