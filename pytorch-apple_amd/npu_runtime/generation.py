"""Prefill → decode greedy generation over static KV caches.

Restates the reference's generation loop (`examples/run_qwen.py:84-200`):

* the prompt is padded to the prefill graph's length T under a causal mask
  (`:90-99`), so no real row sees a padding column;
* the first token is the argmax of the prefill logits at the last real position
  (`:121-125`);
* each decode step feeds the previous token at position ``prompt_len + step``, with
  the mask open on ``0 .. pos`` and ``position_ids = cache_position = pos``
  (`:151-166`), stops at EOS without emitting it (`:182-183`), and hands its updated
  caches to the next step (`:188-190`); the prefill's caches reach the first step
  through the KV mapping record (`:132-146`, `examples/extract_qwen_ir.py:145-173`).

What differs:

* both graphs run over the same static caches ``[1, KVH, S, D]``: the prefill writes
  the prompt's keys and values straight into them (the ``index_copy`` lowering
  updates a cache input in place), so the reference's host-side pad and upload of
  every cache after the prefill (`run_qwen.py:132-146`) does not exist here;
* when a graph has an argmax output (``aten.argmax`` of the logits, int64), the
  token stays on the device and is fed back as the next ``input_ids``; on a backend
  whose buffers are torch tensors, the mask and positions are advanced in place on
  the device (one ``decode_advance`` launch per step when the backend offers one), so a
  decode step needs no host round trip unless ``eos_token_id`` is given (then each token
  is read back to test it, as the reference does);
* on such a backend the caches and the per-step inputs are allocated once per
  generator and rewritten in place by each call (caches zeroed), so every call
  hands the executors the same buffers and their captured HIP graphs are reused;
* closed entries are ``-inf`` and padding rows stay causal (open on ``0 .. i``),
  where the reference closes them completely with fp16 -65504: every row keeps an
  open entry, so no softmax is taken over a fully closed row (NaN with ``-inf``), and
  the attention kernels skip every closed block exactly (a 128-token prefill over a
  2048-position cache reads the first 128 positions, not 2048). Padding rows only
  produce logits nobody reads and cache rows that decode steps overwrite before
  opening them.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np
import torch

FIXED_INPUTS = ("input_ids", "attention_mask", "position_ids", "cache_position")
_TORCH = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _host(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    return t.view(torch.uint16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def prefill_mask(T: int, S: int, prompt_len: int, dtype: str = "bfloat16") -> np.ndarray:
    """[1, 1, T, S]: row i open on 0..i, ``-inf`` elsewhere. A real row (i < prompt_len)
    therefore sees no padding column; padding rows stay causal (see the module docstring)."""
    if not 0 < prompt_len <= T <= S:
        raise ValueError("need 0 < prompt_len <= T <= S")
    i = torch.arange(T).unsqueeze(1)
    j = torch.arange(S).unsqueeze(0)
    m = torch.where(j <= i, 0.0, float("-inf"))
    return _host(m.to(_TORCH[dtype]).reshape(1, 1, T, S))


def decode_mask(S: int, pos: int, dtype: str = "bfloat16") -> np.ndarray:
    """[1, 1, 1, S]: open on 0..pos, ``-inf`` after."""
    m = torch.full((1, 1, 1, S), float("-inf"), dtype=torch.float32)
    m[..., :pos + 1] = 0.0
    return _host(m.to(_TORCH[dtype]))


def _token_output(ir: dict) -> str | None:
    """Name of the graph's argmax-of-logits output, if it has one."""
    producers = {o["name"]: n for n in ir["nodes"] for o in n["outputs"]}
    for o in ir["graph_outputs"]:
        n = producers.get(o["name"])
        if n is not None and n["op_type"] == "aten.argmax.default" and o["dtype"] == "int64":
            return o["name"]
    return None


def _spec(ir: dict, name: str) -> dict:
    return next(s for s in ir["graph_inputs"] if s["name"] == name)


@dataclass
class GenerationResult:
    tokens: list[int]
    prompt_len: int
    ttft_s: float       # prefill through the first token on the host
    decode_s: float     # the decode steps, synchronised at the end

    @property
    def decode_tok_s(self) -> float:
        n = len(self.tokens) - 1
        return n / self.decode_s if n > 0 and self.decode_s > 0 else 0.0


class GreedyGenerator:
    """Greedy generation with a prefill graph and a decode graph, each run by a
    ``DAGExecutor`` (any backend, or the all-CPU plan with ``backend=None``)."""

    def __init__(self, prefill, decode, kv_map: dict, prefill_ir: dict, decode_ir: dict, backend=None):
        self.prefill, self.decode, self.kv_map, self.backend = prefill, decode, kv_map, backend
        self.T = _spec(prefill_ir, "attention_mask")["shape"][-2]
        self.S = int(kv_map["max_cache_len"])
        self.mask_dtype = _spec(decode_ir, "attention_mask")["dtype"]
        self.logits_p = prefill_ir["graph_outputs"][0]["name"]
        self.logits_d = decode_ir["graph_outputs"][0]["name"]
        self.tok_p = _token_output(prefill_ir)
        self.tok_d = _token_output(decode_ir)
        self.cache_specs = [s for s in decode_ir["graph_inputs"] if s["name"] not in FIXED_INPUTS]
        p_caches = [s["name"] for s in prefill_ir["graph_inputs"] if s["name"] not in FIXED_INPUTS]
        if len(p_caches) != len(self.cache_specs):
            raise ValueError("prefill and decode graphs carry different numbers of caches")
        # prefill cache input that feeds each decode cache input (both graphs list them per layer, k then v)
        self.p_cache_of = {d["name"]: p for d, p in zip(self.cache_specs, p_caches)}
        if any(_spec(prefill_ir, p)["shape"][-2] != self.S for p in p_caches):
            raise ValueError("prefill caches must be the decode graph's static caches")
        self._bufs: dict | None = None

    # -- buffers ---------------------------------------------------------------------------

    def _on_device(self) -> bool:
        return self.backend is not None

    def _zeros(self, spec: dict):
        if self._on_device():
            return self.backend.allocate_buffer(torch.zeros(spec["shape"], dtype=_TORCH[spec["dtype"]]))
        return _host(torch.zeros(spec["shape"], dtype=_TORCH[spec["dtype"]]))

    def _put(self, arr: np.ndarray):
        return self.backend.allocate_buffer(arr) if self._on_device() else arr

    def _device_buffers(self) -> dict:
        """Caches and step inputs, allocated on the first call and reused by every later one."""
        if self._bufs is None:
            T, S, dt = self.T, self.S, self.mask_dtype
            b = {d["name"]: self._zeros(d) for d in self.cache_specs}
            b.update(p_ids=self._put(np.zeros((1, T), np.int64)), p_mask=self._put(prefill_mask(T, S, T, dt)),
                     p_pos=self._put(np.zeros((1, T), np.int64)), p_cpos=self._put(np.zeros(T, np.int64)),
                     d_ids=self._put(np.zeros((1, 1), np.int64)), d_mask=self._put(decode_mask(S, 0, dt)),
                     d_pos=self._put(np.zeros((1, 1), np.int64)), d_cpos=self._put(np.zeros(1, np.int64)))
            self._bufs = b
        return self._bufs

    def _token_host(self, val, index: int) -> int:
        if hasattr(val, "to_numpy"):
            val = val.to_numpy()
        return int(np.asarray(val).reshape(-1)[index])

    def _argmax_host(self, logits, row: int) -> int:
        arr = logits.to_numpy() if hasattr(logits, "to_numpy") else np.asarray(logits)
        t = torch.from_numpy(np.ascontiguousarray(arr))
        if t.dtype == torch.int16 or t.dtype == torch.uint16:
            t = t.view(torch.bfloat16)
        t = t.float().reshape(-1, t.shape[-1])
        return int(torch.argmax(t[row]).item())

    # -- generation ------------------------------------------------------------------------

    def generate(self, prompt_ids, max_tokens: int, eos_token_id: int | None = None) -> GenerationResult:
        n = len(prompt_ids)
        if not 0 < n <= self.T:
            raise ValueError(f"prompt length {n} must be in 1..{self.T}")
        if max_tokens < 1 or n + max_tokens - 1 > self.S:
            raise ValueError(f"{n} prompt tokens + {max_tokens - 1} decode steps exceed the cache ({self.S})")
        T, S, dt = self.T, self.S, self.mask_dtype
        ids = np.zeros((1, T), np.int64)
        ids[0, :n] = np.asarray(prompt_ids, np.int64)
        ar = np.arange(T, dtype=np.int64)
        dev = self._on_device()
        if dev:
            b = self._device_buffers()
            for d in self.cache_specs:
                b[d["name"]].native_handle.zero_()
            for key, arr in (("p_ids", ids), ("p_mask", prefill_mask(T, S, n, dt)), ("p_pos", ar.reshape(1, -1)),
                             ("p_cpos", ar), ("d_mask", decode_mask(S, n, dt)), ("d_pos", np.array([[n]], np.int64)),
                             ("d_cpos", np.array([n], np.int64))):
                b[key].write_from_numpy(arr)
            pin = {"input_ids": b["p_ids"], "attention_mask": b["p_mask"], "position_ids": b["p_pos"],
                   "cache_position": b["p_cpos"]}
            caches = {d["name"]: b[d["name"]] for d in self.cache_specs}
        else:
            pin = {"input_ids": ids, "attention_mask": prefill_mask(T, S, n, dt), "position_ids": ar.reshape(1, -1),
                   "cache_position": ar}
            caches = {d["name"]: self._zeros(d) for d in self.cache_specs}
        for d, buf in caches.items():
            pin[self.p_cache_of[d]] = buf

        t0 = time.perf_counter()
        out = self.prefill.execute(pin)
        if self.tok_p is not None:
            first = self._token_host(out[self.tok_p], n - 1)
        else:
            first = self._argmax_host(out[self.logits_p], n - 1)
        ttft = time.perf_counter() - t0
        tokens = [first]
        kv = {}
        for layer in self.kv_map["layers"]:
            kv[layer["decode_key_input"]] = out[layer["prefill_key_output"]]
            kv[layer["decode_value_input"]] = out[layer["prefill_value_output"]]
        if max_tokens == 1 or (eos_token_id is not None and first == eos_token_id):
            return GenerationResult(tokens if first != eos_token_id else [], n, ttft, 0.0)

        fast = dev and self.tok_d is not None
        t1 = time.perf_counter()
        if fast:
            mask_t, pos_t, cpos_t = (b[k].native_handle for k in ("d_mask", "d_pos", "d_cpos"))
            if "advance" not in b:   # one device launch per step when the backend has one
                make = getattr(self.backend, "decode_advance", None)
                b["advance"] = make(b["d_mask"], b["d_pos"], b["d_cpos"]) if make is not None else None
            b["d_ids"].native_handle.fill_(first)
            hist = torch.zeros(max_tokens - 1, dtype=torch.int64, device=pos_t.device)
            cur = b["d_ids"]
            # a decode program that is one persistent step moves its own inputs after each step (one
            # launch per step); folded for this loop only, so other runs of the program see no advance
            folded = [ex for ex in getattr(self.decode, "npu_executors", {}).values()
                      if b["advance"] is not None and getattr(ex, "fold_advance", None) is not None
                      and ex.fold_advance(b["advance"])]
        else:
            cur = np.array([[first]], np.int64)
        steps = 0
        for step in range(max_tokens - 1):
            pos = n + step
            if fast:
                if step and folded:
                    pass   # the previous step moved the inputs itself
                elif step and b["advance"] is not None:
                    b["advance"]()
                elif step:
                    mask_t[..., pos] = 0.0
                    pos_t.fill_(pos)
                    cpos_t.fill_(pos)
                din = {"input_ids": cur, "attention_mask": b["d_mask"], "position_ids": b["d_pos"],
                       "cache_position": b["d_cpos"]}
            else:
                din = {"input_ids": self._put(cur), "attention_mask": self._put(decode_mask(S, pos, dt)),
                       "position_ids": self._put(np.array([[pos]], np.int64)),
                       "cache_position": self._put(np.array([pos], np.int64))}
            din.update(kv)
            out = self.decode.execute(din)
            steps += 1
            if fast:
                cur = out[self.tok_d]
                hist[step].copy_(cur.native_handle.reshape(-1)[0])
                if eos_token_id is not None and int(hist[step].item()) == eos_token_id:
                    break
            else:
                tok = (self._token_host(out[self.tok_d], 0) if self.tok_d is not None
                       else self._argmax_host(out[self.logits_d], 0))
                if eos_token_id is not None and tok == eos_token_id:
                    break
                tokens.append(tok)
                cur = np.array([[tok]], np.int64)
            for layer in self.kv_map["layers"]:
                kv[layer["decode_key_input"]] = out[layer["decode_key_output"]]
                kv[layer["decode_value_input"]] = out[layer["decode_value_output"]]
        if fast:
            for ex in folded:
                ex.fold_advance(None)
            self.backend.synchronize()
            if b.get("advance") is not None:
                b["advance"].check()
        # a persistent decode step that timed out waiting for data (not all of its workgroups
        # resident) produced invalid tokens: raise rather than return them
        for dag in (self.prefill, self.decode):
            for ex in getattr(dag, "npu_executors", {}).values():
                check = getattr(ex, "check", None)
                if check is not None:
                    check()
        if fast:
            got = hist[:steps].cpu().tolist()
            if eos_token_id is not None and eos_token_id in got:
                got = got[:got.index(eos_token_id)]
            tokens += got
        decode_s = time.perf_counter() - t1
        return GenerationResult(tokens, n, ttft, decode_s)
