"""Export HF ``Qwen2ForCausalLM`` graphs over static KV caches, and the KV mapping.

Restates the reference's extraction wrappers (`examples/extract_qwen_ir.py:68-131`)
on this image's transformers (5.x), where ``Cache.update`` no longer receives
``cache_kwargs``:

* ``IndexCopyCache`` — the reference's ``_IndexCopyCache``: per layer, the new
  keys / values are written with an out-of-place ``index_copy(dim 2,
  cache_position)`` into the full static buffer and the whole buffer is returned,
  so attention always runs over ``max_cache_len`` positions and the graph has
  fixed shapes;
* ``QwenStaticWrapper`` — forward(input_ids, attention_mask, position_ids,
  cache_position, *past_kv_flat) → (logits, k_0, v_0, …[, next_token]). The
  reference uses it for decode (`:99-126`); here the same wrapper also exports the
  prefill (T tokens into the static cache, mask [1, 1, T, S]), which writes the
  prompt's KV straight into the caches the decode graph reads, instead of the
  reference's dynamic-cache prefill followed by a host-side pad into the static
  cache (`examples/run_qwen.py:132-146`);
* ``kv_mapping`` — the reference's ``qwen2_kv_mapping.json`` record
  (`examples/extract_qwen_ir.py:145-173`): per layer, which prefill output feeds
  which decode input and which decode output is the updated cache.

Input names follow the reference's decode graph (`extract_qwen_ir.py:255-267`):
``input_ids``, ``attention_mask``, ``position_ids``, ``cache_position``, then
``past_key_{i}`` / ``past_value_{i}``.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from irgen.exporter import extract_ir

FIXED_INPUTS = ("input_ids", "attention_mask", "position_ids", "cache_position")


class IndexCopyCache:
    """Static KV cache updated by out-of-place ``index_copy`` (see module docstring)."""

    is_compileable = False

    def __init__(self, kv_flat, num_layers: int, cache_position: torch.Tensor):
        self.key_cache = [kv_flat[2 * i] for i in range(num_layers)]
        self.value_cache = [kv_flat[2 * i + 1] for i in range(num_layers)]
        self.cache_position = cache_position

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        pos = self.cache_position
        if cache_kwargs and cache_kwargs.get("cache_position") is not None:
            pos = cache_kwargs["cache_position"]
        self.key_cache[layer_idx] = self.key_cache[layer_idx].index_copy(2, pos, key_states)
        self.value_cache[layer_idx] = self.value_cache[layer_idx].index_copy(2, pos, value_states)
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.key_cache[0].shape[-2]

    def get_mask_sizes(self, cache_position, layer_idx: int = 0):
        return self.key_cache[0].shape[-2], 0

    def __len__(self) -> int:
        return len(self.key_cache)


class QwenStaticWrapper(nn.Module):
    """(input_ids, attention_mask, position_ids, cache_position, *kv) → (logits, *kv'[, next_token])."""

    def __init__(self, model: nn.Module, num_layers: int, argmax: bool = False):
        super().__init__()
        self.model = model
        self.num_layers = num_layers
        self.argmax = argmax

    def forward(self, input_ids, attention_mask, position_ids, cache_position, *past_kv_flat):
        cache = IndexCopyCache(past_kv_flat, self.num_layers, cache_position)
        out = self.model(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                         cache_position=cache_position, past_key_values=cache, use_cache=True)
        res = [out.logits]
        for i in range(self.num_layers):
            res += [cache.key_cache[i], cache.value_cache[i]]
        if self.argmax:
            res.append(torch.argmax(out.logits, dim=-1))
        return tuple(res)


def to_dtype_keep_rotary(model: nn.Module, dtype: torch.dtype = torch.bfloat16) -> nn.Module:
    """Cast parameters and buffers to ``dtype`` except the rotary ``inv_freq`` buffers,
    which stay fp32 as in a model loaded with ``from_pretrained(..., dtype=dtype)``
    (HF builds them with an explicit ``.float()``)."""
    keep = {name: b.detach().clone() for name, b in model.named_buffers() if name.endswith("inv_freq")}
    model.to(dtype)
    for name, b in keep.items():
        mod_name, _, attr = name.rpartition(".")
        mod = model.get_submodule(mod_name) if mod_name else model
        setattr(mod, attr, b.float())
    return model


def static_inputs(config, tokens: int, max_cache_len: int, start: int = 0, device: str = "meta",
                  dtype: torch.dtype = torch.bfloat16) -> tuple:
    """Example inputs of the static-cache graph: ``tokens`` ids at positions
    ``start .. start+tokens-1`` over caches of ``max_cache_len``."""
    L = config.num_hidden_layers
    kvh = config.num_key_value_heads
    hd = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
    pos = torch.arange(start, start + tokens, device=device)
    kv = [torch.zeros(1, kvh, max_cache_len, hd, dtype=dtype, device=device) for _ in range(2 * L)]
    return (torch.zeros(1, tokens, dtype=torch.int64, device=device),
            torch.zeros(1, 1, tokens, max_cache_len, dtype=dtype, device=device),
            pos.unsqueeze(0), pos, *kv)


def input_names(num_layers: int) -> list[str]:
    names = list(FIXED_INPUTS)
    for i in range(num_layers):
        names += [f"past_key_{i}", f"past_value_{i}"]
    return names


def export_qwen(model: nn.Module, max_cache_len: int, tokens: int = 1, argmax: bool = False,
                model_name: str | None = None) -> dict:
    """IR of ``model`` (an HF Qwen2ForCausalLM with eager attention) for ``tokens`` query
    tokens over static caches of ``max_cache_len``; weights keyed by HF state-dict names."""
    cfg = model.config
    L = cfg.num_hidden_layers
    dev = next(model.parameters()).device
    dt = next(model.parameters()).dtype
    wrapper = QwenStaticWrapper(model, L, argmax=argmax).eval()
    args = static_inputs(cfg, tokens, max_cache_len, device=str(dev), dtype=dt)
    name = model_name or ("Qwen2_Decode" if tokens == 1 else "Qwen2_Prefill")
    return extract_ir(wrapper, args, model_name=name, input_names=input_names(L), strip_prefix="model.")


def kv_mapping(prefill_ir: dict, decode_ir: dict, num_layers: int, prefill_seq_len: int,
               max_cache_len: int) -> dict:
    """The reference's KV mapping record: prefill outputs 1..2L are the caches (output
    0 is the logits), decode inputs after the four fixed ones are the caches, decode
    outputs 1..2L are the updated caches."""
    pkv = prefill_ir["graph_outputs"][1:1 + 2 * num_layers]
    dkv_in = [s for s in decode_ir["graph_inputs"] if s["name"] not in FIXED_INPUTS]
    dkv_out = decode_ir["graph_outputs"][1:1 + 2 * num_layers]
    if len(pkv) != 2 * num_layers or len(dkv_in) != 2 * num_layers or len(dkv_out) != 2 * num_layers:
        raise ValueError("graphs do not carry 2 caches per layer")
    layers = []
    for i in range(num_layers):
        layers.append({
            "layer": i,
            "prefill_key_output": pkv[2 * i]["name"], "prefill_value_output": pkv[2 * i + 1]["name"],
            "decode_key_input": dkv_in[2 * i]["name"], "decode_value_input": dkv_in[2 * i + 1]["name"],
            "decode_key_output": dkv_out[2 * i]["name"], "decode_value_output": dkv_out[2 * i + 1]["name"],
        })
    return {"num_layers": num_layers, "prefill_seq_len": prefill_seq_len, "max_cache_len": max_cache_len,
            "layers": layers}
