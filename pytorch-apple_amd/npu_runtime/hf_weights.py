"""Weights for an IR graph from a local HF checkpoint directory (safetensors).

Restates the reference's loader (`examples/run_qwen_graph.py:30-100`,
`examples/hf_utils.py:55-150`) for the keys an IR's ``weights`` list names:

* the tensors come from ``model.safetensors.index.json``'s shards when the index
  exists, otherwise from every ``*.safetensors`` file in the directory; only the
  shards that hold a needed key are opened, and only the needed keys are read;
* an IR key missing from the checkpoint is tried without a leading ``model.``
  (wrappers hold the model as ``self.model``);
* a missing ``lm_head.weight`` takes the embedding matrix (tied embeddings);
* a missing rotary ``inv_freq`` is synthesised as ``1 / theta^(2i/d)`` in fp32
  with ``theta`` = ``rope_theta`` from the directory's ``config.json`` (1e6 for
  Qwen2.5; 10000, Qwen2Config's default, when the file has none), as HF builds it
  (the reference hard-codes 10000 and writes it in bf16);
* an empty ``lifted_tensor`` placeholder becomes an empty tensor;
* floating tensors are converted to the IR's declared dtype (bf16 for Qwen2.5).

Tensors are returned as torch tensors on ``device`` (safetensors reads straight
into device memory when ``device`` is a GPU), keyed by IR weight name, ready for
``DAGExecutor.load_weights``.
"""

from __future__ import annotations

import glob
import json
import os

import torch

_TORCH = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32,
          "int64": torch.int64, "int32": torch.int32}


def _shard_index(model_dir: str) -> dict[str, str]:
    """checkpoint key → shard file path."""
    from safetensors import safe_open

    index_path = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(index_path):
        with open(index_path) as f:
            wm = json.load(f).get("weight_map", {})
        return {k: os.path.join(model_dir, v) for k, v in wm.items()}
    out: dict[str, str] = {}
    for path in sorted(glob.glob(os.path.join(model_dir, "*.safetensors"))):
        with safe_open(path, framework="pt") as f:
            for k in f.keys():
                out[k] = path
    return out


def _rope_theta(model_dir: str, default: float) -> float:
    path = os.path.join(model_dir, "config.json")
    if os.path.exists(path):
        with open(path) as f:
            cfg = json.load(f)
        theta = cfg.get("rope_theta")
        if theta is None:
            theta = (cfg.get("rope_parameters") or {}).get("rope_theta")
        if theta is not None:
            return float(theta)
    return default


def load_safetensors_weights(model_dir: str, ir: dict, device: str | torch.device = "cpu",
                             rope_theta: float | None = None) -> dict[str, torch.Tensor]:
    """Every weight ``ir["weights"]`` names, as a tensor of its IR dtype on ``device``."""
    from safetensors import safe_open

    where = _shard_index(model_dir)
    plan: dict[str, str] = {}   # IR key -> checkpoint key
    for w in ir.get("weights", []):
        key = w["name"]
        for cand in (key, key[len("model."):] if key.startswith("model.") else None):
            if cand is not None and cand in where:
                plan[key] = cand
                break
    by_file: dict[str, list[str]] = {}
    for key, ck in plan.items():
        by_file.setdefault(where[ck], []).append(key)
    dev = str(device)
    out: dict[str, torch.Tensor] = {}
    specs = {w["name"]: w for w in ir.get("weights", [])}
    for path, keys in by_file.items():
        with safe_open(path, framework="pt", device=dev) as f:
            for key in keys:
                t = f.get_tensor(plan[key])
                want = _TORCH.get(specs[key].get("dtype", "float32"), t.dtype)
                out[key] = t.to(want) if t.dtype != want else t
    # without rope_theta in config.json HF builds inv_freq with Qwen2Config's default, 10000
    theta = rope_theta if rope_theta is not None else _rope_theta(model_dir, 10000.0)
    for key, w in specs.items():
        if key in out:
            continue
        if key.endswith("lm_head.weight"):
            emb = key.replace("lm_head.weight", "model.embed_tokens.weight")
            src = out.get(emb)
            if src is None:
                ck = next((c for c in (emb, emb[len("model."):]) if c in where), None)
                if ck is not None:
                    with safe_open(where[ck], framework="pt", device=dev) as f:
                        src = f.get_tensor(ck)
            if src is not None:
                out[key] = src.to(_TORCH.get(w.get("dtype", "bfloat16"), src.dtype))
                continue
        if "inv_freq" in key:
            d2 = int(w["shape"][0])
            inv = 1.0 / (theta ** (torch.arange(0, 2 * d2, 2, dtype=torch.int64).float() / (2 * d2)))
            out[key] = inv.to(device=dev, dtype=_TORCH.get(w.get("dtype", "float32"), torch.float32))
            continue
        if "lifted_tensor" in key and list(w["shape"]) == [0]:
            out[key] = torch.empty(0, dtype=_TORCH.get(w.get("dtype", "bfloat16"), torch.bfloat16), device=dev)
            continue
        raise KeyError(f"weight {key} is not in the checkpoint at {model_dir}")
    return out
