"""Seeded synthetic weights and inputs for the benchmark configurations.

Seeds: a ``torch.Generator`` seeded with 0 draws weights, 1 draws activations and
KV caches, 2 draws token ids. Linear weights and biases ~ N(0, 0.02); RMSNorm
weights ~ N(1, 0.02) for the MLP block and exactly 1 for the full model; the
rotary ``inv_freq`` is ``1/theta^(2i/d)`` with the config's theta (1e6; the
reference synthesises it with 10000, D6). bf16 values are generated in fp32 and
rounded, so every consumer sees the same bits.
"""

from __future__ import annotations

import numpy as np
import torch

from irgen.qwen import QWEN2_5_1_5B, QwenConfig, inv_freq

_TD = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32, "int64": torch.int64}


def make_weights(ir: dict, cfg: QwenConfig = QWEN2_5_1_5B, seed: int = 0, norm_std: float = 0.0,
                 device: str = "cpu") -> dict[str, torch.Tensor]:
    """State-dict-keyed weights for every ``ir["weights"]`` entry, in IR order."""
    g = torch.Generator(device=device).manual_seed(seed)
    out: dict[str, torch.Tensor] = {}
    for w in ir["weights"]:
        key, shape, dt = w["name"], tuple(w["shape"]), _TD[w.get("dtype", "float32")]
        if key.endswith("inv_freq"):
            out[key] = inv_freq(cfg).to(device)
            continue
        if "norm" in key:
            t = torch.ones(shape, device=device)
            if norm_std:
                t = t + norm_std * torch.randn(shape, generator=g, device=device)
        else:
            t = 0.02 * torch.randn(shape, generator=g, device=device)
        out[key] = t.to(dt)
    return out


def to_host(t: torch.Tensor) -> np.ndarray:
    """Tensor → numpy host array (bf16 as uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.uint16).numpy()
    return t.numpy()


def mlp_inputs(tokens: int, cfg: QwenConfig = QWEN2_5_1_5B, seed: int = 1) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    return {"x": torch.randn((tokens, cfg.hidden), generator=g).to(_TD[cfg.dtype])}


def attention_inputs(kv_len: int, cfg: QwenConfig = QWEN2_5_1_5B, seed: int = 1) -> dict[str, torch.Tensor]:
    """cfg2: hidden ~ N(0,1), caches ~ N(0,1) (row kv_len-1 is overwritten), mask all 0."""
    g = torch.Generator().manual_seed(seed)
    dt = _TD[cfg.dtype]
    pos = kv_len - 1
    return {
        "hidden_states": torch.randn((1, 1, cfg.hidden), generator=g).to(dt),
        "attention_mask": torch.zeros((1, 1, 1, kv_len), dtype=dt),
        "position_ids": torch.tensor([[pos]], dtype=torch.int64),
        "cache_position": torch.tensor([pos], dtype=torch.int64),
        "past_key_0": torch.randn((1, cfg.kv_heads, kv_len, cfg.head_dim), generator=g).to(dt),
        "past_value_0": torch.randn((1, cfg.kv_heads, kv_len, cfg.head_dim), generator=g).to(dt),
    }


def decode_mask(max_cache_len: int, pos: int, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    m = torch.full((1, 1, 1, max_cache_len), float("-inf"))
    m[..., :pos + 1] = 0.0
    return m.to(dtype)


def decode_inputs(max_cache_len: int, start_pos: int, cfg: QwenConfig = QWEN2_5_1_5B, seed: int = 1,
                  token_seed: int = 2, device: str = "cpu") -> dict[str, torch.Tensor]:
    """cfg3: caches filled ~N(0,1) on positions [0, start_pos), zero after; first token ~U[0, vocab)."""
    g = torch.Generator(device=device).manual_seed(seed)
    dt = _TD[cfg.dtype]
    d: dict[str, torch.Tensor] = {
        "input_ids": torch.randint(0, cfg.vocab, (1, 1), generator=torch.Generator().manual_seed(token_seed)).to(device),
        "attention_mask": decode_mask(max_cache_len, start_pos, dt).to(device),
        "position_ids": torch.tensor([[start_pos]], dtype=torch.int64, device=device),
        "cache_position": torch.tensor([start_pos], dtype=torch.int64, device=device),
    }
    for li in range(cfg.layers):
        for kind in ("key", "value"):
            t = torch.zeros((1, cfg.kv_heads, max_cache_len, cfg.head_dim), dtype=dt, device=device)
            t[:, :, :start_pos] = torch.randn((1, cfg.kv_heads, start_pos, cfg.head_dim), generator=g,
                                              device=device).to(dt)
            d[f"past_{kind}_{li}"] = t
    return d


def prefill_inputs(tokens: int, max_cache_len: int | None = None, cfg: QwenConfig = QWEN2_5_1_5B,
                   token_seed: int = 2, device: str = "cpu") -> dict[str, torch.Tensor]:
    """cfg4: ``tokens`` prompt ids ~U[0, vocab) at positions 0..T-1, causal mask [1, 1, T, S]
    (0 on and below the diagonal, -inf above and past T), empty (zero) static caches of length S."""
    S = max_cache_len or tokens
    dt = _TD[cfg.dtype]
    g = torch.Generator().manual_seed(token_seed)
    mask = torch.full((tokens, S), float("-inf"))
    mask[:, :tokens] = torch.triu(torch.full((tokens, tokens), float("-inf")), diagonal=1)
    d: dict[str, torch.Tensor] = {
        "input_ids": torch.randint(0, cfg.vocab, (1, tokens), generator=g).to(device),
        "attention_mask": mask.to(dt).reshape(1, 1, tokens, S).to(device),
        "position_ids": torch.arange(tokens, dtype=torch.int64).reshape(1, tokens).to(device),
        "cache_position": torch.arange(tokens, dtype=torch.int64).to(device),
    }
    for li in range(cfg.layers):
        for kind in ("key", "value"):
            d[f"past_{kind}_{li}"] = torch.zeros((1, cfg.kv_heads, S, cfg.head_dim), dtype=dt, device=device)
    return d
