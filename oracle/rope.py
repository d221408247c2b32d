"""RoPE tables and rotation, restated (TEST INFRASTRUCTURE ONLY).

Reference: `vllm_ttkv/decode.py:54-122` (`cos_sin_from_cache`: vLLM's `[max_pos, rot]` table is
`cat(cos, sin)` by halves and is duplicated across halves for the `(j, j+d/2)` pairing),
`codec/ttkv_packed_cache.py:486-498` (`_rotate_half`, `rope_apply`), `vllm_ttkv/reference.py:47-60`
(`rope_tables`, theta-only stand-in).

The llama3 frequency ramp is not in the reference (its oracle is theta-only); it is the public
Llama 3 rope-scaling rule (theta 500000, factor 32, low_freq_factor 1, high_freq_factor 4,
original_max_position_embeddings 8192 for Llama-3.2-3B), written here from the closed form and
pinned against `transformers`' own implementation in the CPU tests.
"""
from __future__ import annotations

import math

import torch

LLAMA32_3B_ROPE = dict(theta=500000.0, factor=32.0, low_freq_factor=1.0, high_freq_factor=4.0,
                       original_max_position=8192)


def inv_freq_llama3(d: int, theta: float, factor: float, low_freq_factor: float,
                    high_freq_factor: float, original_max_position: int) -> torch.Tensor:
    """fp32 [d/2] inverse frequencies with the llama3 wavelength ramp."""
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    wavelen = 2 * math.pi / inv
    lo_wl = original_max_position / low_freq_factor
    hi_wl = original_max_position / high_freq_factor
    smooth = (original_max_position / wavelen - low_freq_factor) / (high_freq_factor
                                                                    - low_freq_factor)
    mid = (1 - smooth) * inv / factor + smooth * inv
    return torch.where(wavelen < hi_wl, inv, torch.where(wavelen > lo_wl, inv / factor, mid))


def inv_freq_theta(d: int, theta: float = 10000.0) -> torch.Tensor:
    """reference.py:56-57 (the test stand-in)."""
    return 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))


def vllm_cos_sin_cache(inv_freq: torch.Tensor, max_pos: int) -> torch.Tensor:
    """vLLM's `[max_pos, d]` fp32 table: cos in the first d/2 columns, sin in the second."""
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.cat([freqs.cos(), freqs.sin()], dim=-1).contiguous()


def cos_sin_from_cache(cache: torch.Tensor, positions: torch.Tensor, head_dim: int):
    """decode.py:54-122 -> (cos, sin) each [n, d] fp32, halves duplicated."""
    rot = cache.shape[-1]
    if rot != head_dim:
        raise NotImplementedError("partial rotary")
    idx = positions.to(torch.long)
    if idx.numel() and int(idx.max()) >= cache.shape[0]:
        raise IndexError("position past the model's cos_sin_cache")
    row = cache[idx].to(torch.float32)
    c, s = row[:, :rot // 2], row[:, rot // 2:]
    return torch.cat([c, c], -1).contiguous(), torch.cat([s, s], -1).contiguous()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """ttkv_packed_cache.py:486-493: (j, j+d/2) pairing."""
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def rope_apply(x, cos, sin):
    """ttkv_packed_cache.py:496-498."""
    return x * cos + rotate_half(x) * sin
