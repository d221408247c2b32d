"""RoPE angle tables in vLLM's `cos_sin_cache` layout ([max_pos, d]: cos | sin by halves).

In serving the table comes from the model's own rotary module (vllm_ttkv/impl.py:326-352 in the
reference); this builder exists for benchmarks and tests, with the public Llama 3 rope-scaling
rule (Llama-3.2-3B: theta 500000, factor 32, low/high frequency factors 1 and 4, original
context 8192).
"""
from __future__ import annotations

import math

import torch

LLAMA32_3B_ROPE = dict(theta=500000.0, factor=32.0, low_freq_factor=1.0, high_freq_factor=4.0,
                       original_max_position=8192)


def llama3_inv_freq(d: int = 128, theta: float = 500000.0, factor: float = 32.0,
                    low_freq_factor: float = 1.0, high_freq_factor: float = 4.0,
                    original_max_position: int = 8192) -> torch.Tensor:
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    wavelen = 2 * math.pi / inv
    smooth = (original_max_position / wavelen - low_freq_factor) / (high_freq_factor
                                                                    - low_freq_factor)
    mid = (1 - smooth) * inv / factor + smooth * inv
    lo_wl = original_max_position / low_freq_factor
    hi_wl = original_max_position / high_freq_factor
    return torch.where(wavelen < hi_wl, inv, torch.where(wavelen > lo_wl, inv / factor, mid))


def cos_sin_cache(max_pos: int, d: int = 128, inv_freq: torch.Tensor | None = None,
                  device="cpu") -> torch.Tensor:
    """[max_pos, d] fp32: cos(t * inv_freq) in columns [0, d/2), sin in [d/2, d)."""
    inv = llama3_inv_freq(d, **LLAMA32_3B_ROPE) if inv_freq is None else inv_freq
    t = torch.arange(max_pos, dtype=torch.float32)
    f = torch.outer(t, inv.to(torch.float32))
    return torch.cat([f.cos(), f.sin()], dim=-1).contiguous().to(device)
