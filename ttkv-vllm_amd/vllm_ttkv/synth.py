"""Seeded synthetic inputs with the benchmark's shapes (Llama-3.2-3B attention geometry).

Keys are low rank along tokens with outlier channels, the property the codec exploits:
per KV head h, K_h = Z_h @ B_h + 0.05 * N(0,1) with Z_h ~ N(0,1)[T, 96], B_h ~ N(0, 1/96)[96, d],
and channels 0-7 of every head scaled x8. Z is drawn independently per head, so the first
unfolding [T, H*d] has rank ~H*96 and an r1=110 budget binds (the decoder has no zero rows).
Values V ~ N(0,1); decode queries q ~ N(0,1) rounded to fp16.

All draws come from a torch.Generator on `device`, so the same seed gives the same tensors on
the same device type (CPU draws are what the parity tests and the CPU baseline use).
"""
from __future__ import annotations

import torch

LLAMA32_3B = dict(num_heads=24, num_kv_heads=8, head_dim=128, num_layers=28)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def keys(T: int, H: int = 8, d: int = 128, seed: int = 0, device="cpu", inner: int = 96,
         noise: float = 0.05, outliers: int = 8, outlier_scale: float = 8.0) -> torch.Tensor:
    """Raw (pre-RoPE) keys [H, T, d] fp32."""
    g = _gen(seed, device)
    K = torch.empty(H, T, d, device=device)
    for h in range(H):
        Z = torch.randn(T, inner, generator=g, device=device)
        B = torch.randn(inner, d, generator=g, device=device) * (1.0 / inner) ** 0.5
        K[h] = Z @ B + noise * torch.randn(T, d, generator=g, device=device)
    K[:, :, :outliers] *= outlier_scale
    return K


def values(T: int, H: int = 8, d: int = 128, seed: int = 0, device="cpu") -> torch.Tensor:
    """Values [H, T, d] fp32."""
    return torch.randn(H, T, d, generator=_gen(seed + 7919, device), device=device)


def queries(n: int, HQ: int = 24, d: int = 128, seed: int = 0, device="cpu",
            dtype=torch.float16) -> torch.Tensor:
    """Post-RoPE queries [n, HQ, d] ~ N(0,1) in `dtype`."""
    return torch.randn(n, HQ, d, generator=_gen(seed + 104729, device), device=device).to(dtype)


def shuffled_block_table(seq_lens, block_size: int, seed: int = 0, extra_blocks: int = 0):
    """A block table [B, max_blocks] int32 over a seeded random permutation of physical blocks.

    Returns (block_table, num_blocks). Unused table entries are -1 (never read: a request reads
    only its first ceil(seq_len / block_size) blocks)."""
    need = [-(-int(n) // block_size) for n in seq_lens]
    total = sum(need) + extra_blocks
    perm = torch.randperm(total, generator=_gen(seed + 15485863, "cpu")).to(torch.int32)
    width = max(max(need), 1)
    bt = torch.full((len(need), width), -1, dtype=torch.int32)
    off = 0
    for r, k in enumerate(need):
        bt[r, :k] = perm[off:off + k]
        off += k
    return bt, total
