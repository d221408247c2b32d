"""The two coefficient storage modes that extend the reference format (TEST INFRASTRUCTURE ONLY).

The reference stores a token's r1 coefficients one way only: int8 values and one fp16 ruler
(`vllm_ttkv/layout.py:161-193`, qbits = 8; `pack_k_slots` views the values as int8 bytes, so no
other width can be written by it). The layout's `qbits` selects two more modes here, defined by
this build and not by the reference, so nothing the reference wrote can pin them ("parity
unpinned" against the reference). They are pinned instead by closed forms and brute force in
`tests/test_coef_modes.py`: exactness of every stored value, the quantiser's error bound, the
scale rule checked bit by bit, a bit-at-a-time packer on small inputs, and round trips.

  qbits 16 ("fp16"): the coefficients as fp16, round to nearest even, 2 * r1 bytes, no ruler.
  qbits 4 ("int4, group 32"): for each group of 32 ranks, m = max |c|, scale = m / 7 (IEEE fp32)
      rounded UP to 8 significant bits, then clamped to [2^-14, 9344] (0 when m = 0);
      q = clamp(rint(c / scale), -7, 7); value = q * scale (exact in fp16: 3 + 8 bits).
      Stored as 4 * ceil(r1 / 8) bytes of little-endian 32-bit words, word w holding rank 8w + 2m
      at bits 4m..4m+3 and rank 8w + 2m + 1 at bits 16+4m..16+4m+3 (m = 0..3, two's complement,
      pad nibbles 0), then ceil(r1 / 32) fp16 scales.

The rest of the K slot (the residual rows) and the V slot are the reference's, at the offset
`coeff_bytes + coeff_scale_bytes`. A frozen write computes c = M @ pinv (as the reference's
`encode_frozen`, encode.py:322-324), quantises it by the mode, and forms the residual against the
stored coefficient values: R = K - value @ decoder_f.
"""
from __future__ import annotations

import numpy as np
import torch

SCALE_MIN = 2.0 ** -14
SCALE_MAX = 9344.0  # 73 * 2^7: the largest 8-significant-bit value with 7 * it <= 65504


def coeff_bytes(qbits: int, r1: int) -> int:
    if qbits == 8:
        return r1
    if qbits == 16:
        return 2 * r1
    if qbits == 4:
        return 4 * ((r1 + 7) // 8)
    raise ValueError(f"qbits must be 8, 16 or 4, got {qbits}")


def coeff_scale_bytes(qbits: int, r1: int) -> int:
    return {8: 2, 16: 0, 4: 2 * ((r1 + 31) // 32)}[qbits]


def group_scales(c: torch.Tensor) -> torch.Tensor:
    """c [n, r1] fp32 -> scales [n, ceil(r1/32)] fp32 by the rule above (numpy bit operations)."""
    n, r1 = c.shape
    ng = (r1 + 31) // 32
    a = np.zeros((n, ng * 32), dtype=np.float32)
    a[:, :r1] = np.abs(c.detach().cpu().numpy().astype(np.float32))
    m = a.reshape(n, ng, 32).max(-1)
    s = (m / np.float32(7.0)).astype(np.float32)          # IEEE fp32 division
    u = s.view(np.uint32).copy()
    up = (u & np.uint32(0xFFFF)) != 0
    u[up] = (u[up] & np.uint32(0xFFFF0000)) + np.uint32(0x10000)
    s = u.view(np.float32)
    s = np.minimum(np.maximum(s, np.float32(SCALE_MIN)), np.float32(SCALE_MAX))
    s[m == 0] = 0.0
    return torch.from_numpy(s.astype(np.float32))


def quantise(c: torch.Tensor, qbits: int):
    """c [n, r1] fp32 -> (values fp32 [n, r1], q, scales): the stored coefficient values, and
    for qbits 4 the integers q [n, r1] (int8) and group scales [n, ng] (fp32); for qbits 16 q is
    the fp16 tensor and scales is None."""
    c = c.to(torch.float32)
    if qbits == 16:
        h = c.to(torch.float16)
        return h.to(torch.float32), h, None
    if qbits != 4:
        raise ValueError("quantise() covers the fp16 and 4-bit modes")
    n, r1 = c.shape
    s = group_scales(c)
    sr = s.repeat_interleave(32, dim=1)[:, :r1]
    safe = torch.where(sr > 0, sr, torch.ones_like(sr))
    q = torch.where(sr > 0, torch.clamp(torch.round(c / safe), -7, 7), torch.zeros_like(c))
    return q * sr, q.to(torch.int8), s


def pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """q [n, r1] ints in [-8, 7] -> uint8 [n, 4 * ceil(r1/8)] in the word-interleaved order."""
    n, r1 = q.shape
    W = (r1 + 7) // 8
    a = np.zeros((n, 8 * W), dtype=np.uint32)
    a[:, :r1] = q.cpu().numpy().astype(np.int64) & 15
    a = a.reshape(n, W, 4, 2)                              # rank 8w + 2m + e
    shift = (4 * np.arange(4, dtype=np.uint32))[None, None, :]
    word = ((a[..., 0] << shift) | (a[..., 1] << (shift + np.uint32(16)))).sum(-1, dtype=np.uint32)
    return torch.from_numpy(word.astype("<u4").view(np.uint8).reshape(n, 4 * W).copy())


def unpack_nibbles(b: torch.Tensor, r1: int) -> torch.Tensor:
    """Inverse of pack_nibbles -> int8 [n, r1]."""
    n = b.shape[0]
    W = (r1 + 7) // 8
    word = np.ascontiguousarray(b[:, :4 * W].cpu().numpy()).view("<u4").reshape(n, W)
    shift = 4 * np.arange(4, dtype=np.uint32)
    lo = (word[:, :, None] >> shift) & 15
    hi = (word[:, :, None] >> (shift + 16)) & 15
    q = np.stack([lo, hi], -1).reshape(n, 8 * W)[:, :r1].astype(np.int16)
    q = np.where(q >= 8, q - 16, q)
    return torch.from_numpy(q.astype(np.int8))


def field_bytes(qbits: int, r1: int, q: torch.Tensor, scales) -> torch.Tensor:
    """The coefficient field [n, coeff_bytes + coeff_scale_bytes] uint8 of quantise()'s output."""
    if qbits == 16:
        return q.to(torch.float16).contiguous().view(torch.uint8).reshape(q.shape[0], 2 * r1)
    vals = pack_nibbles(q)
    sb = scales.to(torch.float16).contiguous().view(torch.uint8).reshape(q.shape[0], -1)
    return torch.cat([vals, sb], 1)


def values_from_field(qbits: int, r1: int, field: torch.Tensor) -> torch.Tensor:
    """The stored coefficient values fp32 [n, r1] of a coefficient field (fp16 or 4-bit mode)."""
    n = field.shape[0]
    if qbits == 16:
        return field[:, :2 * r1].contiguous().view(torch.float16).to(torch.float32)
    cb = coeff_bytes(4, r1)
    ng = (r1 + 31) // 32
    q = unpack_nibbles(field[:, :cb], r1).to(torch.float32)
    s = field[:, cb:cb + 2 * ng].contiguous().view(torch.float16).to(torch.float32)
    return q * s.repeat_interleave(32, dim=1)[:, :r1]
