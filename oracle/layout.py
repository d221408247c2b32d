"""Slot geometry and the per-token blob, restated from the reference (TEST INFRASTRUCTURE ONLY).

Reference: `vllm_ttkv/layout.py:44-157` (geometry), `:161-261` (pack/unpack), `:264-275`
(layout_for_config).

One token's blob is `[K slot | V slot]`:
  K slot = r1 int8 coefficients, fp16 coefficient ruler (LE), then for h in 0..H-1 a row of
           bitmap (d/8 B) + MSB-first codes (ceil(res_k*res_bits/8) B) + fp16 ruler (LE);
           zero-padded to a multiple of 16.
  V slot = for h in 0..H-1 a row of bitmap + codes + fp16 ruler; zero-padded to 16.
The codec's row order inside a store is (head, token) = h*n + i.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


def align_up(n: int, a: int) -> int:
    """layout.py:44-47."""
    return n if a <= 1 else ((n + a - 1) // a) * a


def packed_row_bytes(k: int, bits: int) -> int:
    """layout.py:50-53: each row padded to whole bytes."""
    return math.ceil(k * bits / 8)


@dataclass(frozen=True)
class Layout:
    """layout.py:56-157 (`TTKLayout`). All sizes per token."""

    H: int
    d: int
    r1: int
    qbits: int
    res_k: int
    res_bits: int
    v_lanes: int
    v_bits: int
    align: int = 16

    def __post_init__(self):
        if self.d % 8:
            raise ValueError(f"head dim {self.d} is not a multiple of 8")
        if self.res_k > self.d or self.v_lanes > self.d:
            raise ValueError("lane count exceeds d")

    @property
    def coeff_bytes(self) -> int:
        """layout.py:98-101 for qbits 8; qbits 16 and 4 are this build's own modes
        (`coef_modes`)."""
        if self.qbits == 8:
            return self.r1
        from .coef_modes import coeff_bytes
        return coeff_bytes(self.qbits, self.r1)

    @property
    def coeff_scale_bytes(self) -> int:
        from .coef_modes import coeff_scale_bytes
        return coeff_scale_bytes(self.qbits, self.r1)

    @property
    def k_pb(self) -> int:
        return packed_row_bytes(self.res_k, self.res_bits)

    @property
    def v_pb(self) -> int:
        return packed_row_bytes(self.v_lanes, self.v_bits)

    @property
    def k_row_bytes(self) -> int:
        return self.d // 8 + self.k_pb + 2

    @property
    def v_row_bytes(self) -> int:
        return self.d // 8 + self.v_pb + 2

    @property
    def k_field_off(self) -> int:
        """Byte offset of head 0's residual row inside the K slot."""
        return self.coeff_bytes + self.coeff_scale_bytes

    @property
    def k_slot_bytes(self) -> int:
        return align_up(self.k_field_off + self.H * self.k_row_bytes, self.align)

    @property
    def v_slot_bytes(self) -> int:
        return align_up(self.H * self.v_row_bytes, self.align)

    @property
    def v_offset(self) -> int:
        return self.k_slot_bytes

    def compressed_bytes_per_token(self) -> int:
        return self.k_slot_bytes + self.v_slot_bytes

    def dense_bytes_per_token(self) -> int:
        return 2 * self.H * self.d * 2

    def ratio(self) -> float:
        return self.dense_bytes_per_token() / self.compressed_bytes_per_token()


def layout_for_config(cfg: dict, r1: int, H: int = 8, d: int = 128) -> Layout:
    """layout.py:264-275: res_k from the FRACTION, v_lanes ABSOLUTE."""
    return Layout(H=H, d=d, r1=r1, qbits=cfg["qbits"],
                  res_k=max(int(d * cfg["res_frac"]), 1), res_bits=cfg["res_bits"],
                  v_lanes=cfg["k_lanes"], v_bits=cfg["vbits"])


def _f16_bytes(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float16).contiguous().view(torch.uint8).reshape(-1, 2)


def pack_k_slots(lay: Layout, coeff_q, coeff_scale, bitmap, packed, scale) -> torch.Tensor:
    """layout.py:161-193. coeff_q [n,r1] int8, coeff_scale [n] fp16, residual rows over H*n
    rows in (head, token) order -> [n, k_slot_bytes] uint8. For qbits 16 / 4 (`coef_modes`),
    coeff_q / coeff_scale are `coef_modes.quantise`'s q and scales."""
    n = coeff_q.shape[0]
    if bitmap.shape[0] != lay.H * n:
        raise ValueError("residual rows != H*n")
    out = torch.zeros(n, lay.k_slot_bytes, dtype=torch.uint8)
    if lay.qbits == 8:
        out[:, :lay.coeff_bytes] = coeff_q.contiguous().view(torch.uint8)
        out[:, lay.coeff_bytes:lay.coeff_bytes + 2] = _f16_bytes(coeff_scale)
    else:  # this build's fp16 / 4-bit modes: coeff_q, coeff_scale as coef_modes.quantise gives
        from .coef_modes import field_bytes
        out[:, :lay.k_field_off] = field_bytes(lay.qbits, lay.r1, coeff_q, coeff_scale)
    for h in range(lay.H):
        base = lay.k_field_off + h * lay.k_row_bytes
        rows = slice(h * n, (h + 1) * n)
        out[:, base:base + lay.d // 8] = bitmap[rows]
        out[:, base + lay.d // 8:base + lay.d // 8 + lay.k_pb] = packed[rows]
        out[:, base + lay.d // 8 + lay.k_pb:base + lay.k_row_bytes] = _f16_bytes(scale[rows])
    return out


def unpack_k_slots(lay: Layout, slots: torch.Tensor):
    """layout.py:196-219 -> (coeff_q int8 [n,r1], coeff_scale fp16 [n], (bitmap, packed, scale)).
    For qbits 16 / 4 (`coef_modes`): (the stored coefficient values fp32 [n, r1], None, rows)."""
    n = slots.shape[0]
    if lay.qbits == 8:
        coeff_q = slots[:, :lay.coeff_bytes].clone().view(torch.int8)
        coeff_scale = slots[:, lay.coeff_bytes:lay.coeff_bytes + 2].clone().view(
            torch.float16).reshape(n)
    else:
        from .coef_modes import values_from_field
        coeff_q, coeff_scale = values_from_field(lay.qbits, lay.r1, slots[:, :lay.k_field_off]), None
    bm, pk, sc = [], [], []
    for h in range(lay.H):
        base = lay.k_field_off + h * lay.k_row_bytes
        bm.append(slots[:, base:base + lay.d // 8])
        pk.append(slots[:, base + lay.d // 8:base + lay.d // 8 + lay.k_pb])
        sc.append(slots[:, base + lay.d // 8 + lay.k_pb:base + lay.k_row_bytes].clone()
                  .view(torch.float16).reshape(n))
    return coeff_q, coeff_scale, (torch.cat(bm).contiguous(), torch.cat(pk).contiguous(),
                                  torch.cat(sc).contiguous())


def pack_v_slots(lay: Layout, bitmap, packed, scale) -> torch.Tensor:
    """layout.py:222-239."""
    if bitmap.shape[0] % lay.H:
        raise ValueError("V rows not a multiple of H")
    n = bitmap.shape[0] // lay.H
    out = torch.zeros(n, lay.v_slot_bytes, dtype=torch.uint8)
    for h in range(lay.H):
        base = h * lay.v_row_bytes
        rows = slice(h * n, (h + 1) * n)
        out[:, base:base + lay.d // 8] = bitmap[rows]
        out[:, base + lay.d // 8:base + lay.d // 8 + lay.v_pb] = packed[rows]
        out[:, base + lay.d // 8 + lay.v_pb:base + lay.v_row_bytes] = _f16_bytes(scale[rows])
    return out


def unpack_v_slots(lay: Layout, slots: torch.Tensor):
    """layout.py:242-261 -> (bitmap, packed, scale) over H*n rows."""
    n = slots.shape[0]
    bm, pk, sc = [], [], []
    for h in range(lay.H):
        base = h * lay.v_row_bytes
        bm.append(slots[:, base:base + lay.d // 8])
        pk.append(slots[:, base + lay.d // 8:base + lay.d // 8 + lay.v_pb])
        sc.append(slots[:, base + lay.d // 8 + lay.v_pb:base + lay.v_row_bytes].clone()
                  .view(torch.float16).reshape(n))
    return (torch.cat(bm).contiguous(), torch.cat(pk).contiguous(), torch.cat(sc).contiguous())


def split_blob(lay: Layout, blob: torch.Tensor):
    """decode.py:286-304."""
    k = lay.k_slot_bytes
    if blob.shape[-1] != k + lay.v_slot_bytes:
        raise ValueError("blob width does not match the layout")
    return blob[:, :k].contiguous(), blob[:, k:].contiguous()
