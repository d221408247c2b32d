"""What one cache slot holds: the per-token blob's byte geometry.

Same public surface as the reference's `vllm_ttkv/layout.py:44-157, 264-275` (`align_up`,
`packed_row_bytes`, `TTKLayout`, `layout_for_config`) so callers and calibration tooling keep
working. The byte format is the reference's, unchanged:

    blob   = [K slot | V slot], each zero-padded to `align` (16) bytes
    K slot = r1 int8 coefficients | fp16 coefficient ruler | H x (bitmap d/8 | codes | fp16 ruler)
    V slot = H x (bitmap d/8 | codes | fp16 ruler)

Packing and unpacking are done on the GPU by `libttkv_hip` (the write and read kernels); this
module only owns the arithmetic that sizes the cache and addresses the fields.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

# The three shipped allocations (codec/ttkv_codec.py:272-298). `res_frac` is a FRACTION of d;
# `k_lanes` (the V lane count) is ABSOLUTE.
CONFIGS = {
    "safe": dict(tols=0.20, qbits=8, res_frac=0.633, res_bits=3, k_lanes=81, vbits=3),
    "tight": dict(tols=0.20, qbits=8, res_frac=0.25, res_bits=3, k_lanes=45, vbits=3),
    "campaign4x": dict(tols=0.20, qbits=8, res_frac=0.50, res_bits=4, k_lanes=64, vbits=4),
}


def align_up(n: int, a: int) -> int:
    return n if a <= 1 else ((n + a - 1) // a) * a


def packed_row_bytes(k: int, bits: int) -> int:
    """Each row's code stream is padded to whole bytes."""
    return math.ceil(k * bits / 8)


@dataclass(frozen=True)
class TTKLayout:
    """Byte layout of one layer's compressed cache; every size is per token."""

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
            raise ValueError(f"head dim {self.d} is not a multiple of 8; the lane bitmap is d/8 "
                             f"bytes, so d must be a whole number of bytes")
        if self.res_k > self.d:
            raise ValueError(f"res_k={self.res_k} exceeds d={self.d}")
        if self.v_lanes > self.d:
            raise ValueError(f"v_lanes={self.v_lanes} exceeds d={self.d}: `k_lanes` is an "
                             f"ABSOLUTE lane count and has to be re-derived for this head dim")

    @property
    def coeff_bytes(self) -> int:
        if (self.r1 * self.qbits) % 8:
            raise ValueError(f"r1={self.r1} at qbits={self.qbits} is not a whole number of bytes")
        return self.r1 * self.qbits // 8

    @property
    def coeff_scale_bytes(self) -> int:
        return 2

    @property
    def k_row_bytes(self) -> int:
        return self.d // 8 + packed_row_bytes(self.res_k, self.res_bits) + 2

    @property
    def v_row_bytes(self) -> int:
        return self.d // 8 + packed_row_bytes(self.v_lanes, self.v_bits) + 2

    @property
    def k_slot_bytes(self) -> int:
        return align_up(self.coeff_bytes + self.coeff_scale_bytes + self.H * self.k_row_bytes,
                        self.align)

    @property
    def v_slot_bytes(self) -> int:
        return align_up(self.H * self.v_row_bytes, self.align)

    @property
    def v_offset(self) -> int:
        return self.k_slot_bytes

    def dense_bytes_per_token(self) -> int:
        return 2 * self.H * self.d * 2

    def compressed_bytes_per_token(self) -> int:
        return self.k_slot_bytes + self.v_slot_bytes

    def ratio(self) -> float:
        return self.dense_bytes_per_token() / self.compressed_bytes_per_token()


def layout_for_config(cfg: dict, r1: int, H: int = 8, d: int = 128) -> TTKLayout:
    return TTKLayout(H=H, d=d, r1=r1, qbits=cfg["qbits"],
                     res_k=max(int(d * cfg["res_frac"]), 1), res_bits=cfg["res_bits"],
                     v_lanes=cfg["k_lanes"], v_bits=cfg["vbits"])
