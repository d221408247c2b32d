"""What one cache slot holds: the per-token blob's byte geometry.

Same public surface as the reference's `vllm_ttkv/layout.py:44-157, 264-275` (`align_up`,
`packed_row_bytes`, `TTKLayout`, `layout_for_config`) so callers and calibration tooling keep
working. The byte format is the reference's, unchanged:

    blob   = [K slot | V slot], each zero-padded to `align` (16) bytes
    K slot = r1 int8 coefficients | fp16 coefficient ruler | H x (bitmap d/8 | codes | fp16 ruler)
    V slot = H x (bitmap d/8 | codes | fp16 ruler)

The layout's `qbits` also selects two coefficient fields of this library's own, which the
reference cannot write (its packer views the coefficients as int8, layout.py:179):
    qbits 16: r1 fp16 coefficients, no ruler
    qbits 4 : 4-bit coefficients in [-7, 7] with one fp16 scale per group of 32 ranks
              (4 * ceil(r1/8) bytes of word-interleaved nibbles, then ceil(r1/32) scales)
They are offered as the `safe_fp16` and `campaign4x_int4g32` allocations (`EXTENSION_CONFIGS`).

On the serving path, packing and unpacking are done on the GPU by `libttkv_hip` (the write and
read kernels). This module owns the arithmetic that sizes the cache and addresses the fields, and
the same byte moves as tensor operations (`pack_k_slots` and friends) for callers that hold a
store as separate row arrays.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

# The three shipped allocations (codec/ttkv_codec.py:272-298). `res_frac` is a FRACTION of d;
# `k_lanes` (the V lane count) is ABSOLUTE.
CONFIGS = {
    "safe": dict(tols=0.20, qbits=8, res_frac=0.633, res_bits=3, k_lanes=81, vbits=3),
    "tight": dict(tols=0.20, qbits=8, res_frac=0.25, res_bits=3, k_lanes=45, vbits=3),
    "campaign4x": dict(tols=0.20, qbits=8, res_frac=0.50, res_bits=4, k_lanes=64, vbits=4),
}

# This library's own coefficient modes on the reference's residual / V geometry (not in the
# reference: fp16 coefficients; 4-bit coefficients with fp16 scales per 32 ranks). Looked up by
# name like the shipped allocations (`config_named`).
EXTENSION_CONFIGS = {
    "safe_fp16": dict(CONFIGS["safe"], qbits=16),
    "campaign4x_int4g32": dict(CONFIGS["campaign4x"], qbits=4),
}


def config_named(name: str) -> dict:
    """A shipped allocation or one of `EXTENSION_CONFIGS`, by name."""
    if name in CONFIGS:
        return CONFIGS[name]
    if name in EXTENSION_CONFIGS:
        return EXTENSION_CONFIGS[name]
    raise KeyError(f"unknown allocation {name!r}: one of {sorted(CONFIGS) + sorted(EXTENSION_CONFIGS)}")


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
        if self.qbits not in (8, 16, 4):
            raise ValueError(f"qbits={self.qbits}: the coefficient field is int8 (8, the "
                             f"reference's), fp16 (16) or 4-bit with group-32 scales (4)")

    @property
    def coeff_bytes(self) -> int:
        """Bytes of the coefficient values: r1 (int8), 2 * r1 (fp16), 4 * ceil(r1/8) (4-bit)."""
        if self.qbits == 8:
            return self.r1
        return 2 * self.r1 if self.qbits == 16 else 4 * ((self.r1 + 7) // 8)

    @property
    def coef_groups(self) -> int:
        """4-bit mode: groups of 32 ranks, one fp16 scale each; 0 otherwise."""
        return (self.r1 + 31) // 32 if self.qbits == 4 else 0

    @property
    def coeff_scale_bytes(self) -> int:
        """The int8 mode's fp16 ruler, the 4-bit mode's group scales, nothing for fp16."""
        return 2 if self.qbits == 8 else 2 * self.coef_groups

    @property
    def k_field(self) -> int:
        """Offset of head 0's residual row in the K slot."""
        return self.coeff_bytes + self.coeff_scale_bytes

    @property
    def k_row_bytes(self) -> int:
        return self.d // 8 + packed_row_bytes(self.res_k, self.res_bits) + 2

    @property
    def v_row_bytes(self) -> int:
        return self.d // 8 + packed_row_bytes(self.v_lanes, self.v_bits) + 2

    @property
    def k_slot_bytes(self) -> int:
        return align_up(self.k_field + self.H * self.k_row_bytes, self.align)

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


# ---------------------------------------------------------------- host-side slot (un)packing
# The write kernel packs slots on the device; these are the same byte moves as torch tensor
# operations, for callers that hold a store as separate row arrays (the reference's
# `pack_k_slots` / `unpack_k_slots` / `pack_v_slots` / `unpack_v_slots`, layout.py:161-261).
# A "row store" is any object with `rows` (H*n), `bitmap` [H*n, d/8] u8, `packed` [H*n, PB] u8
# and `scale` [H*n] fp16, rows in (head, token) order h*n + i. Each field of all H heads moves as
# ONE strided copy through a [n, H, row_bytes] view of the slot, not a loop over heads.

def _head_rows(slots, off: int, H: int, row: int):
    """`slots[:, off + h*row + b]` as a [n, H, row] view (no copy)."""
    return slots[:, off:off + H * row].unflatten(1, (H, row))


def _put_rows(view, bitmap, packed, scale, n: int, H: int, bm: int, pb: int):
    """Scatter (head, token)-ordered row fields into a [n, H, row] slot view."""
    view[:, :, :bm] = bitmap.reshape(H, n, bm).transpose(0, 1)
    view[:, :, bm:bm + pb] = packed.reshape(H, n, pb).transpose(0, 1)
    view[:, :, bm + pb:bm + pb + 2] = (scale.to(torch.float16).contiguous().view(torch.uint8)
                                       .reshape(H, n, 2).transpose(0, 1))


def _take_rows(view, n: int, H: int, bm: int, pb: int):
    """Gather a [n, H, row] slot view back into (head, token)-ordered row fields."""
    hv = view.transpose(0, 1)                                   # [H, n, row]
    bitmap = hv[:, :, :bm].reshape(H * n, bm).contiguous()
    packed = hv[:, :, bm:bm + pb].reshape(H * n, pb).contiguous()
    scale = hv[:, :, bm + pb:bm + pb + 2].contiguous().view(torch.float16).reshape(H * n)
    return bitmap, packed, scale


def _check_rows(rows, lay: TTKLayout, n: int, pb: int, what: str):
    if int(rows.rows) != lay.H * n:
        raise ValueError(f"{what} holds {rows.rows} rows, expected H*n = {lay.H}*{n}")
    if tuple(rows.bitmap.shape) != (lay.H * n, lay.d // 8) or tuple(rows.packed.shape) != (
            lay.H * n, pb) or rows.scale.numel() != lay.H * n:
        raise ValueError(f"{what} fields are bitmap {tuple(rows.bitmap.shape)}, packed "
                         f"{tuple(rows.packed.shape)}, scale {tuple(rows.scale.shape)}; the "
                         f"layout needs [{lay.H * n}, {lay.d // 8}], [{lay.H * n}, {pb}], "
                         f"[{lay.H * n}]")


# 4-bit mode: word w of the coefficient values holds rank 8w + 2m at bits 4m and rank 8w + 2m + 1
# at bits 16 + 4m (m = 0..3), so that a shift and a mask give two consecutive ranks as the low
# nibbles of a 16-bit pair.
_NIB_SHIFT = torch.tensor([4 * (k // 2) + 16 * (k % 2) for k in range(8)])  # rank 8w + k


def _pack_int4(q: torch.Tensor) -> torch.Tensor:
    n, r1 = q.shape
    W = (r1 + 7) // 8
    nib = torch.zeros(n, 8 * W, dtype=torch.int64, device=q.device)
    nib[:, :r1] = q.to(torch.int64) & 15
    words = (nib.reshape(n, W, 8) << _NIB_SHIFT.to(q.device)).sum(-1)   # disjoint bits
    return torch.stack([(words >> (8 * b)) & 255 for b in range(4)], -1).reshape(n, 4 * W) \
        .to(torch.uint8)


def _unpack_int4(b: torch.Tensor, r1: int) -> torch.Tensor:
    n = b.shape[0]
    W = (r1 + 7) // 8
    by = b[:, :4 * W].to(torch.int64).reshape(n, W, 4)
    words = by[..., 0] | (by[..., 1] << 8) | (by[..., 2] << 16) | (by[..., 3] << 24)
    nib = (words.unsqueeze(-1) >> _NIB_SHIFT.to(b.device)) & 15
    nib = nib.reshape(n, 8 * W)[:, :r1]
    return torch.where(nib >= 8, nib - 16, nib).to(torch.int8)


def pack_k_slots(lay: TTKLayout, coeff_q: torch.Tensor, coeff_scale, resid) -> torch.Tensor:
    """`[n, k_slot_bytes]` uint8 K slots from coefficients `[n, r1]` int8, their ruler `[n]`
    fp16 and the residual row store over H*n rows (reference layout.py:161-193). Padding bytes
    are zero. In this library's own modes `coeff_q` is fp16 `[n, r1]` (qbits 16, no
    `coeff_scale`) or int8 `[n, r1]` in [-7, 7] with fp16 group scales `[n, ceil(r1/32)]`
    (qbits 4)."""
    n = coeff_q.shape[0]
    pb = packed_row_bytes(lay.res_k, lay.res_bits)
    _check_rows(resid, lay, n, pb, "the residual")
    want = torch.float16 if lay.qbits == 16 else torch.int8
    if tuple(coeff_q.shape) != (n, lay.r1) or coeff_q.dtype != want:
        raise ValueError(f"coeff_q must be {want} [{n}, {lay.r1}], got {coeff_q.dtype} "
                         f"{tuple(coeff_q.shape)}")
    out = torch.zeros(n, lay.k_slot_bytes, dtype=torch.uint8, device=coeff_q.device)
    cb = lay.coeff_bytes
    if lay.qbits == 8:
        out[:, :cb] = coeff_q.contiguous().view(torch.uint8)
        out[:, cb:cb + 2] = (coeff_scale.to(torch.float16).contiguous().view(torch.uint8)
                             .reshape(n, 2))
    elif lay.qbits == 16:
        out[:, :cb] = coeff_q.contiguous().view(torch.uint8)
    else:
        if coeff_q.numel() and int(coeff_q.abs().amax()) > 7:
            raise ValueError("4-bit coefficients lie in [-7, 7]")
        if tuple(coeff_scale.shape) != (n, lay.coef_groups):
            raise ValueError(f"coeff_scale must be [{n}, {lay.coef_groups}] group scales")
        out[:, :cb] = _pack_int4(coeff_q)
        out[:, cb:lay.k_field] = (coeff_scale.to(torch.float16).contiguous().view(torch.uint8)
                                  .reshape(n, 2 * lay.coef_groups))
    _put_rows(_head_rows(out, lay.k_field, lay.H, lay.k_row_bytes), resid.bitmap, resid.packed,
              resid.scale, n, lay.H, lay.d // 8, pb)
    return out


def coefficient_values(lay: TTKLayout, coeff_q: torch.Tensor, coeff_scale) -> torch.Tensor:
    """The fp32 coefficients `[n, r1]` a slot's coefficient field stands for (exact): cq * ruler
    (int8), the fp16 values, or q * group scale (4-bit)."""
    if lay.qbits == 8:
        return coeff_q.to(torch.float32) * coeff_scale.to(torch.float32).reshape(-1, 1)
    if lay.qbits == 16:
        return coeff_q.to(torch.float32)
    s = coeff_scale.to(torch.float32).repeat_interleave(32, dim=1)[:, :lay.r1]
    return coeff_q.to(torch.float32) * s


def unpack_k_slots(lay: TTKLayout, slots: torch.Tensor):
    """Inverse of `pack_k_slots` (reference layout.py:196-219):
    `(coeff_q [n, r1] int8, coeff_scale [n] fp16, (bitmap, packed, scale))`, the residual rows in
    (head, token) order; in the fp16 / 4-bit modes the coefficient fields `pack_k_slots` takes."""
    n = slots.shape[0]
    if slots.dtype != torch.uint8 or slots.dim() != 2 or slots.shape[1] < lay.k_slot_bytes:
        raise ValueError(f"K slots must be uint8 [n, >= {lay.k_slot_bytes}]")
    cb = lay.coeff_bytes
    if lay.qbits == 8:
        coeff_q = slots[:, :cb].contiguous().view(torch.int8)
        coeff_scale = slots[:, cb:cb + 2].contiguous().view(torch.float16).reshape(n)
    elif lay.qbits == 16:
        coeff_q = slots[:, :cb].contiguous().view(torch.float16)
        coeff_scale = None
    else:
        coeff_q = _unpack_int4(slots[:, :cb], lay.r1)
        coeff_scale = slots[:, cb:lay.k_field].contiguous().view(torch.float16)
    rows = _take_rows(_head_rows(slots, lay.k_field, lay.H, lay.k_row_bytes), n, lay.H,
                      lay.d // 8, packed_row_bytes(lay.res_k, lay.res_bits))
    return coeff_q, coeff_scale, rows


def pack_v_slots(lay: TTKLayout, rows) -> torch.Tensor:
    """`[n, v_slot_bytes]` uint8 V slots from a row store over H*n rows (reference
    layout.py:222-239). Padding bytes are zero."""
    if int(rows.rows) % lay.H:
        raise ValueError(f"V store holds {rows.rows} rows, not a multiple of H={lay.H}")
    n = int(rows.rows) // lay.H
    pb = packed_row_bytes(lay.v_lanes, lay.v_bits)
    _check_rows(rows, lay, n, pb, "the V store")
    out = torch.zeros(n, lay.v_slot_bytes, dtype=torch.uint8, device=rows.bitmap.device)
    _put_rows(_head_rows(out, 0, lay.H, lay.v_row_bytes), rows.bitmap, rows.packed, rows.scale,
              n, lay.H, lay.d // 8, pb)
    return out


def unpack_v_slots(lay: TTKLayout, slots: torch.Tensor):
    """Inverse of `pack_v_slots` (reference layout.py:242-261): `(bitmap, packed, scale)` over
    H*n rows in (head, token) order."""
    if slots.dtype != torch.uint8 or slots.dim() != 2 or slots.shape[1] < lay.v_slot_bytes:
        raise ValueError(f"V slots must be uint8 [n, >= {lay.v_slot_bytes}]")
    return _take_rows(_head_rows(slots, 0, lay.H, lay.v_row_bytes), slots.shape[0], lay.H,
                      lay.d // 8, packed_row_bytes(lay.v_lanes, lay.v_bits))
