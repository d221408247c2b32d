"""torch-facing container-layout reads over the libttkv_hip C ABI: the drop-in for the codec's
fused container kernels (`codec/ttkv_cuda.py` `krt` :169-257 and `v_out` :144-166; CUDA bodies in
`codec/ttkv_kernels.cu`).

Same call shapes and argument meaning as the codec's launchers: a single sequence passes
`[HQ, HD]` queries / `[HQ, n]` weights and gets 2-D results back; a pooled batch passes `[B, ...]`.
Rows (the K residual or V) are any object with `bitmap`, `packed`, `scale` and `bits` (the codec's
`PackedRows`, or `PackedRows` here). Launches go on torch's current stream; there is no CPU path.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from . import _hip


class PackedRows(NamedTuple):
    """bitmap [rows, d/8] u8, packed [rows, PB] u8 (MSB-first codes of the set lanes), scale
    [rows] (fp16 or fp32), bits per code (ttkv_packed_cache.py:193-271)."""
    bitmap: torch.Tensor
    packed: torch.Tensor
    scale: torch.Tensor
    bits: int


def _rows(rows, n_rows: int, what: str):
    bm = rows.bitmap.contiguous()
    pk = rows.packed.contiguous()
    sc = rows.scale.to(torch.float32).reshape(-1).contiguous()
    if bm.dtype != torch.uint8 or pk.dtype != torch.uint8:
        raise ValueError(f"{what}: bitmap and packed must be uint8")
    if bm.shape[0] != n_rows or pk.shape[0] != n_rows or sc.numel() != n_rows:
        raise ValueError(f"{what} has {bm.shape[0]} rows, expected B*H*n = {n_rows} "
                         f"(slab order b*(H*n) + h*n + i)")
    if bm.shape[1] != 16:
        raise ValueError(f"{what}: bitmap rows must be d/8 = 16 bytes")
    return bm, pk, sc, int(pk.shape[1]), int(rows.bits)


def krt(coeff_q, coeff_scale, dec_q, dec_scale, resid, cos, sin, q, n, HQ, G, HD, mode=7):
    """s [HQ, n] (or [B, HQ, n]) fp32: post-RoPE scores, UNSCALED, straight from a pre-RoPE
    container (see `ttkv_container_krt` in include/ttkv_hip.h).

    coeff_q [B*n, r1] int8 (row b*n + i), coeff_scale [B*n]; dec_q [r1, H*HD] int8 (shared) or
    [B, r1, H*HD] with dec_scale [r1] / [B, r1] (the decoder is converted to fp32 here, as the
    codec's launcher does); resid: rows of the K residual or None; cos / sin [n, HD] fp32 at
    absolute positions, halves duplicated as rotate-half tables are (only columns [0, HD/2) are
    read, as the codec kernel does); q [HQ, HD] or [B, HQ, HD] fp32 post-RoPE."""
    if mode != 7:
        raise NotImplementedError("only the full computation (mode 7) is built; the codec's "
                                  "partial modes exist for timing decomposition")
    if q.dtype != torch.float32:
        raise ValueError("q must be fp32")
    two_d = q.dim() == 2
    q3 = (q.unsqueeze(0) if two_d else q).contiguous()
    if q3.dim() != 3 or q3.shape[1] != HQ or q3.shape[2] != HD:
        raise ValueError(f"krt takes [B, HQ, HD] or [HQ, HD], got {tuple(q.shape)}")
    B = int(q3.shape[0])
    if HQ % G:
        raise ValueError(f"HQ={HQ} is not a multiple of G={G}")
    H = HQ // G
    if coeff_q.dtype != torch.int8 or dec_q.dtype != torch.int8:
        raise ValueError("coeff_q / dec_q are int8")
    if int(coeff_q.shape[0]) != B * n:
        raise ValueError(f"coeff_q has {int(coeff_q.shape[0])} rows, expected B*n = {B * n} "
                         f"(row = b*n + i)")
    r1 = int(coeff_q.shape[1])
    if dec_q.dim() == 2:
        dec_f = dec_q.to(torch.float32) * dec_scale.to(torch.float32).reshape(-1, 1)
        per_seq = 0
    else:
        if int(dec_q.shape[0]) != B:
            raise ValueError(f"decoder has {int(dec_q.shape[0])} sequences, expected {B}")
        dec_f = dec_q.to(torch.float32) * dec_scale.to(torch.float32).unsqueeze(-1)
        per_seq = 1
    if tuple(dec_f.shape[-2:]) != (r1, H * HD):
        raise ValueError(f"decoder is {tuple(dec_f.shape)}, expected [..., {r1}, {H * HD}]")
    dec_f = dec_f.contiguous()
    cq = coeff_q.contiguous()
    cs = coeff_scale.to(torch.float32).reshape(-1).contiguous()
    for t, nm in ((cos, "cos"), (sin, "sin")):
        if t.dtype != torch.float32 or tuple(t.shape) != (n, HD):
            raise ValueError(f"{nm} must be fp32 [n={n}, {HD}], got {tuple(t.shape)} {t.dtype}")
    cos, sin = cos.contiguous(), sin.contiguous()
    if resid is None:
        bm = pk = sc = None
        pb, bits = 1, 3
    else:
        bm, pk, sc, pb, bits = _rows(resid, B * H * n, "residual")
    s = torch.empty(B, HQ, n, dtype=torch.float32, device=q.device)
    rc = _hip.lib().ttkv_container_krt(
        H, HQ, HD, B, n, r1, cq.data_ptr(), cs.data_ptr(), dec_f.data_ptr(), per_seq,
        _hip.ptr(bm), _hip.ptr(pk), _hip.ptr(sc), pb, bits, cos.data_ptr(), sin.data_ptr(),
        q3.data_ptr(), s.data_ptr(), _hip.stream_ptr(q.device))
    _hip.check(rc, "ttkv_container_krt")
    return s[0] if two_d else s


def v_out(p, rows, n, HQ, G, HD):
    """o [HQ, HD] (or [B, HQ, HD]) fp32 = sum_i p[., p, i] * V[h(p), i] from the container's V rows
    (see `ttkv_container_v_out`). `p` may be a slice whose token axis is contiguous (its head and
    batch strides are passed through); `o` is zero-filled here because the launch accumulates tile
    partials with atomic adds."""
    if p.dtype != torch.float32 or p.stride(-1) != 1:
        raise ValueError("p must be fp32 and contiguous along the token axis")
    two_d = p.dim() == 2
    p3 = p.unsqueeze(0) if two_d else p
    B = int(p3.shape[0])
    if p3.shape[1] != HQ or p3.shape[2] < n:
        raise ValueError(f"p is {tuple(p.shape)}; expected [B, {HQ}, >= {n}]")
    if HQ % G:
        raise ValueError(f"HQ={HQ} is not a multiple of G={G}")
    H = HQ // G
    bm, pk, sc, pb, bits = _rows(rows, B * H * n, "V rows")
    o = torch.zeros(B, HQ, HD, dtype=torch.float32, device=p.device)
    rc = _hip.lib().ttkv_container_v_out(
        H, HQ, HD, B, n, p3.data_ptr(), p3.stride(1), p3.stride(0), bm.data_ptr(), pk.data_ptr(),
        sc.data_ptr(), pb, bits, o.data_ptr(), _hip.stream_ptr(p.device))
    _hip.check(rc, "ttkv_container_v_out")
    return o[0] if two_d else o
