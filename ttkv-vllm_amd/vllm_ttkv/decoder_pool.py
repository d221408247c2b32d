"""The decoder pool's storage form: the codec's int8 decoder, laid out for the kernels.

The reference stores a fitted decoder as `dec_q [r1, H*d]` int8 plus one fp16 ruler per rank
(`dec_scale [r1]`), and reads it as `decoder_f = dec_q * dec_scale` in fp32
(codec/ttkv_packed_cache.py:284-293; vllm_ttkv/encode.py:257-298 produces it). The pool keeps
that form, transposed so that each decoder column's ranks are contiguous:

    q     [slots, H*d, R] int8      q[s, j, a] = dec_q of rank a, column j
    scale [slots, R]      fp32      the rank's ruler
    R = decoder_ranks(r1); ranks a >= r1 hold 0 with ruler 0

`float(q) * scale` is the reference's fp32 decoder value exactly: an 8-bit integer times an
11-bit fp16 ruler needs 19 of fp32's 24 significand bits. The pool is 1 + 4/(H*d) bytes per
decoder value instead of 4.
"""
from __future__ import annotations

from typing import NamedTuple

import torch


def decoder_ranks(r1: int) -> int:
    """Ranks R a pool column holds: 64 for r1 <= 64, 128 for r1 <= 128, else r1 rounded up to
    64 (the kernels read a column's ranks in whole 8-, 16- and 64-byte groups;
    `ttkv_decoder_ranks` in the C ABI returns the same)."""
    r1 = int(r1)
    if r1 <= 0:
        raise ValueError(f"r1 must be positive, got {r1}")
    return 64 if r1 <= 64 else 128 if r1 <= 128 else (r1 + 63) // 64 * 64


class DecoderPool(NamedTuple):
    """Decoders in the kernels' layout: `q [..., H*d, R]` int8 and `scale [..., R]` fp32."""

    q: torch.Tensor
    scale: torch.Tensor

    @property
    def slots(self) -> int:
        return int(self.q.shape[0])

    def slot(self, i: int) -> "DecoderPool":
        """Slot `i` of a pool (views)."""
        return DecoderPool(self.q[i], self.scale[i])


# The largest |q| of a codec row is qmax = 127 (encode.py:257-298 quantises each rank row by its
# own max / 127), so the ruler is max|row| / 127, exactly. Any other exact int8 form is found by
# trying the other largest magnitudes.
_QMAX_ORDER = (127, 128) + tuple(range(126, 0, -1))


def _exact_int8_rows(x: torch.Tensor):
    """Rows `x [n, k]` fp32 -> (q [n, k] fp32 holding integers in [-128, 127], s [n]) with
    q * s == x exactly (checked in float64, so the fp32 product is exact too); zero rows get
    s = 0. Raises ValueError when some row has no such form."""
    if not bool(torch.isfinite(x).all()):
        raise ValueError("the decoder holds non-finite values")
    # float64 throughout: the candidate ruler max|row| / m and the quotients are exact there
    # whenever the row has the form (fp32 division on the device need not round correctly)
    x64 = x.double()
    amax = x64.abs().amax(-1)
    q = torch.zeros_like(x64)
    s = torch.zeros_like(amax)
    todo = amax > 0
    for m in _QMAX_ORDER:
        if not bool(todo.any()):
            break
        sm = amax / m
        qm = torch.round(x64 / torch.where(todo, sm, torch.ones_like(sm)).unsqueeze(-1))
        ok = todo & (qm * sm.unsqueeze(-1) == x64).all(-1)
        ok &= (qm.amax(-1) <= 127) & (qm.amin(-1) >= -128) & (sm.float().double() == sm)
        q = torch.where(ok.unsqueeze(-1), qm, q)
        s = torch.where(ok, sm, s)
        todo &= ~ok
    if bool(todo.any()):
        bad = torch.nonzero(todo).flatten()[:4].tolist()
        raise ValueError(
            f"decoder rank row(s) {bad} are not int8 values times one ruler: the pool stores the "
            f"codec's int8 decoder (dec_q * dec_scale), which every fitted decoder is")
    return q.float(), s.float()


def pack_decoders(decoder_f: torch.Tensor) -> DecoderPool:
    """fp32 decoders `[r1, H*d]` or `[slots, r1, H*d]` -> their exact pool form (same leading
    shape, on the same device). Raises ValueError for a decoder that is not int8 x ruler."""
    if decoder_f.dtype != torch.float32:
        raise TypeError(f"decoder_f must be fp32, got {decoder_f.dtype}")
    if decoder_f.dim() not in (2, 3):
        raise ValueError(f"decoder_f is [r1, H*d] or [slots, r1, H*d]; got "
                         f"{tuple(decoder_f.shape)}")
    x = decoder_f.reshape(-1, *decoder_f.shape[-2:])
    S, r1, hd = x.shape
    R = decoder_ranks(r1)
    q, s = _exact_int8_rows(x.reshape(S * r1, hd))
    pq = torch.zeros(S, hd, R, dtype=torch.int8, device=x.device)
    ps = torch.zeros(S, R, dtype=torch.float32, device=x.device)
    pq[:, :, :r1] = q.reshape(S, r1, hd).transpose(1, 2).to(torch.int8)
    ps[:, :r1] = s.reshape(S, r1)
    if decoder_f.dim() == 2:
        return DecoderPool(pq[0], ps[0])
    return DecoderPool(pq, ps)


def from_codec(dec_q: torch.Tensor, dec_scale: torch.Tensor) -> DecoderPool:
    """The codec's own form (`dec_q [r1, H*d]` int8, `dec_scale [r1]` fp16 or fp32) -> the pool
    form of one decoder, with no search."""
    if dec_q.dtype != torch.int8 or dec_q.dim() != 2:
        raise ValueError(f"dec_q must be int8 [r1, H*d], got {dec_q.dtype} "
                         f"{tuple(dec_q.shape)}")
    r1, hd = dec_q.shape
    if tuple(dec_scale.shape) != (r1,):
        raise ValueError(f"dec_scale must be [{r1}], got {tuple(dec_scale.shape)}")
    R = decoder_ranks(r1)
    pq = torch.zeros(hd, R, dtype=torch.int8, device=dec_q.device)
    ps = torch.zeros(R, dtype=torch.float32, device=dec_q.device)
    pq[:, :r1] = dec_q.t()
    ps[:r1] = dec_scale.to(torch.float32)
    return DecoderPool(pq, ps)


def unpack_decoders(pool: DecoderPool, r1: int) -> torch.Tensor:
    """The fp32 decoders `[..., r1, H*d]` a pool holds (`float(q) * scale`, exact)."""
    q = pool.q[..., :r1].to(torch.float32).transpose(-1, -2)
    return q * pool.scale[..., :r1].unsqueeze(-1)


def empty_pool(slots: int, r1: int, H: int, d: int, device) -> DecoderPool:
    """A zero pool of `slots` decoders (every value 0)."""
    R = decoder_ranks(r1)
    return DecoderPool(torch.zeros(slots, H * d, R, dtype=torch.int8, device=device),
                       torch.zeros(slots, R, dtype=torch.float32, device=device))
