"""The write half: raw K and V of new tokens into packed slots.

Two phases, as in the reference (vllm_ttkv/encode.py:1-36):
  * a request's FIRST chunk is fitted -- TT-SVD of the [n, d, H] key block, tokens first, capped
    at the layer's rank budget and zero-padded to it (`fit_into_budget`, encode.py:257-298). The
    fit runs on the device through torch's linear algebra (rocSOLVER on ROCm); it happens once
    per request and layer and its bits are LAPACK-dependent, as they are in the reference.
  * every later token is projected onto that frozen decoder and packed by the HIP write kernel
    (`kernels.write_paged`, K3), which also packs the first chunk from the fit's coefficients.

`KDecoder` keeps the decoder and its pseudo-inverse (encode.py:178-211).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .layout import TTKLayout


def _ruler(x: torch.Tensor, divisor: int) -> torch.Tensor:
    """`x / divisor` as the reference's CUDA store computes it: a multiply by the fp32
    reciprocal (select_triton.py:76-84)."""
    inv = torch.tensor(1.0 / divisor, dtype=torch.float32).item()
    return x * inv


class KDecoder:
    """A request's frozen decoder `[r1, H*d]` fp32 and its cached pseudo-inverse `[H*d, r1]`."""

    __slots__ = ("decoder_f", "_pinv")

    def __init__(self, decoder_f: torch.Tensor):
        if decoder_f.dim() != 2:
            raise ValueError(f"a decoder is [r1, H*d]; got {tuple(decoder_f.shape)}")
        self.decoder_f = decoder_f.to(torch.float32).contiguous()
        self._pinv = None

    @property
    def pinv(self) -> torch.Tensor:
        if self._pinv is None:
            self._pinv = torch.linalg.pinv(self.decoder_f).contiguous()
        return self._pinv


@dataclass
class FittedK:
    """A fitted first chunk: int8 coefficients [n, r1], their fp32 ruler [n] (the residual is
    computed against the fp32 ruler and the fp16 one is stored, encode.py:328-336), the padded
    decoder, and the natural rank before padding."""

    coeff_q: torch.Tensor
    coeff_scale: torch.Tensor
    decoder: KDecoder
    fitted_rank: int
    budget: int


def _tt_svd(X: torch.Tensor, tol: float, max_rank: int | None):
    """Energy-truncated TT-SVD (codec/ttkv_codec.py:78-109)."""
    dims = list(X.shape)
    rest = X.reshape(dims[0], -1)
    cores, r_prev = [], 1
    for k in range(len(dims) - 1):
        M = rest.reshape(r_prev * dims[k], -1)
        U, S, Vh = torch.linalg.svd(M, full_matrices=False)
        e = S.pow(2)
        tail = torch.flip(torch.cumsum(torch.flip(e, [0]), 0), [0]) / (e.sum() + 1e-30)
        hit = torch.nonzero(tail <= tol ** 2, as_tuple=False)
        r = int(hit[0].item()) + 1 if hit.numel() else int(S.numel())
        r = max(1, min(r, int(S.numel())))
        if max_rank is not None:
            r = max(1, min(r, max_rank))
        cores.append(U[:, :r].reshape(r_prev, dims[k], r))
        rest = (S[:r].unsqueeze(1) * Vh[:r, :]).reshape(r, *dims[k + 1:])
        r_prev = r
    cores.append(rest.reshape(r_prev, dims[-1], 1))
    return cores


def _quant_core(c: torch.Tensor, qbits: int) -> torch.Tensor:
    """Per-row symmetric quantise-dequantise (ttkv_codec.py:142-163, per-token rows for [1,n,r])."""
    q = 2 ** (qbits - 1) - 1
    rows = int(c.shape[1]) if int(c.shape[0]) == 1 else int(c.shape[0])
    M = c.reshape(rows, -1)
    s = _ruler(M.abs().amax(1, keepdim=True).clamp(min=1e-12), q)
    return (torch.clamp(torch.round(M / s), -q, q) * s).reshape(c.shape)


def fit_into_budget(K: torch.Tensor, lay: TTKLayout, cfg: dict) -> FittedK:
    """First chunk: K [H, n, d] raw -> FittedK at the layout's rank budget (encode.py:257-298 /
    ttkv_packed_cache.py:337-375)."""
    H, n, d = K.shape
    if (H, d) != (lay.H, lay.d):
        raise ValueError(f"K is [H={H}, n={n}, d={d}] but the layout is for H={lay.H}, d={lay.d}")
    if K.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError(f"raw keys arrived as {K.dtype}")
    K = K.to(torch.float32)
    qm = 2 ** (lay.qbits - 1) - 1
    cores = _tt_svd(K.permute(1, 2, 0).contiguous(), cfg["tols"], lay.r1)   # [n, d, H]
    r1 = int(cores[0].shape[2])
    c = cores[0].reshape(n, r1)
    cs = _ruler(c.abs().amax(1, keepdim=True), qm)
    cs = torch.where(cs == 0, torch.ones_like(cs), cs)
    cq = torch.clamp(torch.round(c / cs), -(qm + 1), qm).to(torch.int8)
    g2 = _quant_core(cores[1], lay.qbits)
    g3 = _quant_core(cores[2], lay.qbits)
    dec = torch.einsum("ajb,bh->ahj", g2, g3[:, :, 0]).reshape(r1, H * d)
    rmax = dec.abs().amax(1, keepdim=True)
    sc = _ruler(torch.where(rmax == 0, torch.ones_like(rmax), rmax), qm)
    dec_q = torch.clamp(torch.round(dec / sc), -(qm + 1), qm)
    dec_f = dec_q * sc.to(torch.float16).to(torch.float32)          # int8 * fp16 row ruler
    coeff_q = torch.zeros(n, lay.r1, dtype=torch.int8, device=K.device)
    coeff_q[:, :r1] = cq
    padded = torch.zeros(lay.r1, H * d, dtype=torch.float32, device=K.device)
    padded[:r1] = dec_f
    return FittedK(coeff_q=coeff_q, coeff_scale=cs.reshape(n), decoder=KDecoder(padded),
                   fitted_rank=r1, budget=lay.r1)
