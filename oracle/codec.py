"""Bit format and TT-SVD fit, restated from the reference codec (TEST INFRASTRUCTURE ONLY).

Reference: `codec/ttkv_packed_cache.py:50-100` (code streams), `:138-167, 234-241` (bitmaps),
`:170-183` (`_quant_rows`, `_topk_mask`), `:193-271` (`PackedRows.build/materialise`),
`:337-385` (`build_k_layer`, `build_v_layer`); `codec/ttkv_codec.py:78-109` (`tt_svd`),
`:142-163` (`quant_cores`), `:272-298` (`CONFIGS`).

RULER ROUNDING (`ruler_mode`). The reference writes every ruler as `rmax / (2**(bits-1) - 1)`, a
tensor divided by a Python scalar. torch on CUDA evaluates that as a multiply by the fp32
reciprocal, torch on CPU as a correctly rounded division (checked in
`tests/test_oracle_codec.py::test_torch_scalar_division_semantics`). The shipped store -- the one
the reference's fused write reproduces byte for byte (`vllm_ttkv/select_triton.py:76-84, 119-120,
195-201`) -- is the CUDA one, so `ruler_mode="gpu"` (reciprocal multiply) is the default and is
what the HIP write kernel implements. `ruler_mode="cpu"` is what the same Python computes on a CPU.

TIES in the top-k lane selection follow the reference's fused kernel: every lane strictly above
the k-th largest magnitude, then the lowest-index lanes equal to it (`select_triton.py:181-193`).
`torch.topk` documents no tie order; on tie-free rows the two select the same set.
"""
from __future__ import annotations

import numpy as np
import torch

D = 128

# ttkv_codec.py:272-298. `tols` is the fit's dropped-energy tolerance; `k_lanes` is the V lane
# count (absolute), `res_frac` the K residual lane FRACTION of d.
CONFIGS = {
    "safe": dict(tols=0.20, qbits=8, res_frac=0.633, res_bits=3, k_lanes=81, vbits=3),
    "tight": dict(tols=0.20, qbits=8, res_frac=0.25, res_bits=3, k_lanes=45, vbits=3),
    "campaign4x": dict(tols=0.20, qbits=8, res_frac=0.50, res_bits=4, k_lanes=64, vbits=4),
}


def inv_ruler(bits: int) -> float:
    """fp32(1 / (2**(bits-1) - 1)): the reciprocal torch-CUDA multiplies by
    (select_triton.py:119-120)."""
    return float(np.float32(1.0 / (2 ** (bits - 1) - 1)))


def ruler_div(x: torch.Tensor, divisor: int, ruler_mode: str) -> torch.Tensor:
    """`x / divisor` for a Python-int divisor, as the reference's platform evaluates it."""
    if ruler_mode == "gpu":
        return x * torch.tensor(float(np.float32(1.0 / divisor)), dtype=torch.float32)
    if ruler_mode == "cpu":
        return x / divisor
    raise ValueError(f"ruler_mode {ruler_mode!r}")


# ------------------------------------------------------------------ code streams and bitmaps
def pack_bits_rows(vals: torch.Tensor, bits: int) -> torch.Tensor:
    """ttkv_packed_cache.py:50-66. [rows,k] ints < 2**bits -> uint8 [rows, ceil(k*bits/8)],
    MSB-first, one stream per row, each row padded with zero bits to whole bytes."""
    v = vals.to(torch.int64).numpy()
    rows, k = v.shape
    sh = np.arange(bits - 1, -1, -1)
    planes = ((v[:, :, None] >> sh) & 1).astype(np.uint8).reshape(rows, k * bits)
    return torch.from_numpy(np.packbits(planes, axis=1, bitorder="big")).contiguous()


def unpack_bits_rows(packed: torch.Tensor, k: int, bits: int) -> torch.Tensor:
    """ttkv_packed_cache.py:69-100. uint8 [rows,B] -> int32 [rows,k]."""
    p = packed.numpy()
    rows = p.shape[0]
    planes = np.unpackbits(p, axis=1, bitorder="big")[:, :k * bits].reshape(rows, k, bits)
    w = (1 << np.arange(bits - 1, -1, -1)).astype(np.int32)
    return torch.from_numpy((planes.astype(np.int32) * w).sum(-1).astype(np.int32))


def pack_mask(mask: torch.Tensor) -> torch.Tensor:
    """ttkv_packed_cache.py:234-241. bool [rows,d] -> uint8 [rows,d//8]; lane j -> byte j>>3,
    bit 7-(j&7)."""
    return torch.from_numpy(np.packbits(mask.numpy().astype(np.uint8), axis=1,
                                        bitorder="big")).contiguous()


def unpack_bitmap_rows(bitmap: torch.Tensor, d: int) -> torch.Tensor:
    """ttkv_packed_cache.py:138-167."""
    return torch.from_numpy(np.unpackbits(bitmap.numpy(), axis=1, bitorder="big")[:, :d]
                            .astype(bool))


def topk_mask(M: torch.Tensor, k: int) -> torch.Tensor:
    """ttkv_packed_cache.py:179-183 with the reference fused kernel's tie rule
    (select_triton.py:181-193): exactly k lanes per row."""
    a = M.abs()
    t = torch.sort(a, dim=1, descending=True).values[:, k - 1:k]           # k-th largest
    above = a > t
    tie = a == t
    need = k - above.sum(1, keepdim=True)
    sel = above | (tie & (torch.cumsum(tie.to(torch.int64), 1) <= need))
    return sel


# ------------------------------------------------------------------ per-row container
def packed_rows_build(X: torch.Tensor, mask: torch.Tensor, bits: int, k: int,
                      ruler_mode: str = "gpu"):
    """ttkv_packed_cache.py:203-231. X [rows,d] float, mask with exactly k per row ->
    (bitmap u8 [rows,d/8], packed u8 [rows,ceil(k*bits/8)], scale fp16 [rows])."""
    X = X.to(torch.float32)
    rows = X.shape[0]
    off = 2 ** (bits - 1)
    vals = torch.where(mask, X, torch.zeros_like(X))
    rmax = vals.abs().amax(1, keepdim=True)
    sc = ruler_div(torch.where(rmax == 0, torch.ones_like(rmax), rmax), off - 1, ruler_mode)
    q = torch.clamp(torch.round(vals / sc), -off, off - 1)
    q = torch.where(mask, q, torch.zeros_like(q)) + off
    codes = q[mask].reshape(rows, k).to(torch.int64)
    return pack_mask(mask), pack_bits_rows(codes, bits), sc.to(torch.float16).reshape(rows)


def packed_rows_materialise(bitmap, packed, scale, d: int, k: int, bits: int) -> torch.Tensor:
    """ttkv_packed_cache.py:247-271 -> dense fp32 [rows,d]."""
    rows = bitmap.shape[0]
    mask = unpack_bitmap_rows(bitmap, d)
    vals = (unpack_bits_rows(packed, k, bits) - 2 ** (bits - 1)).to(torch.float32)
    vals = vals * scale.to(torch.float32).unsqueeze(1)
    o = torch.zeros(rows * d, dtype=torch.float32)
    o[mask.reshape(-1)] = vals.reshape(-1)
    return o.reshape(rows, d)


def build_rows(X: torch.Tensor, k: int, bits: int, ruler_mode: str = "gpu"):
    """Top-k magnitude selection then `packed_rows_build` (build_v_layer / residual path)."""
    return packed_rows_build(X, topk_mask(X.to(torch.float32), k), bits, k, ruler_mode)


def quant_rows(M: torch.Tensor, qbits: int, ruler_mode: str = "gpu"):
    """ttkv_packed_cache.py:170-176 -> (int8 [rows,d], fp16 scale [rows])."""
    qm = 2 ** (qbits - 1) - 1
    rmax = M.abs().amax(1, keepdim=True)
    sc = ruler_div(torch.where(rmax == 0, torch.ones_like(rmax), rmax), qm, ruler_mode)
    q = torch.clamp(torch.round(M / sc), -(qm + 1), qm).to(torch.int8)
    return q, sc.to(torch.float16).reshape(-1)


# ------------------------------------------------------------------ the fit (LAPACK-dependent)
def tt_svd(X: torch.Tensor, tol: float, max_rank=None):
    """ttkv_codec.py:78-109. Energy-truncated TT-SVD. Bits depend on LAPACK; with the CPU torch
    the reference ran on they match its output exactly (tests/test_golden.py)."""
    dims = list(X.shape)
    rest = X.reshape(dims[0], -1).contiguous()
    cores, ranks, r_prev = [], [], 1
    for k in range(len(dims) - 1):
        M = rest.reshape(r_prev * dims[k], -1).contiguous()
        U, S, Vh = torch.linalg.svd(M, full_matrices=False)
        e = S.pow(2)
        tail = torch.flip(torch.cumsum(torch.flip(e, [0]), 0), [0]) / (e.sum() + 1e-30)
        hit = torch.nonzero(tail <= tol ** 2, as_tuple=False)
        r = int(hit[0].item()) + 1 if hit.numel() else int(S.numel())
        r = max(1, min(r, int(S.numel())))
        if max_rank is not None:
            r = max(1, min(r, max_rank))
        ranks.append(r)
        cores.append(U[:, :r].reshape(r_prev, dims[k], r).contiguous())
        rest = (S[:r].unsqueeze(1) * Vh[:r, :]).reshape(r, *dims[k + 1:]).contiguous()
        r_prev = r
    cores.append(rest.reshape(r_prev, dims[-1], 1).contiguous())
    ranks.append(1)
    return cores, ranks


def quant_cores(cores, qbits: int, ruler_mode: str = "gpu"):
    """ttkv_codec.py:121-163 with PER_TOKEN_CORE_RULER=True."""
    q = 2 ** (qbits - 1) - 1
    out = []
    for c in cores:
        rows = int(c.shape[1]) if int(c.shape[0]) == 1 else int(c.shape[0])
        M = c.reshape(rows, -1)
        s = ruler_div(M.abs().amax(1, keepdim=True).clamp(min=1e-12), q, ruler_mode)
        out.append((torch.clamp(torch.round(M / s), -q, q) * s).reshape(c.shape).contiguous())
    return out


def build_k_layer(K: torch.Tensor, tol: float, qbits: int, res_frac: float, res_bits: int,
                  max_rank=None, ruler_mode: str = "gpu"):
    """ttkv_packed_cache.py:337-375. K [H,n,d] -> dict(coeff_q [n,r1] i8, coeff_scale [n] f16,
    dec_q [r1,H*d] i8, dec_scale [r1] f16, decoder_f [r1,H*d] f32, resid (bm,pk,sc), r1, res_k)."""
    H, n, dd = K.shape
    K = K.to(torch.float32)
    cores, _ = tt_svd(K.permute(1, 2, 0).contiguous(), tol, max_rank)     # [n, d, H], tokens first
    r1 = int(cores[0].shape[2])
    qm = 2 ** (qbits - 1) - 1
    c = cores[0].reshape(n, r1)
    cscale = ruler_div(c.abs().amax(1, keepdim=True), qm, ruler_mode)
    cscale = torch.where(cscale == 0, torch.ones_like(cscale), cscale)
    cq = torch.clamp(torch.round(c / cscale), -(qm + 1), qm).to(torch.int8)
    qc = quant_cores(cores[1:], qbits, ruler_mode)
    dec = torch.einsum("ajb,bh->ahj", qc[0], qc[1][:, :, 0]).reshape(r1, H * dd).contiguous()
    dec_q, dec_scale = quant_rows(dec, qbits, ruler_mode)
    dec_f = dec_q.to(torch.float32) * dec_scale.to(torch.float32).unsqueeze(1)
    kflat = (cq.to(torch.float32) * cscale) @ dec_f                       # [n, H*d], m = h*d + j
    kr = max(int(dd * res_frac), 1)
    Kd = kflat.reshape(n, H, dd).permute(1, 0, 2)
    R = (K - Kd).reshape(H * n, dd)
    resid = build_rows(R, kr, res_bits, ruler_mode)
    return dict(coeff_q=cq, coeff_scale=cscale.to(torch.float16).reshape(n), dec_q=dec_q,
                dec_scale=dec_scale, decoder_f=dec_f, resid=resid, r1=r1, res_k=kr)


def build_v_layer(V: torch.Tensor, k_lanes: int, bits: int, ruler_mode: str = "gpu"):
    """ttkv_packed_cache.py:378-385. V [H,n,d] -> (bitmap, packed, scale) over H*n rows."""
    H, n, dd = V.shape
    return build_rows(V.reshape(H * n, dd).to(torch.float32), k_lanes, bits, ruler_mode)
