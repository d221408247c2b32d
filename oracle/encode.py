"""Write path, restated from the reference (TEST INFRASTRUCTURE ONLY).

Reference: `vllm_ttkv/encode.py:257-298` (`fit_into_budget`), `:301-351` (`encode_frozen`),
`:431-443` (`encode_v`), `:446-508` (`check_slot_ids`, `write_slots`), `:582-603`
(`pack_and_write`, torch arm).

The frozen encode splits into three stages so a test can hand the oracle the HIP kernel's own
intermediates and demand bit-exact bytes from there on (the projection matmul's summation order
is implementation-defined on every platform, so bytes are pinned from the quantiser inputs on):
  project      c = M @ pinv                             (float; tolerance)
  quantise     cs = max|c| * fp32(1/127), cq = rint(c/cs)  (bit-exact given c)
  residual     R = K - (cq*cs) @ decoder_f              (float; tolerance)
  pack         select / quantise / bitmap / codes       (bit-exact given R)
"""
from __future__ import annotations

import torch

from . import codec
from .layout import Layout, pack_k_slots, pack_v_slots


def fit_into_budget(K: torch.Tensor, lay: Layout, cfg: dict, ruler_mode: str = "gpu"):
    """encode.py:257-298. K [H,n,d] raw -> fitted store zero-padded to lay.r1. The TT-SVD makes
    the result LAPACK-dependent; pinned by invariants and, on the CPU, bit-exactly against vectors
    the reference wrote (tests/golden/ref_encode_*.npz)."""
    H, n, d = K.shape
    kl = codec.build_k_layer(K, cfg["tols"], cfg["qbits"], cfg["res_frac"], cfg["res_bits"],
                             max_rank=lay.r1, ruler_mode=ruler_mode)
    r = kl["r1"]
    coeff_q = torch.zeros(n, lay.r1, dtype=torch.int8)
    coeff_q[:, :r] = kl["coeff_q"]
    dec = torch.zeros(lay.r1, H * d, dtype=torch.float32)
    dec[:r] = kl["decoder_f"]
    return dict(coeff_q=coeff_q, coeff_scale=kl["coeff_scale"], resid=kl["resid"],
                decoder_f=dec, fitted_rank=r)


def pinv(decoder_f: torch.Tensor) -> torch.Tensor:
    """encode.py:197-208: [r1, H*d] -> [H*d, r1]."""
    return torch.linalg.pinv(decoder_f.to(torch.float32))


def project(K: torch.Tensor, pinv_m: torch.Tensor) -> torch.Tensor:
    """encode.py:322-324. K [H,n,d] -> c [n,r1] = M @ pinv, M token-major with m = h*d + j."""
    H, n, d = K.shape
    return K.permute(1, 0, 2).reshape(n, H * d).to(torch.float32) @ pinv_m


def quantise_coeffs(c: torch.Tensor, qbits: int = 8, ruler_mode: str = "gpu"):
    """encode.py:328-332 -> (cq int8 [n,r1], cs fp32 [n,1]). Bit-exact given c."""
    qm = 2 ** (qbits - 1) - 1
    cs = codec.ruler_div(c.abs().amax(1, keepdim=True), qm, ruler_mode)
    cs = torch.where(cs == 0, torch.ones_like(cs), cs)
    cq = torch.clamp(torch.round(c / cs), -(qm + 1), qm)
    return cq.to(torch.int8), cs


def residual(K: torch.Tensor, cq: torch.Tensor, cs: torch.Tensor,
             decoder_f: torch.Tensor) -> torch.Tensor:
    """encode.py:334-336. R [H*n, d] (head, token) = K - (cq*cs_fp32) @ decoder_f."""
    H, n, d = K.shape
    kd = ((cq.to(torch.float32) * cs) @ decoder_f).reshape(n, H, d).permute(1, 0, 2)
    return (K.to(torch.float32) - kd).reshape(H * n, d)


def encode_frozen(K: torch.Tensor, decoder_f: torch.Tensor, lay: Layout, pinv_m=None,
                  ruler_mode: str = "gpu"):
    """encode.py:301-351. K [H,n,d] raw -> dict(coeff_q, coeff_scale fp16, c, R, resid)."""
    if decoder_f.shape[0] != lay.r1:
        raise ValueError("decoder rank != layout r1")
    pm = pinv(decoder_f) if pinv_m is None else pinv_m
    c = project(K, pm)
    cq, cs = quantise_coeffs(c, lay.qbits, ruler_mode)
    R = residual(K, cq, cs, decoder_f)
    resid = codec.build_rows(R, lay.res_k, lay.res_bits, ruler_mode)
    return dict(coeff_q=cq, coeff_scale=cs.to(torch.float16).reshape(-1), c=c, R=R, resid=resid)


def encode_frozen_mode(K: torch.Tensor, decoder_f: torch.Tensor, lay: Layout, pinv_m=None,
                       c=None):
    """The frozen write in this build's fp16 / 4-bit coefficient modes (`coef_modes`): c as
    `encode_frozen` projects it (or as given), quantised by the mode, and the residual against the
    stored values. -> dict(coeff_q, coeff_scale, values, c, R, resid) for `k_slots_from`."""
    from . import coef_modes
    if decoder_f.shape[0] != lay.r1:
        raise ValueError("decoder rank != layout r1")
    if c is None:
        c = project(K, pinv(decoder_f) if pinv_m is None else pinv_m)
    vals, q, s = coef_modes.quantise(c, lay.qbits)
    H, n, d = K.shape
    kd = (vals @ decoder_f.to(torch.float32)).reshape(n, H, d).permute(1, 0, 2)
    R = (K.to(torch.float32) - kd).reshape(H * n, d)
    resid = codec.build_rows(R, lay.res_k, lay.res_bits, "gpu")
    return dict(coeff_q=q, coeff_scale=s, values=vals, c=c, R=R, resid=resid)


def encode_v(V: torch.Tensor, lay: Layout, ruler_mode: str = "gpu"):
    """encode.py:431-443 -> (bitmap, packed, scale) over H*n rows; V in [H,n,d]."""
    return codec.build_v_layer(V.to(torch.float32), lay.v_lanes, lay.v_bits, ruler_mode)


def k_slots_from(lay: Layout, coeff_q, coeff_scale, resid) -> torch.Tensor:
    return pack_k_slots(lay, coeff_q, coeff_scale, *resid)


def v_slots_from(lay: Layout, vrows) -> torch.Tensor:
    return pack_v_slots(lay, *vrows)


def check_slot_ids(slot_ids: torch.Tensor, n_slots: int) -> None:
    """encode.py:446-468."""
    if slot_ids.numel() == 0:
        return
    lo, hi = int(slot_ids.min()), int(slot_ids.max())
    if lo < 0:
        raise RuntimeError(f"slot_mapping contains {lo} (PAD_SLOT_ID)")
    if hi >= n_slots:
        raise IndexError(f"slot {hi} is outside the cache, which holds {n_slots} slots")


def write_slots(flat: torch.Tensor, slot_ids: torch.Tensor, k_slots, v_slots, lay: Layout):
    """encode.py:471-508. flat [n_slots, W>=C] uint8, in place."""
    C = lay.compressed_bytes_per_token()
    check_slot_ids(slot_ids, flat.shape[0])
    flat[slot_ids.to(torch.long), :C] = torch.cat([k_slots, v_slots], dim=-1)
