"""Container-layout reads, restated on the CPU (TEST INFRASTRUCTURE ONLY: imported by tests/, never
by the product path).

The codec's pooled container (codec/ttkv_packed_cache.py:337-385) holds one store as separate
arrays instead of slots: coeff_q [B*n, r1] int8, coeff_scale [B*n], a decoder, and per-(head, token)
rows (bitmap, packed codes, scale) in row order b*H*n + h*n + i. Its two fused readers
(codec/ttkv_kernels.cu `ttkv_krt` / `ttkv_v_out`, launched by codec/ttkv_cuda.py:144-257) compute

  krt   : s[b, p, i] = q[b, p] . RoPE_i(K_pre[b, h(p), i])          UNSCALED (ttkv_cuda.py:169-229)
          K_pre[b, h, i, j] = (cq[b*n+i] . cs[b*n+i]) @ decoder_f[:, h*d+j] + resid[b, h, i, j]
  v_out : o[b, p, :] = sum_i p[b, p, i] * V[b, h(p), i, :]           (ttkv_cuda.py:144-166)

with h(p) = p // (HQ // H), the residual / V rows materialised as (code - 2^(bits-1)) * scale on
the bitmap's set lanes (ttkv_packed_cache.py:247-271) and the rotation that of
`rope_apply` (ttkv_packed_cache.py:486-498) with cos / sin [n, d] at absolute positions. These are
the same formulas as reference.py:47-109 over slots; tests/test_oracle_container.py pins them to
the slot oracle (which the golden vectors pin) on containers packed into slots.
"""
from __future__ import annotations

import torch

from .codec import packed_rows_materialise
from .rope import rope_apply


def rows_dense(bitmap, packed, scale, B: int, H: int, n: int, d: int, k: int, bits: int,
               dtype=torch.float64) -> torch.Tensor:
    """Rows [B*H*n, ...] -> dense [B, H, n, d] (ttkv_packed_cache.py:247-271)."""
    m = packed_rows_materialise(bitmap, packed, scale, d, k, bits)
    return m.to(dtype).reshape(B, H, n, d)


def krt(coeff_q, coeff_scale, decoder_f, resid, cos, sin, q, n: int, H: int, d: int = 128,
        res_k: int | None = None, res_bits: int | None = None, dtype=torch.float64):
    """q [B, HQ, d] (or [HQ, d]) -> s [B, HQ, n] (or [HQ, n]), unscaled.

    decoder_f [r1, H*d] (shared) or [B, r1, H*d]; resid = (bitmap, packed, scale) or None."""
    two_d = q.dim() == 2
    q3 = (q.unsqueeze(0) if two_d else q).to(dtype)
    B, HQ, _ = q3.shape
    G = HQ // H
    r1 = coeff_q.shape[1]
    c = coeff_q.to(dtype) * coeff_scale.to(dtype).reshape(-1, 1)             # [B*n, r1]
    c = c.reshape(B, n, r1)
    dec = decoder_f.to(dtype)
    if dec.dim() == 2:
        dec = dec.unsqueeze(0).expand(B, -1, -1)
    K = torch.einsum("bia,bam->bim", c, dec).reshape(B, n, H, d).permute(0, 2, 1, 3)  # [B,H,n,d]
    if resid is not None:
        K = K + rows_dense(*resid, B, H, n, d, res_k, res_bits, dtype)
    Kp = rope_apply(K, cos.to(dtype), sin.to(dtype))                        # per-row angles
    s = torch.einsum("bpd,bpnd->bpn", q3, Kp[:, torch.arange(HQ) // G])
    return s[0] if two_d else s


def v_out(p, rows, n: int, H: int, d: int = 128, k: int | None = None, bits: int | None = None,
          dtype=torch.float64):
    """p [B, HQ, n] (or [HQ, n]) -> o [B, HQ, d] (or [HQ, d])."""
    two_d = p.dim() == 2
    p3 = (p.unsqueeze(0) if two_d else p).to(dtype)
    B, HQ, _ = p3.shape
    G = HQ // H
    V = rows_dense(*rows, B, H, n, d, k, bits, dtype)                       # [B, H, n, d]
    o = torch.einsum("bpn,bpnd->bpd", p3, V[:, torch.arange(HQ) // G])
    return o[0] if two_d else o
