"""The write half: raw K and V of new tokens into packed slots.

Two phases, as in the reference (vllm_ttkv/encode.py:1-36):
  * a request's FIRST chunk is fitted -- the energy-truncated tensor-train factorisation of the
    [n, d, H] key block, tokens first, capped at the layer's rank budget and zero-padded to it
    (`fit_into_budget`, encode.py:257-298). It runs on the device as GEMMs plus small dense
    factorisations (subspace iteration on a Gram matrix, see `_leading_factors`), once per
    request and layer; like the reference's SVD-based fit, its bits depend on the linear algebra
    underneath, and it is pinned by invariants (rank rule, zero padding, least squares).
  * every later token is projected onto that frozen decoder and packed by the HIP write kernel
    (`kernels.write_paged`, K3), which also packs the first chunk from the fit's coefficients.

`KDecoder` keeps the decoder and its pseudo-inverse (encode.py:178-211).
"""
from __future__ import annotations

from dataclasses import dataclass
import math

import torch

from .decoder_pool import DecoderPool, decoder_ranks, pack_decoders
from .layout import TTKLayout


def _ruler(x: torch.Tensor, divisor: int) -> torch.Tensor:
    """`x / divisor` as the reference's CUDA store computes it: a multiply by the fp32
    reciprocal (select_triton.py:76-84)."""
    inv = torch.tensor(1.0 / divisor, dtype=torch.float32).item()
    return x * inv


def _pinv_rows(D: torch.Tensor) -> torch.Tensor:
    """Moore-Penrose pseudo-inverse `[k, r]` of a wide float32 matrix D `[r, k]` (r <= k), as
    `torch.linalg.pinv(D)` defines it -- singular values at or below max(r, k) * eps(fp32) times
    the largest treated as zero -- computed from the r x r Gram matrix instead of an SVD of D:
    with D D^T = U diag(s^2) U^T, pinv(D) = D^T U diag(1 / s^2) U^T over the kept s. The Gram
    matrix is formed in float64 (its eigenvalues are the squared singular values, so float64
    keeps them to ~1e-8 relative) and solved by the host's LAPACK (~0.5 ms at r = 110, where the
    device SVD of D takes ~5 ms). Rows of D that are exactly zero (rank below the budget) get
    exactly zero columns."""
    r, k = D.shape
    nz = D.abs().amax(1) > 0
    out = torch.zeros(k, r, dtype=torch.float32, device=D.device)
    if not bool(nz.any()):
        return out
    Dn = D[nz].to(torch.float64)
    lam, U = torch.linalg.eigh((Dn @ Dn.T).cpu())
    cut = (max(r, k) * torch.finfo(torch.float32).eps * lam.max().clamp(min=0.0).sqrt()) ** 2
    inv = torch.where(lam > cut, 1.0 / lam, torch.zeros_like(lam))
    Ginv = ((U * inv) @ U.T).to(D.device)
    out[:, nz] = (Dn.T @ Ginv).to(torch.float32)
    return out


class KDecoder:
    """A request's frozen decoder `[r1, H*d]` fp32 and its cached pseudo-inverse `[H*d, r1]`
    (encode.py:198-208 uses `torch.linalg.pinv`; `_pinv_rows` computes the same matrix), plus
    its pool form (`packed`: the codec's int8 decoder as the kernels read it), given by the fit
    or derived exactly from `decoder_f` on first use."""

    __slots__ = ("decoder_f", "_pinv", "_packed")

    def __init__(self, decoder_f: torch.Tensor, packed: DecoderPool | None = None):
        if decoder_f.dim() != 2:
            raise ValueError(f"a decoder is [r1, H*d]; got {tuple(decoder_f.shape)}")
        self.decoder_f = decoder_f.to(torch.float32).contiguous()
        self._pinv = None
        self._packed = packed

    @property
    def packed(self) -> DecoderPool:
        if self._packed is None:
            self._packed = pack_decoders(self.decoder_f)
        return self._packed

    @property
    def pinv(self) -> torch.Tensor:
        if self._pinv is None:
            D = self.decoder_f
            self._pinv = (_pinv_rows(D) if D.shape[0] <= D.shape[1]
                          else torch.linalg.pinv(D)).contiguous()
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


# ---------------------------------------------------------------- the fit's factorisation
# The first-chunk fit is the reference's energy-truncated tensor-train decomposition of the
# [n, d, H] key block (codec/ttkv_codec.py:78-109): a rank-r1 factorisation of the n x (d*H)
# unfolding M, then of the (r1*d) x H remainder. Only the LEADING r1 singular triplets of M
# (r1 <= the layer's budget, 110) and its total energy are used, so no full SVD is computed. In
# float64, the smaller Gram matrix of M (M^T M, d*H = 1024 wide, or M M^T for a chunk of fewer
# tokens) is formed with one GEMM; randomized subspace iteration on it with a Rayleigh-Ritz step
# (Halko, Martinsson & Tropp, SIAM Review 53(2), 2011, sections 4.5 and 5) gives the leading
# eigenpairs, i.e. the leading singular values and vectors of M. Squaring the condition number is
# harmless here: the kept components lie within tol of the top of the spectrum and the arithmetic
# is float64. The rank follows the reference's energy rule from the leading spectrum and the
# exact total (the Gram trace). The second stage has only H columns and is solved through its
# H x H Gram matrix exactly. Singular vectors are defined up to sign; a sign flip of a component
# flips the coefficient column and the decoder row together and leaves the fitted keys unchanged.
# Each component's sign is fixed here so that the largest-magnitude entry of its left vector is
# positive, which makes the fit's signs the same on every device.

_OVERSAMPLE = 128     # extra subspace columns beyond the rank budget
_ITERS = 24           # multiplications by G: the error decays like (s_{r+p+1} / s_r)^(2 * iters)
_RANGE_SEED = 0x7E5   # fixed start-block seed: the fit is deterministic
_QR_SPREAD = 1e8      # largest diagonal spread of R accepted for a block of several multiplications
_MAX_STEP = 8         # multiplications between two Cholesky QRs at most


def _chol_qr_spread(Y: torch.Tensor):
    """Cholesky QR of Y with its status: (Y R^-1, spread of |diag R|, ok). The small Gram matrix
    Y^T Y (<= 238 x 238, float64) goes to the host, whose LAPACK factors it and inverts R; Y R^-1
    is then one GEMM on Y's device. At 1024 x 238 that takes 0.45 ms per QR where the device's
    potrf + triangular solve take 0.67 ms, with the same one host round trip (the status read)."""
    W = (Y.T @ Y).cpu()
    R, info = torch.linalg.cholesky_ex(W, upper=True)
    d = R.diagonal().abs()
    if int(info) != 0 or not float(d.min()) > 0.0:
        return None, float("inf"), False
    Ri = torch.linalg.solve_triangular(R, torch.eye(R.shape[0], dtype=R.dtype), upper=True)
    return Y @ Ri.to(Y.device), float(d.max() / d.min()), True
def _energy_rank(e: torch.Tensor, total: float, tol: float) -> int | None:
    """The reference's rank rule on a descending energy spectrum e (squared singular values):
    r = 1 + the first index i at which the energy of components i, i+1, ... is <= tol^2 of the
    total (codec/ttkv_codec.py:97-100). `e` may hold only the leading values: the energy from i on
    is the total minus the leading partial sum. None when no index of `e` qualifies."""
    before = torch.cumsum(e, 0) - e                      # energy of components < i
    tail = (total - before) / (total + 1e-30)
    hit = torch.nonzero(tail <= tol ** 2, as_tuple=False)
    return int(hit[0].item()) + 1 if hit.numel() else None


def _fix_signs(U: torch.Tensor, SVh: torch.Tensor):
    """Flip each component so the largest-magnitude entry of its column of U is positive."""
    pick = U.abs().argmax(0, keepdim=True)
    s = torch.where(torch.gather(U, 0, pick) < 0, -1.0, 1.0).to(U.dtype)   # [1, r]
    return U * s, SVh * s.T


def _nonzero(S: torch.Tensor) -> torch.Tensor:
    """Divisors for U = M V / S. The energy rule can keep one component of (numerically) zero
    energy -- the first one whose tail is below tol^2 -- whose left vector is arbitrary; dividing
    its rounding noise by ~0 would blow it up, so it gets a zero column instead (its decoder row
    is zero too: the fitted keys are the same)."""
    return torch.where(S > S[:1] * 1e-12, S, torch.full_like(S, float("inf")))


def _eigh_host(A: torch.Tensor):
    """Eigenpairs (ascending) of a small symmetric float64 matrix, solved by the host's LAPACK and
    returned on A's device. At the sizes used here (<= 238) one host solve takes ~2 ms where the
    device solver's tridiagonalisation and divide-and-conquer kernels take ~5 ms."""
    lam, V = torch.linalg.eigh(A.cpu())
    return lam.to(A.device), V.to(A.device)


def _leading_eigh(G: torch.Tensor, count: int):
    """Leading `count` eigenpairs (descending) of a symmetric positive semidefinite float64 G,
    from randomized subspace iteration with a Rayleigh-Ritz step; exact when `count` spans G.

    Only the block's span matters between steps, so G multiplies it several times between two
    Cholesky QRs as long as the block stays well conditioned: after each QR the spread of R's
    diagonal gives the growth per multiplication g, and the next block takes
    log(_QR_SPREAD) / log(g) multiplications (at most _MAX_STEP). A block whose factor comes out
    more spread than _QR_SPREAD (or whose factorisation fails) is redone one multiplication at a
    time. On the spectra of key blocks (g ~ 50-60) that is 4 multiplications per QR: 9 QRs
    instead of 26 for the same 24 multiplications and the same span to rounding (a spread of at
    most 10^8 leaves the block's smallest direction ~10^-8 of float64's precision lost). The final basis
    gets a second QR (CholeskyQR2: orthonormal to working precision). If a single-step
    factorisation meets a numerically rank-deficient block, the iteration is redone with
    Householder QR."""
    dim = G.shape[0]
    p = min(count + _OVERSAMPLE, dim)
    if p == dim:
        lam, V = _eigh_host(G)
        return lam.flip(0).clamp(min=0.0), V.flip(1)
    gen = torch.Generator(device=G.device)
    gen.manual_seed(_RANGE_SEED)
    Y0 = G @ torch.randn(dim, p, generator=gen, dtype=torch.float64, device=G.device)
    Q, spread, ok = _chol_qr_spread(Y0)
    done, step = 0, 1
    while ok and done < _ITERS:
        k = min(step, _ITERS - done)
        Y = Q
        for _ in range(k):
            Y = G @ Y
        Qn, spread, ok_n = _chol_qr_spread(Y)
        if k > 1 and (not ok_n or spread > _QR_SPREAD):
            step = 1                                   # redo this block one step at a time
            continue
        ok = ok_n
        if not ok:
            break
        Q, done = Qn, done + k
        g = max(spread ** (1.0 / k), 1.0 + 1e-6)
        step = max(1, min(_MAX_STEP, int(math.log(_QR_SPREAD) / math.log(g))))
    if ok:
        Q, _, ok = _chol_qr_spread(Q)
    if not ok:                                          # Householder QR throughout instead
        Q = torch.linalg.qr(Y0, mode="reduced")[0]
        for _ in range(_ITERS):
            Q = torch.linalg.qr(G @ Q, mode="reduced")[0]
    lam, W = _eigh_host(Q.T @ G @ Q)                      # Rayleigh-Ritz on span(Q)
    return lam.flip(0).clamp(min=0.0), (Q @ W).flip(1)


def _leading_factors(M: torch.Tensor, tol: float, max_rank: int):
    """Rank-r factorisation M ~ U_r diag(S_r) Vh_r of a [m, k] matrix by the energy rule, capped at
    max_rank: the leading r singular triplets only. Returns (U_r fp32 [m, r], SVh_r fp32 [r, k])
    with SVh_r = diag(S_r) Vh_r."""
    Md = M.to(torch.float64)
    m, k = Md.shape
    right = k <= m                                        # eigenvectors of M^T M are V
    G = Md.T @ Md if right else Md @ Md.T
    lam, E = _leading_eigh(G, max_rank)
    r = _energy_rank(lam, float(torch.trace(G)), tol)
    r = max(1, min(lam.numel() if r is None else r, max_rank))
    if right:
        S = lam[:r].sqrt()
        U = (Md @ E[:, :r]) / _nonzero(S)                 # left singular vectors
        SVh = S[:, None] * E[:, :r].T
    else:
        U = E[:, :r]
        SVh = U.T @ Md                                    # diag(S) Vh = U^T M
    U, SVh = _fix_signs(U, SVh)
    return U.to(torch.float32), SVh.to(torch.float32)


def _narrow_factors(M: torch.Tensor, tol: float):
    """The same factorisation for a [m, c] matrix with few columns (c = H), uncapped, through the
    c x c Gram matrix: M = U diag(S) Vh with M^T M = V diag(S^2) V^T."""
    Md = M.to(torch.float64)
    m, c = Md.shape
    # the c x c Gram matrix as a sum of partial Grams over row blocks (one GEMM with a c x c
    # output and m-long reductions runs on a single workgroup), then its eigenpairs on the host
    # (c = H = 8: microseconds there, where a device solver pays several launches)
    blk = 128 if m % 128 == 0 else 1
    Gc = torch.matmul(Md.reshape(m // blk, blk, c).transpose(1, 2),
                      Md.reshape(m // blk, blk, c)).sum(0)
    lam, V = torch.linalg.eigh(Gc.cpu())
    lam, V = lam.flip(0).clamp(min=0.0), V.flip(1).to(Md.device)
    total = float(lam.sum())
    r = _energy_rank(lam, total, tol)
    r = max(1, int(lam.numel()) if r is None else r)
    S = lam[:r].sqrt().to(Md.device)
    U = (Md @ V[:, :r]) / _nonzero(S)                     # left singular vectors
    SVh = S[:, None] * V[:, :r].T
    U, SVh = _fix_signs(U, SVh)
    return U.to(torch.float32), SVh.to(torch.float32)


def _tt_factors(X: torch.Tensor, tol: float, max_rank: int):
    """Cores [1, n, r1], [r1, d, r2], [r2, H, 1] of X [n, d, H] (tokens first)."""
    n, d, H = X.shape
    U1, R1 = _leading_factors(X.reshape(n, d * H), tol, max_rank)
    r1 = int(U1.shape[1])
    U2, R2 = _narrow_factors(R1.reshape(r1 * d, H), tol)
    r2 = int(U2.shape[1])
    return [U1.reshape(1, n, r1), U2.reshape(r1, d, r2), R2.reshape(r2, H, 1)]


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
    # The decoder is int8 x fp16 rank ruler in every coefficient mode (the pool's form); the
    # coefficients below are the int8 mode's. The fp16 and 4-bit modes store the projection
    # onto this decoder instead (the write kernel quantises it), so they take only the decoder.
    qm = 127
    cores = _tt_factors(K.permute(1, 2, 0).contiguous(), cfg["tols"], lay.r1)  # [n, d, H]
    r1 = int(cores[0].shape[2])
    c = cores[0].reshape(n, r1)
    cs = _ruler(c.abs().amax(1, keepdim=True), qm)
    cs = torch.where(cs == 0, torch.ones_like(cs), cs)
    cq = torch.clamp(torch.round(c / cs), -(qm + 1), qm).to(torch.int8)
    g2 = _quant_core(cores[1], 8)
    g3 = _quant_core(cores[2], 8)
    dec = torch.einsum("ajb,bh->ahj", g2, g3[:, :, 0]).reshape(r1, H * d)
    rmax = dec.abs().amax(1, keepdim=True)
    sc = _ruler(torch.where(rmax == 0, torch.ones_like(rmax), rmax), qm)
    dec_q = torch.clamp(torch.round(dec / sc), -(qm + 1), qm)
    s16 = sc.to(torch.float16).to(torch.float32)
    dec_f = dec_q * s16                                              # int8 * fp16 row ruler
    coeff_q = torch.zeros(n, lay.r1, dtype=torch.int8, device=K.device)
    coeff_q[:, :r1] = cq
    padded = torch.zeros(lay.r1, H * d, dtype=torch.float32, device=K.device)
    padded[:r1] = dec_f
    # the pool form of the same decoder: column-major int8 ranks and their rulers
    R = decoder_ranks(lay.r1)
    pq = torch.zeros(H * d, R, dtype=torch.int8, device=K.device)
    ps = torch.zeros(R, dtype=torch.float32, device=K.device)
    pq[:, :r1] = dec_q.t().to(torch.int8)
    ps[:r1] = s16.reshape(r1)
    return FittedK(coeff_q=coeff_q, coeff_scale=cs.reshape(n),
                   decoder=KDecoder(padded, DecoderPool(pq, ps)), fitted_rank=r1, budget=lay.r1)
