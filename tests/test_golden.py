"""The oracle and the product's fit against vectors written by the reference implementation
itself (`tests/golden/make_fixtures.py`, run in the build container, CPU torch).

The reference ran on the CPU, where its rulers are correctly rounded divisions, so the oracle is
run with `ruler_mode="cpu"` and must reproduce every byte. The product's fit uses the rulers of
the reference's CUDA store (a multiply by the fp32 reciprocal), which differ from the CPU ones by
at most one ulp; it is held to the fixture within that.
"""
from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

from oracle import codec as oc
from oracle import encode as oe
from oracle.layout import layout_for_config

GOLDEN = pathlib.Path(__file__).parent / "golden"
CASES = sorted(GOLDEN.glob("ref_encode_*.npz"))


def load(path):
    z = np.load(path)
    f = {k: z[k] for k in z.files}
    name = str(f["config"])
    cfg = oc.CONFIGS[name]
    lay = layout_for_config(cfg, int(f["r1"]), H=int(f["H"]), d=int(f["d"]))
    return f, cfg, lay


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def test_fixtures_present():
    assert len(CASES) >= 2


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_fit_matches_reference(path):
    f, cfg, lay = load(path)
    K0 = t(f["K0"]).float()
    fit = oe.fit_into_budget(K0, lay, cfg, ruler_mode="cpu")
    assert fit["fitted_rank"] == int(f["fit_rank"])
    assert torch.equal(fit["decoder_f"], t(f["fit_decoder_f"]))
    assert torch.equal(fit["coeff_q"], t(f["fit_coeff_q"]))
    cs16 = fit["coeff_scale"].to(torch.float16).reshape(-1)
    assert torch.equal(cs16, t(f["fit_coeff_scale"]))
    slots = oe.k_slots_from(lay, fit["coeff_q"], cs16, fit["resid"])
    assert torch.equal(slots, t(f["fit_k_slots"]))


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_pinv_matches_reference(path):
    f, _, _ = load(path)
    pm = oe.pinv(t(f["fit_decoder_f"]))
    torch.testing.assert_close(pm, t(f["pinv"]), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_frozen_encode_matches_reference(path):
    f, _, lay = load(path)
    K1 = t(f["K1"]).float()
    enc = oe.encode_frozen(K1, t(f["fit_decoder_f"]), lay, pinv_m=t(f["pinv"]), ruler_mode="cpu")
    assert torch.equal(enc["coeff_q"], t(f["frozen_coeff_q"]))
    assert torch.equal(enc["coeff_scale"], t(f["frozen_coeff_scale"]))
    assert torch.equal(enc["R"], t(f["frozen_resid_src"]))
    slots = oe.k_slots_from(lay, enc["coeff_q"], enc["coeff_scale"], enc["resid"])
    assert torch.equal(slots, t(f["frozen_k_slots"]))


def tie_rows(X: torch.Tensor, k: int) -> torch.Tensor:
    """Rows whose k-th largest magnitude is shared with a lane outside the top k."""
    a = X.abs()
    srt = torch.sort(a, dim=1, descending=True).values
    return srt[:, k - 1] == srt[:, k]


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_v_encode_matches_reference(path):
    """Bit-exact on every row whose lane selection has no tie at the k-th magnitude. On a tied
    row the reference's torch path keeps whichever lane `torch.topk` returns, the oracle the
    lowest index (the fused store's rule); handed the same lanes the oracle packs the same
    bytes, which pins everything after the selection on those rows too."""
    f, _, lay = load(path)
    V0 = t(f["V0"]).float()
    H, n, d = V0.shape
    ref = t(f["v_slots"])
    slots = oe.v_slots_from(lay, oe.encode_v(V0, lay, ruler_mode="cpu"))
    X = V0.reshape(H * n, d)                                   # rows in (head, token) order
    tied = tie_rows(X, lay.v_lanes).reshape(H, n).t()          # [n, H]
    rb = lay.v_row_bytes
    differs = (slots != ref)[:, :H * rb].reshape(n, H, rb).any(-1)
    assert not bool((differs & ~tied).any())
    assert torch.equal(slots[:, H * rb:], ref[:, H * rb:])
    idx = torch.topk(X.abs(), lay.v_lanes, dim=1).indices
    mask = torch.zeros_like(X, dtype=torch.bool).scatter_(1, idx, True)
    rows = oc.packed_rows_build(X, mask, lay.v_bits, lay.v_lanes, ruler_mode="cpu")
    assert torch.equal(oe.v_slots_from(lay, rows), ref)


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_product_fit_matches_reference(path):
    """The shipped fit (`vllm_ttkv.encode.fit_into_budget`, run here on the CPU) against the
    reference's: same rank, decoder and coefficients within one code, once each component's sign
    is aligned. A singular vector is defined up to sign; the reference's signs
    are whatever its LAPACK routine returns, and flipping component i flips decoder row i and
    coefficient column i together, leaving the fitted keys (their product) unchanged."""
    from vllm_ttkv import encode as penc
    from vllm_ttkv.layout import layout_for_config as product_layout

    f, cfg, _ = load(path)
    lay = product_layout(cfg, int(f["r1"]), H=int(f["H"]), d=int(f["d"]))
    fit = penc.fit_into_budget(t(f["K0"]).float(), lay, cfg)
    assert fit.fitted_rank == int(f["fit_rank"])
    ref_dec = t(f["fit_decoder_f"])
    dec = fit.decoder.decoder_f
    sign = torch.where((dec * ref_dec).sum(1) < 0, -1.0, 1.0)     # per component
    assert bool((sign[fit.fitted_rank:] == 1).all())              # padding rows are zero
    # decoder: within a ruler ulp, except where a value within rounding noise of a half-code
    # (in the decoder or in one of the two quantised cores it is the product of) rounds to the
    # neighbouring code: at most one code step, in at most 0.1% of the entries
    qm = 2 ** (lay.qbits - 1) - 1
    step = ref_dec.abs().amax(1, keepdim=True) / qm
    err = (dec * sign[:, None] - ref_dec).abs()
    assert bool((err <= 1.01 * step + 1e-6).all())
    near = err <= 2e-3 * float(ref_dec.abs().max())
    assert float((~near).float().mean()) < 1e-3
    cq = fit.coeff_q.to(torch.int32) * sign.to(torch.int32)
    dq = (cq - t(f["fit_coeff_q"]).to(torch.int32)).abs()
    assert int(dq.max()) <= 1
    assert float((dq != 0).float().mean()) < 0.02
    torch.testing.assert_close(fit.coeff_scale.to(torch.float16), t(f["fit_coeff_scale"]),
                               rtol=1e-3, atol=0)
    # the fitted keys themselves, sign-free: within the quantisation step of the reference's
    mine = (fit.coeff_q.float() * fit.coeff_scale[:, None].float()) @ dec
    ref = (t(f["fit_coeff_q"]).float() * t(f["fit_coeff_scale"]).float()[:, None]) @ ref_dec
    assert float((mine - ref).norm() / ref.norm()) < 2e-2


PACKED = GOLDEN / "ref_packed_rows.npz"
ATTEND = GOLDEN / "ref_attend_safe.npz"


def _packed_keys():
    z = np.load(PACKED)
    return sorted({k.rsplit("_", 1)[0] for k in z.files if k.endswith("_X")})


@pytest.mark.parametrize("key", _packed_keys())
def test_packed_rows_build_matches_reference(key):
    """PackedRows.build on the reference's own (X, mask) pairs: bitmap, MSB-first code stream and
    fp16 ruler bytes identical (CPU rulers: correctly rounded division)."""
    z = np.load(PACKED)
    X, mask = t(z[f"{key}_X"]), t(z[f"{key}_mask"])
    bits, k = int(z[f"{key}_bits"]), int(z[f"{key}_k"])
    bm, pk, sc = oc.packed_rows_build(X, mask, bits, k, ruler_mode="cpu")
    assert torch.equal(bm, t(z[f"{key}_bitmap"]))
    assert torch.equal(pk, t(z[f"{key}_packed"]))
    assert torch.equal(sc, t(z[f"{key}_scale"]))


def test_attention_oracle_matches_reference():
    """Scores, causal multi-query scores and both attention orders against the reference's
    reference.py on the same fitted store (fp32 CPU; summation order may differ, so 1e-5)."""
    from oracle import attend
    z = np.load(ATTEND)
    lay = layout_for_config(oc.CONFIGS[str(z["config"])], int(z["r1"]), H=int(z["H"]),
                            d=int(z["d"]))
    ks, vs, dec = t(z["k_slots"]), t(z["v_slots"]), t(z["decoder_f"])
    cos, sin, q, qm = t(z["cos"]), t(z["sin"]), t(z["q"]), t(z["qm"])
    p0 = int(z["p0"])

    def close(got, want):
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)

    close(attend.raw_scores(lay, ks, dec, q, cos, sin), t(z["raw_scores"]))
    close(attend.raw_scores_multi(lay, ks, dec, qm, cos, sin), t(z["raw_scores_multi"]))
    causal = attend.raw_scores_multi(lay, ks, dec, qm, cos, sin, p0=p0)
    want = t(z["raw_scores_multi_causal"])
    assert torch.equal(torch.isinf(causal), torch.isinf(want))
    close(causal[~torch.isinf(want)], want[~torch.isinf(want)])
    close(attend.attend_raw_store(lay, ks, vs, dec, q, cos, sin), t(z["attend_raw_store"]))
    close(attend.oracle_attend(lay, ks, vs, dec, q, cos, sin), t(z["oracle_attend"]))
