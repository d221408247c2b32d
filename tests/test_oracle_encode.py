"""Pins for the oracle's write path (oracle/encode.py): the frozen projection's invariants, the
coefficient quantiser's closed form, exact zero padding of the rank budget.

Reference: vllm_ttkv/encode.py:257-351; tests/test_encode.py:91-293 (padding exact, budget
monotone, least squares)."""
import numpy as np
import torch

from oracle import codec, encode
from oracle.layout import layout_for_config
from vllm_ttkv import synth


def test_zero_padding_is_exact():
    """A fit at natural rank r < r1 pads coefficients and decoder rows with zeros; the product is
    unchanged and the pseudo-inverse has zero columns there (encode.py:287-296)."""
    cfg = codec.CONFIGS["safe"]
    K = synth.keys(48, seed=3)
    lay = layout_for_config(cfg, r1=110)
    fk = encode.fit_into_budget(K, lay, cfg)
    r = fk["fitted_rank"]
    assert r < 110
    assert int(fk["coeff_q"][:, r:].abs().sum()) == 0
    assert float(fk["decoder_f"][r:].abs().sum()) == 0.0
    pm = encode.pinv(fk["decoder_f"])
    assert float(pm[:, r:].abs().max()) < 1e-6


def test_quantise_coeffs_closed_form():
    c = torch.randn(9, 110, generator=torch.Generator().manual_seed(1))
    c[3] = 0
    cq, cs = encode.quantise_coeffs(c)
    s = c.abs().amax(1, keepdim=True) * torch.tensor(np.float32(1 / 127))
    s = torch.where(s == 0, torch.ones_like(s), s)
    assert torch.equal(cs, s)
    assert torch.equal(cq, torch.clamp(torch.round(c / s), -128, 127).to(torch.int8))
    assert cs[3].item() == 1.0 and int(cq[3].abs().sum()) == 0
    ok = [i for i in range(9) if i != 3]
    assert torch.all(cq[ok].abs().amax(1) == 127)


def test_frozen_projection_is_least_squares():
    """c = M @ pinv(decoder) satisfies the normal equations, and projecting the fit's own chunk
    reconstructs it no worse than the fit's quantised coefficients (test_encode.py:238-259)."""
    cfg = codec.CONFIGS["safe"]
    lay = layout_for_config(cfg, r1=110)
    K = synth.keys(96, seed=7)
    fk = encode.fit_into_budget(K[:, :64].contiguous(), lay, cfg)
    dec = fk["decoder_f"].double()
    M = K[:, 64:].permute(1, 0, 2).reshape(32, -1).double()
    c = encode.project(K[:, 64:].contiguous(), encode.pinv(fk["decoder_f"])).double()
    normal = (M - c @ dec) @ dec.T
    assert normal.abs().max() < 1e-3 * M.abs().max() * dec.abs().max()
    Mf = K[:, :64].permute(1, 0, 2).reshape(64, -1).double()
    cf = encode.project(K[:, :64].contiguous(), encode.pinv(fk["decoder_f"])).double()
    fit_c = fk["coeff_q"].double() * fk["coeff_scale"].double().unsqueeze(1)
    assert (Mf - cf @ dec).norm() <= (Mf - fit_c @ dec).norm() * 1.0001


def test_frozen_encode_residual_definition():
    cfg = codec.CONFIGS["campaign4x"]
    lay = layout_for_config(cfg, r1=110)
    K = synth.keys(80, seed=9)
    fk = encode.fit_into_budget(K[:, :64].contiguous(), lay, cfg)
    out = encode.encode_frozen(K[:, 64:].contiguous(), fk["decoder_f"], lay)
    cq, cs = encode.quantise_coeffs(out["c"])
    R = (K[:, 64:] - ((cq.float() * cs) @ fk["decoder_f"]).reshape(16, 8, 128).permute(1, 0, 2))
    assert torch.equal(out["R"], R.reshape(8 * 16, 128))
    assert torch.equal(out["coeff_scale"], cs.to(torch.float16).reshape(-1))
