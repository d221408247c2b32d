"""The product's host-side slot (un)packing (`vllm_ttkv.layout.pack_k_slots` and friends) against
slot bytes the REFERENCE wrote (tests/golden/ref_encode_*.npz: `fit_k_slots`, `frozen_k_slots`,
`v_slots`, with the coefficients and rulers they were packed from), against the oracle's packer
on random row stores, and by round trips. Reference: vllm_ttkv/layout.py:161-261 and its test
tests/test_layout.py (pack, then unpack, must be a faithful rearrangement)."""
import pathlib
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import layout as olayout
from vllm_ttkv import layout as play

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def _rows(bitmap, packed, scale):
    return SimpleNamespace(rows=bitmap.shape[0], bitmap=bitmap, packed=packed, scale=scale)


@pytest.mark.parametrize("fname,cfg", [("ref_encode_safe_r16.npz", "safe"),
                                       ("ref_encode_campaign4x_r64.npz", "campaign4x")])
@pytest.mark.parametrize("which", ["fit", "frozen"])
def test_reference_k_slot_bytes_round_trip(fname, cfg, which):
    z = np.load(GOLD / fname)
    lay = play.layout_for_config(play.CONFIGS[cfg], int(z["r1"]))
    ref = torch.from_numpy(z[f"{which}_k_slots"])
    assert ref.shape[1] == lay.k_slot_bytes
    cq, cs, (bm, pk, sc) = play.unpack_k_slots(lay, ref)
    assert torch.equal(cq, torch.from_numpy(z[f"{which}_coeff_q"]))
    assert torch.equal(cs.view(torch.int16),
                       torch.from_numpy(z[f"{which}_coeff_scale"]).view(torch.int16))
    again = play.pack_k_slots(lay, cq, cs, _rows(bm, pk, sc))
    assert torch.equal(again, ref), "pack(unpack(reference bytes)) != reference bytes"


@pytest.mark.parametrize("fname,cfg", [("ref_encode_safe_r16.npz", "safe"),
                                       ("ref_encode_campaign4x_r64.npz", "campaign4x")])
def test_reference_v_slot_bytes_round_trip(fname, cfg):
    z = np.load(GOLD / fname)
    lay = play.layout_for_config(play.CONFIGS[cfg], int(z["r1"]))
    ref = torch.from_numpy(z["v_slots"])
    bm, pk, sc = play.unpack_v_slots(lay, ref)
    assert bm.shape == (lay.H * ref.shape[0], 16)
    assert torch.equal(play.pack_v_slots(lay, _rows(bm, pk, sc)), ref)


@pytest.mark.parametrize("cfg", ["safe", "tight", "campaign4x"])
def test_pack_equals_the_oracle_packer(cfg):
    """Random row stores: the product's strided copies put every byte where the oracle's
    per-head loop does (and zero the padding)."""
    g = torch.Generator().manual_seed(7)
    c = play.CONFIGS[cfg]
    lay = play.layout_for_config(c, 110)
    olay = olayout.layout_for_config(c, 110)
    n, H = 37, lay.H
    kpb = play.packed_row_bytes(lay.res_k, lay.res_bits)
    vpb = play.packed_row_bytes(lay.v_lanes, lay.v_bits)
    cq = torch.randint(-128, 128, (n, lay.r1), generator=g, dtype=torch.int8)
    cs = torch.rand(n, generator=g).to(torch.float16)
    kb = torch.randint(0, 256, (H * n, 16), generator=g, dtype=torch.uint8)
    kp = torch.randint(0, 256, (H * n, kpb), generator=g, dtype=torch.uint8)
    ks = torch.randn(H * n, generator=g).to(torch.float16)
    vb = torch.randint(0, 256, (H * n, 16), generator=g, dtype=torch.uint8)
    vp = torch.randint(0, 256, (H * n, vpb), generator=g, dtype=torch.uint8)
    vs = torch.randn(H * n, generator=g).to(torch.float16)
    k = play.pack_k_slots(lay, cq, cs, _rows(kb, kp, ks))
    v = play.pack_v_slots(lay, _rows(vb, vp, vs))
    assert torch.equal(k, olayout.pack_k_slots(olay, cq, cs, kb, kp, ks))
    assert torch.equal(v, olayout.pack_v_slots(olay, vb, vp, vs))
    cq2, cs2, (kb2, kp2, ks2) = play.unpack_k_slots(lay, k)
    assert torch.equal(cq2, cq) and torch.equal(cs2.view(torch.int16), cs.view(torch.int16))
    assert torch.equal(kb2, kb) and torch.equal(kp2, kp)
    assert torch.equal(ks2.view(torch.int16), ks.view(torch.int16))
    vb2, vp2, vs2 = play.unpack_v_slots(lay, v)
    assert torch.equal(vb2, vb) and torch.equal(vp2, vp)
    assert torch.equal(vs2.view(torch.int16), vs.view(torch.int16))


def test_pack_refuses_a_row_count_that_is_not_h_times_n():
    lay = play.layout_for_config(play.CONFIGS["safe"], 110)
    rows = _rows(torch.zeros(8 * 3 + 1, 16, dtype=torch.uint8),
                 torch.zeros(8 * 3 + 1, 31, dtype=torch.uint8), torch.zeros(8 * 3 + 1))
    with pytest.raises(ValueError):
        play.pack_k_slots(lay, torch.zeros(3, 110, dtype=torch.int8), torch.zeros(3), rows)
    with pytest.raises(ValueError):
        play.pack_v_slots(lay, rows)
