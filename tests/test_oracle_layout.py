"""Pins for slot geometry and the per-token blob (oracle/layout.py and the package's layout.py).

Closed-form offsets for the three shipped allocations (layout.py:98-157 arithmetic, done by hand)
and the reference's own slot assertions (test_layout.py, test_decode_conventions.py:169-215)."""
import numpy as np
import pytest
import torch

from oracle import codec
from oracle.layout import (Layout, layout_for_config, pack_k_slots, pack_v_slots, split_blob,
                           unpack_k_slots, unpack_v_slots)
from vllm_ttkv import layout as plib

# (config, r1) -> (k_row, k_slot, v_row, v_slot, blob)
TABLE = {
    ("safe", 110): (49, 512, 49, 400, 912),
    ("campaign4x", 110): (50, 512, 50, 400, 912),
    ("tight", 110): (30, 352, 35, 288, 640),
    ("safe", 64): (49, 464, 49, 400, 864),
}


@pytest.mark.parametrize("key", sorted(TABLE))
def test_closed_form_geometry(key):
    cfg, r1 = key
    for L in (layout_for_config(codec.CONFIGS[cfg], r1), plib.layout_for_config(plib.CONFIGS[cfg], r1)):
        got = (L.k_row_bytes, L.k_slot_bytes, L.v_row_bytes, L.v_slot_bytes,
               L.compressed_bytes_per_token())
        assert got == TABLE[key]
        assert L.v_offset == L.k_slot_bytes and L.k_slot_bytes % 16 == 0


def test_reference_slot_arithmetic():
    """test_decode_conventions.py:186-209 (r1=64, 64 lanes @4b both sides)."""
    lay = plib.TTKLayout(H=8, d=128, r1=64, qbits=8, res_k=64, res_bits=4, v_lanes=64, v_bits=4)
    k_raw = lay.coeff_bytes + 2 + lay.H * lay.k_row_bytes
    v_raw = lay.H * lay.v_row_bytes
    assert lay.k_slot_bytes == -(-k_raw // 16) * 16 and lay.v_slot_bytes == -(-v_raw // 16) * 16
    for r1, frac, rb, kl, vb in ((100, 0.633, 3, 81, 3), (103, 0.25, 3, 45, 3), (96, 0.5, 4, 64, 4)):
        L = plib.TTKLayout(H=8, d=128, r1=r1, qbits=8, res_k=int(128 * frac), res_bits=rb,
                           v_lanes=kl, v_bits=vb)
        end = L.coeff_bytes + 2 + 8 * L.k_row_bytes
        assert end <= L.k_slot_bytes <= end + 16


def test_layout_refusals():
    with pytest.raises(ValueError):
        plib.TTKLayout(H=8, d=100, r1=8, qbits=8, res_k=8, res_bits=3, v_lanes=8, v_bits=3)
    with pytest.raises(ValueError, match="v_lanes"):
        plib.TTKLayout(H=16, d=64, r1=8, qbits=8, res_k=40, res_bits=3, v_lanes=81, v_bits=3)


def test_pack_unpack_round_trip_and_field_offsets():
    lay = layout_for_config(codec.CONFIGS["safe"], 110)
    g = torch.Generator().manual_seed(0)
    n = 5
    cq = torch.randint(-128, 128, (n, 110), generator=g, dtype=torch.int8)
    cs = torch.rand(n, generator=g).to(torch.float16)
    bm, pk, sc = codec.build_rows(torch.randn(8 * n, 128, generator=g), 81, 3)
    ks = pack_k_slots(lay, cq, cs, bm, pk, sc)
    assert ks.shape == (n, 512)
    cq2, cs2, (bm2, pk2, sc2) = unpack_k_slots(lay, ks)
    assert torch.equal(cq2, cq) and torch.equal(cs2, cs)
    assert torch.equal(bm2, bm) and torch.equal(pk2, pk) and torch.equal(sc2, sc)
    # head h row of token i starts at 112 + 49h: bitmap, 31 code bytes, fp16 ruler LE
    h, i = 5, 3
    row = ks[i, 112 + 49 * h:112 + 49 * h + 49]
    assert torch.equal(row[:16], bm[h * n + i]) and torch.equal(row[16:47], pk[h * n + i])
    assert row[47:49].clone().view(torch.float16).item() == sc[h * n + i].item()
    assert int(ks[:, 504:].abs().sum()) == 0                 # padding
    vs = pack_v_slots(lay, bm, pk, sc)
    assert all(torch.equal(a, b) for a, b in zip(unpack_v_slots(lay, vs), (bm, pk, sc)))
    k2, v2 = split_blob(lay, torch.cat([ks, vs], 1))
    assert torch.equal(k2, ks) and torch.equal(v2, vs)
    with pytest.raises(ValueError):
        split_blob(lay, ks)
