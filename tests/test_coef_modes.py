"""The fp16 and 4-bit (group-32) coefficient modes, `qbits` 16 and 4. CPU only.

These modes are this build's own: the reference writes only int8 coefficients (its packer views
them as int8 bytes, layout.py:179), so nothing it wrote can pin them. They are pinned here by what
their definition fixes: the scale rule recomputed with frexp arithmetic instead of bit masks, the
quantiser's error bound, exactness of every stored value in fp16, a bit-at-a-time packer written
from the format's text, round trips through both the oracle's and the product's packers, and the
byte geometry the C ABI computes."""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import codec, coef_modes
from oracle import encode as oenc
from oracle.layout import layout_for_config as olayout
from oracle.layout import pack_k_slots as opack
from vllm_ttkv import _hip
from vllm_ttkv.layout import (EXTENSION_CONFIGS, TTKLayout, coefficient_values, config_named,
                              layout_for_config, pack_k_slots, unpack_k_slots)


def _coeffs(n, r1, seed, spread=True):
    g = torch.Generator().manual_seed(seed)
    c = torch.randn(n, r1, generator=g)
    if spread:  # groups of very different magnitude, exact zeros, a zero group
        c = c * (10.0 ** torch.randint(-5, 4, (n, 1), generator=g)).float()
        c[:, 3] = 0.0
        c[0, 32:64] = 0.0
    return c


def _scale_by_frexp(m: float) -> float:
    """The 4-bit group scale from its definition, with float64 arithmetic: m / 7 in fp32, rounded
    up to 8 significant bits, clamped to [2^-14, 9344]; 0 for m = 0."""
    if m == 0.0:
        return 0.0
    s0 = float(np.float32(m) / np.float32(7.0))
    mant, ex = math.frexp(s0)                      # s0 = mant * 2^ex, mant in [0.5, 1)
    s = math.ceil(mant * 256.0) / 256.0 * 2.0 ** ex
    return min(max(s, 2.0 ** -14), 9344.0)


def _sig_bits(x: float) -> int:
    if x == 0.0:
        return 0
    mant, _ = math.frexp(abs(x))
    k = 0
    while mant != math.floor(mant):
        mant *= 2.0
        k += 1
    return k


def test_geometry_closed_form_and_abi():
    """r1 = 110: fp16 coefficients take 220 bytes and no ruler; 4-bit ones 56 bytes (14 words)
    plus 4 scales. The product layout, the oracle layout and the C ABI agree on every size."""
    L = _hip.lib()
    for name, cfg in EXTENSION_CONFIGS.items():
        for r1 in (14, 64, 96, 110, 128, 143):
            lay = layout_for_config(cfg, r1)
            ol = olayout(cfg, r1)
            assert lay.k_field == ol.k_field_off
            assert lay.k_slot_bytes == ol.k_slot_bytes
            assert lay.compressed_bytes_per_token() == ol.compressed_bytes_per_token()
            assert L.ttkv_blob_bytes(_hip.Layout.of(lay)) == lay.compressed_bytes_per_token()
    f = layout_for_config(config_named("safe_fp16"), 110)
    assert (f.coeff_bytes, f.coeff_scale_bytes, f.k_field) == (220, 0, 220)
    q = layout_for_config(config_named("campaign4x_int4g32"), 110)
    assert (q.coeff_bytes, q.coef_groups, q.coeff_scale_bytes, q.k_field) == (56, 4, 8, 64)
    with pytest.raises(ValueError):
        TTKLayout(H=8, d=128, r1=110, qbits=6, res_k=81, res_bits=3, v_lanes=81, v_bits=3)
    assert L.ttkv_blob_bytes(_hip.Layout(8, 128, 110, 6, 81, 3, 81, 3)) == -1


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_group_scale_rule(seed):
    """Every group scale equals the frexp restatement, has at most 8 significant bits, covers the
    group's largest magnitude (7 * scale >= m), and is the smallest such value (one 8-bit step
    below it does not)."""
    c = _coeffs(16, 110, seed)
    c[1, :32] = 1e-7                                 # clamps to 2^-14
    c[2, 64:96] = 1e6                                # clamps to 9344 (saturates)
    s = coef_modes.group_scales(c)
    for i in range(c.shape[0]):
        for g in range(s.shape[1]):
            m = float(c[i, 32 * g:32 * g + 32].abs().max())
            want = _scale_by_frexp(m)
            got = float(s[i, g])
            assert got == want, (i, g, m, got, want)
            assert _sig_bits(got) <= 8
            if m > 0 and want not in (2.0 ** -14, 9344.0):
                assert 7.0 * got >= float(np.float32(m) / np.float32(7.0)) * 7.0
                mant, ex = math.frexp(got)
                below = (mant * 256 - 1) / 256 * 2.0 ** ex
                assert below < float(np.float32(m) / np.float32(7.0))
    assert float(s[0, 1]) == 0.0                    # the all-zero group
    assert float(s[1, 0]) == 2.0 ** -14 and float(s[2, 2]) == 9344.0


@pytest.mark.parametrize("seed", [0, 1])
def test_int4_quantiser_bounds_and_exactness(seed):
    """q in [-7, 7]; |c - q*s| <= s/2 wherever |c| <= 7s (everywhere but the saturated group);
    q*s is exactly representable in fp16; an all-zero group stores zeros."""
    c = _coeffs(32, 110, seed)
    c[2, 64:96] = 1e6
    vals, q, s = coef_modes.quantise(c, 4)
    assert int(q.abs().max()) <= 7
    sr = s.repeat_interleave(32, 1)[:, :110]
    inside = c.abs() <= 7 * sr
    assert bool(inside[~(c.abs() > 1e5)].all())
    assert bool(((c - vals).abs() <= sr / 2)[inside].all())
    assert torch.equal(vals.half().float(), vals)
    assert torch.equal(vals, q.float() * sr)
    assert bool((vals[0, 32:64] == 0).all())
    assert float(vals[2, 64:96].abs().max()) == 7 * 9344.0


def test_fp16_mode_is_round_to_nearest():
    """The fp16 mode stores IEEE round-to-nearest-even fp16 of each coefficient (numpy's
    conversion, an independent implementation), including overflow to inf."""
    c = _coeffs(8, 110, 5)
    c[0, 0] = 70000.0
    vals, h, s = coef_modes.quantise(c, 16)
    assert s is None
    with np.errstate(over="ignore"):
        want = c.numpy().astype(np.float16)
    assert np.array_equal(h.numpy(), want)
    assert torch.equal(vals, torch.from_numpy(want.astype(np.float32)))
    assert math.isinf(float(vals[0, 0]))


def _brute_pack(q_row, r1):
    """The 4-bit values' bytes from the format's text, one bit at a time: word w holds rank
    8w + 2m at bits 4m..4m+3 and rank 8w + 2m + 1 at bits 16+4m..16+4m+3, little-endian."""
    W = (r1 + 7) // 8
    bits = [0] * (32 * W)
    for w in range(W):
        for m in range(4):
            for e in range(2):
                r = 8 * w + 2 * m + e
                v = (int(q_row[r]) & 15) if r < r1 else 0
                for b in range(4):
                    bits[32 * w + 16 * e + 4 * m + b] = (v >> b) & 1
    out = []
    for byte in range(4 * W):
        out.append(sum(bits[8 * byte + b] << b for b in range(8)))
    return out


@pytest.mark.parametrize("r1", [1, 7, 8, 33, 110, 128])
def test_nibble_packers_match_brute_force(r1):
    g = torch.Generator().manual_seed(r1)
    q = torch.randint(-8, 8, (6, r1), generator=g, dtype=torch.int8)
    ob = coef_modes.pack_nibbles(q)
    for i in range(q.shape[0]):
        assert ob[i].tolist() == _brute_pack(q[i].tolist(), r1)
    assert torch.equal(coef_modes.unpack_nibbles(ob, r1), q)


def _store(lay, n, seed):
    g = torch.Generator().manual_seed(seed)
    R = torch.randn(lay.H * n, lay.d, generator=g)
    bm, pk, sc = codec.build_rows(R, lay.res_k, lay.res_bits)
    return bm, pk, sc


@pytest.mark.parametrize("name", sorted(EXTENSION_CONFIGS))
def test_product_and_oracle_slots_agree(name):
    """The product's `pack_k_slots` writes the oracle's bytes for both modes; `unpack_k_slots`
    gives the fields back, and `coefficient_values` the oracle's stored values."""
    cfg = EXTENSION_CONFIGS[name]
    lay, ol = layout_for_config(cfg, 110), olayout(cfg, 110)
    n = 24
    c = _coeffs(n, 110, 9)
    vals, q, s = coef_modes.quantise(c, lay.qbits)
    bm, pk, sc = _store(lay, n, 3)
    ob = opack(ol, q, s, bm, pk, sc)
    rows = SimpleNamespace(rows=bm.shape[0], bitmap=bm, packed=pk, scale=sc)
    pq = q
    ps = None if lay.qbits == 16 else s.half()
    pb = pack_k_slots(lay, pq, ps, rows)
    assert torch.equal(pb, ob)
    cq2, cs2, (bm2, pk2, sc2) = unpack_k_slots(lay, pb)
    assert torch.equal(cq2, pq) and torch.equal(bm2, bm) and torch.equal(pk2, pk)
    assert torch.equal(sc2, sc.half())
    if ps is not None:
        assert torch.equal(cs2, ps)
    assert torch.equal(coefficient_values(lay, cq2, cs2), vals)
    assert torch.equal(coef_modes.values_from_field(lay.qbits, 110, pb[:, :lay.k_field]), vals)


@pytest.mark.parametrize("name", sorted(EXTENSION_CONFIGS))
def test_frozen_encode_round_trip(name):
    """An oracle frozen write in the mode reads back (dense reconstruction from the slot bytes)
    as stored values @ decoder + materialised residual rows, and the fp16 mode's key error before
    the residual is no larger than the int8 mode's on the same decoder (finer coefficients)."""
    from oracle import attend
    cfg = EXTENSION_CONFIGS[name]
    ol = olayout(cfg, 40)
    base = olayout(dict(cfg, qbits=8), 40)
    g = torch.Generator().manual_seed(11)
    Z = torch.randn(64, 12, generator=g)
    K = (Z @ torch.randn(12, ol.H * ol.d, generator=g) / 12 ** 0.5).reshape(64, ol.H, ol.d)
    K = K.permute(1, 0, 2).contiguous() + 0.05 * torch.randn(ol.H, 64, ol.d, generator=g)
    dec_q = torch.randint(-127, 128, (40, ol.H * ol.d), generator=g).float()
    dec = dec_q * (torch.rand(40, 1, generator=g) + 0.5).half().float() * 2 ** -7
    e = oenc.encode_frozen_mode(K, dec, ol)
    slots = opack(ol, e["coeff_q"], e["coeff_scale"], *e["resid"])
    got = attend.dense_k_from_slots(ol, slots, dec, torch.float64)
    resid = codec.packed_rows_materialise(*e["resid"], ol.d, ol.res_k, ol.res_bits).double()
    want = (e["values"].double() @ dec.double()).reshape(64, ol.H, ol.d).permute(1, 0, 2) \
        + resid.reshape(ol.H, 64, ol.d)
    assert torch.allclose(got, want, rtol=0, atol=1e-9)
    if ol.qbits == 16:
        e8 = oenc.encode_frozen(K, dec, base)
        k8 = (e8["coeff_q"].float() * e8["coeff_scale"].float()[:, None]) @ dec
        kf = e["values"] @ dec
        Kt = K.permute(1, 0, 2).reshape(64, -1)
        assert float((Kt - kf).abs().max()) <= float((Kt - k8).abs().max())


def test_kernels_refuse_int8_coefficients_in_other_modes():
    """The write's int8 coefficient input belongs to the int8 mode; the C ABI refuses it for the
    fp16 / 4-bit modes before any launch (dummy pointers only)."""
    from test_abi import _write_call
    L = _hip.lib()
    for name in EXTENSION_CONFIGS:
        lay = layout_for_config(config_named(name), 110)
        assert _write_call(lay, cq_in=1, cs_in=1, slot_stride=1024) == 1
        assert b"coeff_q_in" in L.ttkv_last_error()


def test_read_kernels_refuse_unbuilt_shapes():
    """The fp16 / 4-bit modes are built for G = 3 and 64 < r1 <= 128; other shapes are refused
    on the host with a message (dummy pointers only)."""
    from test_abi import _decode_call, _prefill_call
    L = _hip.lib()
    for name in EXTENSION_CONFIGS:
        lay = layout_for_config(config_named(name), 110)
        w = lay.compressed_bytes_per_token() // 16 * 16 + 16
        assert _decode_call(lay, num_heads=8, slot_stride=w) == 2
        assert b"fp16 and 4-bit" in L.ttkv_last_error()
        small = layout_for_config(config_named(name), 40)
        assert _decode_call(small, slot_stride=w) == 2
        assert _prefill_call(lay, num_heads=16, slot_stride=w) == 2
        assert b"fp16 and 4-bit" in L.ttkv_last_error()
