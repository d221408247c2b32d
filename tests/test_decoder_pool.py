"""The decoder pool's storage form (`vllm_ttkv.decoder_pool`): the codec's int8 decoder with one
ruler per rank, column-major, padded to `decoder_ranks(r1)` ranks. CPU only.

Pinned by the decoders the reference itself wrote (tests/golden/: its fit's `decoder_f`, which is
`dec_q * dec_scale` by construction, ttkv_packed_cache.py:284-293), by the oracle codec's own
(dec_q, dec_scale) pairs, and by the C ABI's `ttkv_decoder_ranks`."""
import pathlib

import numpy as np
import pytest
import torch

from oracle import codec
from vllm_ttkv import synth
from vllm_ttkv.decoder_pool import (DecoderPool, decoder_ranks, empty_pool, from_codec,
                                    pack_decoders, unpack_decoders)

GOLDEN = pathlib.Path(__file__).parent / "golden"


@pytest.mark.parametrize("case,key", [("ref_encode_safe_r16", "fit_decoder_f"),
                                      ("ref_encode_campaign4x_r64", "fit_decoder_f"),
                                      ("ref_attend_safe", "decoder_f")])
def test_reference_decoders_pack_exactly(case, key):
    """Every decoder the reference wrote is int8 x one ruler per rank: the pool holds it with no
    loss (`float(q) * scale` reproduces every fp32 value bit for bit), padded ranks are zero."""
    dec = torch.from_numpy(np.load(GOLDEN / f"{case}.npz")[key]).float()
    r1, hd = dec.shape
    p = pack_decoders(dec)
    R = decoder_ranks(r1)
    assert p.q.dtype == torch.int8 and tuple(p.q.shape) == (hd, R)
    assert p.scale.dtype == torch.float32 and tuple(p.scale.shape) == (R,)
    assert torch.equal(unpack_decoders(p, r1), dec)
    assert not bool(p.q[:, r1:].any()) and not bool(p.scale[r1:].any())
    # the rulers are the codec's fp16 rulers (exact in fp16)
    assert torch.equal(p.scale, p.scale.half().float())


def test_codec_pairs_map_directly():
    """The oracle codec's (dec_q [r1, H*d] int8, dec_scale [r1] fp16) pair gives the same pool as
    packing its fp32 decoder: rows whose largest |q| is 127 (every fitted row) match
    byte for byte."""
    cfg = codec.CONFIGS["safe"]
    K = synth.keys(96, seed=4)
    kl = codec.build_k_layer(K, cfg["tols"], cfg["qbits"], cfg["res_frac"], cfg["res_bits"],
                             max_rank=40)
    a = from_codec(kl["dec_q"], kl["dec_scale"])
    b = pack_decoders(kl["decoder_f"])
    r1 = kl["r1"]
    assert torch.equal(unpack_decoders(a, r1), kl["decoder_f"])
    assert torch.equal(unpack_decoders(b, r1), kl["decoder_f"])
    full = kl["dec_q"].abs().amax(1) == 127
    assert bool(full.all())
    assert torch.equal(a.q, b.q) and torch.equal(a.scale, b.scale)


def test_batched_pack_and_other_largest_magnitudes():
    """A batch of decoders packs slot by slot; a row whose largest |q| is not 127 (a hand-made
    codec row) is still found exactly; zero rows get ruler 0."""
    g = torch.Generator().manual_seed(0)
    decs = []
    for s, qmax in enumerate((127, 100, 128, 3)):
        q = torch.randint(-qmax, qmax + 1, (50, 1024), generator=g).float()
        q[:, 0] = -qmax if qmax == 128 else qmax
        q = q.clamp(-128, 127)
        ruler = (torch.rand(50, generator=g) + 0.5).half().float() * 2.0 ** -(8 + s)
        d = q * ruler[:, None]
        d[7] = 0.0
        decs.append(d)
    p = pack_decoders(torch.stack(decs))
    assert isinstance(p, DecoderPool) and p.slots == 4 and p.q.shape == (4, 1024, 64)
    got = unpack_decoders(p, 50)
    for s in range(4):
        assert torch.equal(got[s], decs[s])
        assert float(p.scale[s, 7]) == 0.0


@pytest.mark.parametrize("bad", ["random", "nan"])
def test_non_codec_decoders_are_refused(bad):
    """A decoder that is not int8 x ruler (the pool cannot hold it without loss) is refused
    with an error, never rounded."""
    d = torch.randn(16, 1024)
    if bad == "nan":
        d = (torch.randint(-127, 128, (16, 1024)).float() * 0.01).half().float()
        d[3, 5] = float("nan")
    with pytest.raises(ValueError):
        pack_decoders(d)


def test_decoder_ranks_matches_the_c_abi():
    """`decoder_ranks` is the C ABI's `ttkv_decoder_ranks` (the library loads without a GPU),
    and every kernel's rank window fits inside it: K1's 16-rank units (r1 padded to 64, 112, 128
    or 160), K2's 32-rank steps and K3's whole 64-rank chunks."""
    from vllm_ttkv import _hip
    L = _hip.lib()
    for r1 in range(1, 300):
        R = decoder_ranks(r1)
        assert L.ttkv_decoder_ranks(r1) == R
        assert R >= r1 and R % 64 == 0
        ku = 4 if r1 <= 64 else 7 if r1 <= 112 else 8 if r1 <= 128 else 10 if r1 <= 160 else 0
        if ku:
            assert 16 * ku <= R
        assert 32 * ((r1 + 31) // 32) <= R
    assert L.ttkv_decoder_ranks(0) == -1
    with pytest.raises(ValueError):
        decoder_ranks(0)


def test_empty_pool_shapes():
    p = empty_pool(3, 110, 8, 128, "cpu")
    assert p.q.shape == (3, 1024, 128) and p.scale.shape == (3, 128)
    assert not bool(p.q.any()) and not bool(p.scale.any())
    assert p.slot(1).q.shape == (1024, 128)


@pytest.mark.gpu
def test_device_packing_matches_the_host():
    """Packing on the device gives the host's pool, rows whose largest |q| is not 127 included
    (the search works in float64: fp32 division on the device need not round correctly, and a
    row of largest |q| 126 was refused once for that)."""
    g = torch.Generator().manual_seed(5)
    q = torch.randint(-127, 128, (110, 512), generator=g).float()
    q[:, 0] = 126.0
    q[:40].clamp_(-126, 126)
    q[40:60].clamp_(-100, 100)
    q[60:70] = q[60:70].clamp(-128, 127)
    q[60:70, 1] = -128.0
    ruler = (torch.rand(110, generator=g) * 0.02 + 0.005).half().float()
    dec = q * ruler[:, None]
    host = pack_decoders(dec)
    dev = pack_decoders(dec.cuda())
    assert torch.equal(dev.q.cpu(), host.q) and torch.equal(dev.scale.cpu(), host.scale)
    assert torch.equal(unpack_decoders(dev, 110).cpu(), dec)
