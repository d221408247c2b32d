"""Pins for the oracle's bit format (oracle/codec.py): brute-force packers, closed forms of the
ruler and code, the tie rule, and planted-mistake controls showing the checks discriminate.

Reference: codec/ttkv_packed_cache.py:50-271, vllm_ttkv/select_triton.py:24-91, 181-232."""
import numpy as np
import pytest
import torch

from oracle import codec


def brute_pack(vals, bits):
    """Bit-by-bit MSB-first packer: code i occupies stream bits [i*bits, (i+1)*bits), byte b
    holds stream bits 8b..8b+7 with stream bit 8b at the byte's MSB; zero padded."""
    rows, k = vals.shape
    nb = (k * bits + 7) // 8
    out = np.zeros((rows, nb), dtype=np.uint8)
    for r in range(rows):
        for i in range(k):
            for t in range(bits):
                bit = (int(vals[r, i]) >> (bits - 1 - t)) & 1
                p = i * bits + t
                out[r, p // 8] |= bit << (7 - p % 8)
    return out


def brute_bitmap(mask):
    rows, d = mask.shape
    out = np.zeros((rows, d // 8), dtype=np.uint8)
    for r in range(rows):
        for j in range(d):
            if mask[r, j]:
                out[r, j >> 3] |= 1 << (7 - (j & 7))
    return out


@pytest.mark.parametrize("bits,k", [(3, 81), (3, 45), (4, 64), (3, 32), (4, 7)])
def test_code_stream_matches_brute_force(bits, k):
    g = torch.Generator().manual_seed(bits * 100 + k)
    v = torch.randint(0, 2 ** bits, (5, k), generator=g)
    got = codec.pack_bits_rows(v, bits).numpy()
    assert np.array_equal(got, brute_pack(v.numpy(), bits))
    assert torch.equal(codec.unpack_bits_rows(torch.from_numpy(got), k, bits), v.to(torch.int32))


def test_lsb_first_packer_is_rejected():
    """Planted mistake: an LSB-first packer produces different bytes, so the brute-force check
    above would catch a bit-order error."""
    v = torch.tensor([[1, 2, 3, 4, 5, 6, 7, 0]])
    msb = codec.pack_bits_rows(v, 3).numpy()
    rev = brute_pack(np.array([[int(f"{x:03b}"[::-1], 2) for x in v[0]]]), 3)
    assert not np.array_equal(msb, rev)


def test_bitmap_lane_order():
    g = torch.Generator().manual_seed(1)
    m = torch.rand(6, 128, generator=g) > 0.4
    got = codec.pack_mask(m).numpy()
    assert np.array_equal(got, brute_bitmap(m.numpy()))
    assert torch.equal(codec.unpack_bitmap_rows(torch.from_numpy(got), 128), m)
    one = torch.zeros(1, 128, dtype=torch.bool)
    one[0, 9] = True                                        # lane 9 -> byte 1, bit 6
    assert codec.pack_mask(one)[0, 1].item() == 0b01000000


@pytest.mark.parametrize("bits,k", [(3, 81), (4, 64), (3, 45)])
def test_packed_rows_closed_form(bits, k):
    """Per row: exactly k lanes (the k largest magnitudes), ruler = fp16(rowmax * fp32(1/(2^(b-1)
    -1))), stored code = clamp(rint(x / ruler32), -2^(b-1), 2^(b-1)-1) + 2^(b-1) in lane order."""
    g = torch.Generator().manual_seed(bits + k)
    X = torch.randn(40, 128, generator=g) * 0.7
    bm, pk, sc = codec.build_rows(X, k, bits)
    mask = codec.unpack_bitmap_rows(bm, 128)
    assert torch.all(mask.sum(1) == k)
    a = X.abs()
    kth = torch.sort(a, 1, descending=True).values[:, k - 1:k]
    assert torch.equal(mask, a >= kth)                      # tie-free data: the k largest
    off = 2 ** (bits - 1)
    inv = np.float32(1.0 / (off - 1))
    r32 = (a.amax(1) * torch.tensor(inv)).float()
    assert torch.equal(sc, r32.to(torch.float16))
    codes = codec.unpack_bits_rows(pk, k, bits)
    for r in range(X.shape[0]):
        lanes = torch.nonzero(mask[r]).flatten()            # increasing lane order
        q = torch.clamp(torch.round(X[r, lanes] / r32[r]), -off, off - 1) + off
        assert torch.equal(codes[r], q.to(torch.int32))
    assert int(codes.min()) >= 1                            # |q| <= 2^(b-1)-1: code 0 unused


def test_materialise_inverts_within_half_a_step():
    g = torch.Generator().manual_seed(5)
    X = torch.randn(16, 128, generator=g)
    bm, pk, sc = codec.build_rows(X, 81, 3)
    D = codec.packed_rows_materialise(bm, pk, sc, 128, 81, 3)
    mask = codec.unpack_bitmap_rows(bm, 128)
    assert torch.all(D[~mask] == 0)
    err = (D - X).abs()[mask].reshape(16, 81)
    assert torch.all(err <= sc.float().unsqueeze(1) * 0.5 * (1 + 2e-3) + 1e-6)


def test_zero_rows_and_ties():
    """All-zero rows keep the first k lanes and carry the ruler fp16(1/(2^(b-1)-1)); ties at the
    threshold go to the lowest lane (select_triton.py:188-193, test_encode_triton.py:296-325)."""
    X = torch.zeros(2, 128)
    X[1, :] = 1.0
    X[1, 100:] = 2.0                                        # 28 lanes of 2, then ties at 1
    bm, pk, sc = codec.build_rows(X, 81, 3)
    mask = codec.unpack_bitmap_rows(bm, 128)
    assert torch.equal(mask[0], torch.arange(128) < 81)
    assert sc[0].item() == float(torch.tensor(1.0 / 3, dtype=torch.float16))
    assert torch.equal(mask[1, 100:], torch.ones(28, dtype=torch.bool))
    assert torch.equal(mask[1, :53], torch.ones(53, dtype=torch.bool))
    assert not mask[1, 53:100].any()
    D = codec.packed_rows_materialise(bm, pk, sc, 128, 81, 3)
    assert float(D[0].abs().max()) == 0.0


def test_torch_scalar_division_semantics():
    """The reference writes rulers as `x / (2^(b-1)-1)`. torch on CPU divides exactly; the
    reference's CUDA store multiplies by the fp32 reciprocal (select_triton.py:76-84). The oracle
    exposes both; they differ only at the last fp32 ulp."""
    x = torch.rand(1 << 16, generator=torch.Generator().manual_seed(2)) * 10
    exact = torch.from_numpy((x.numpy().astype(np.float64) / 3).astype(np.float32))
    assert torch.equal(x / 3, exact)                                  # CPU torch: exact
    assert torch.equal(codec.ruler_div(x, 3, "cpu"), exact)
    gpu = codec.ruler_div(x, 3, "gpu")
    assert torch.equal(gpu, x * torch.tensor(np.float32(1 / 3)))
    diff = (gpu != exact)
    assert 0.1 < diff.float().mean() < 0.6                            # differs often ...
    ulps = (gpu.view(torch.int32) - exact.view(torch.int32)).abs()
    assert int(ulps.max()) <= 1                                       # ... by one ulp at most


def test_topk_mask_matches_torch_topk_on_tie_free_rows():
    g = torch.Generator().manual_seed(9)
    X = torch.randn(30, 128, generator=g)
    m = codec.topk_mask(X, 64)
    ref = torch.zeros_like(X, dtype=torch.bool)
    ref.scatter_(1, torch.topk(X.abs(), 64, dim=1).indices, True)
    assert torch.equal(m, ref)


def test_quant_rows_closed_form():
    g = torch.Generator().manual_seed(4)
    M = torch.randn(7, 33, generator=g)
    q, sc = codec.quant_rows(M, 8)
    s32 = M.abs().amax(1, keepdim=True) * torch.tensor(np.float32(1 / 127))
    assert torch.equal(sc, s32.to(torch.float16).reshape(-1))
    assert torch.equal(q, torch.clamp(torch.round(M / s32), -128, 127).to(torch.int8))
    assert int(q.abs().max(1).values.min()) == 127
