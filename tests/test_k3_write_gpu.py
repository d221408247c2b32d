"""K3 (write/encode) on the GPU against the CPU oracle.

Bytes are pinned bit-exactly from the quantiser inputs on (the kernel's own projection c and
residual R, which it can export), exactly as the reference pins its fused write against the torch
packer from the same FittedK (tests/test_encode_triton.py:100-121 in the reference). The float
stages (projection, reconstruction) are checked at fp32 tolerance against the oracle."""
import pytest
import torch

from helpers import D, H, dec_pool_of
from oracle import codec, encode
from oracle.layout import layout_for_config, unpack_v_slots
from oracle import attend
from vllm_ttkv import kernels, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(cfg_name, n_new, seed, r1=110, fit_on=96):
    cfg = codec.CONFIGS[cfg_name]
    lay = layout_for_config(cfg, r1=r1)
    K = synth.keys(fit_on + n_new, seed=seed)
    fk = encode.fit_into_budget(K[:, :fit_on].contiguous(), lay, cfg)
    dec = fk["decoder_f"]
    pinv = encode.pinv(dec)
    Knew = K[:, fit_on:].contiguous()                       # [H, n, d]
    V = synth.values(n_new, seed=seed + 1) * 0.3
    return lay, dec, pinv, Knew, V


def _run(lay, dec, pinv, Knew, V, slots, n_slots, v_dtype=torch.float32, cq_in=None, cs_in=None):
    n = Knew.shape[1]
    C = lay.compressed_bytes_per_token()
    page = torch.zeros(n_slots, C, dtype=torch.uint8, device=DEV)
    bt = torch.zeros(1, 1, dtype=torch.int32, device=DEV)    # request 0 owns block 0
    dec_map = torch.zeros(1, dtype=torch.int32, device=DEV)  # block 0 -> decoder slot 0
    qsl = torch.tensor([0, n], dtype=torch.int32, device=DEV)
    c_out = torch.zeros(n, lay.r1, device=DEV)
    r_out = torch.zeros(n, H * D, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.write_paged(lay, Knew.permute(1, 0, 2).contiguous().to(DEV),
                        V.permute(1, 0, 2).contiguous().to(v_dtype).to(DEV),
                        slots.to(DEV), qsl, bt, dec_map, dec_pool_of([dec], DEV),
                        pinv.t().unsqueeze(0).contiguous().to(DEV), page,
                        coeff_q_in=None if cq_in is None else cq_in.to(DEV),
                        coeff_scale_in=None if cs_in is None else cs_in.to(DEV),
                        coeff_out=c_out, resid_out=r_out, error_word=err)
    torch.cuda.synchronize()
    return page.cpu(), c_out.cpu(), r_out.cpu(), int(err.item())


@pytest.mark.parametrize("cfg", ["safe", "tight", "campaign4x"])
def test_write_bytes_exact_from_quantiser_inputs(cfg):
    lay, dec, pinv, Knew, V = _setup(cfg, 9, seed=21)
    _check_write(lay, dec, pinv, Knew, V, cfg)


@pytest.mark.parametrize("r1", [150, 200])
def test_write_large_rank_budgets(r1):
    """Rank budgets past 128 (the decoder pool pads them to 192 / 256 ranks, read as whole
    64-rank chunks per lane in the residual): a codec-form decoder with every rank active
    (int8 rows times fp16 rank rulers, as the codec stores them) and its pseudo-inverse."""
    lay = layout_for_config(codec.CONFIGS["safe"], r1=r1)
    g = torch.Generator().manual_seed(r1)
    q = torch.randint(-127, 128, (r1, H * D), generator=g).float()
    ruler = (torch.rand(r1, generator=g) * 0.02 + 0.005).half().float()
    dec = q * ruler[:, None]
    pinv = encode.pinv(dec)
    Knew = synth.keys(9, seed=r1 + 1)
    V = synth.values(9, seed=r1 + 2) * 0.3
    _check_write(lay, dec, pinv, Knew, V, f"r1={r1}")


def _check_write(lay, dec, pinv, Knew, V, label):
    slots = torch.tensor([5, 0, 17, 3, 30, 8, 11, 2, 25], dtype=torch.int64)
    print(f"[k3] {label}", flush=True)
    page, c, R, err = _run(lay, dec, pinv, Knew, V, slots, 32)
    assert err == 0
    # float stages at fp32 tolerance
    c_ref = encode.project(Knew, pinv)
    assert (c - c_ref).abs().max() <= 1e-4 * c_ref.abs().max() + 1e-7
    cq, cs = encode.quantise_coeffs(c)                      # from the kernel's own c
    R_ref = encode.residual(Knew, cq, cs, dec)              # [H*n, d] (head, token)
    R_k = R.reshape(-1, H, D).permute(1, 0, 2).reshape(H * Knew.shape[1], D)
    assert (R_k - R_ref).abs().max() <= 1e-4
    # bytes: bit-exact from (c, R, V)
    k_slots = encode.k_slots_from(lay, cq, cs.to(torch.float16).reshape(-1),
                                  codec.build_rows(R_k, lay.res_k, lay.res_bits))
    v_slots = encode.v_slots_from(lay, encode.encode_v(V, lay))
    want = torch.cat([k_slots, v_slots], dim=1)
    got = page[slots]
    nbad = int((got != want).sum())
    assert nbad == 0, f"{label}: {nbad} of {want.numel()} bytes differ"
    untouched = torch.ones(32, dtype=torch.bool)
    untouched[slots] = False
    assert int(page[untouched].abs().sum()) == 0, "bytes outside the written slots changed"


def test_write_bf16_value_is_exact():
    lay, dec, pinv, Knew, V = _setup("safe", 5, seed=7)
    V = V.to(torch.bfloat16).float()                        # values representable in bf16
    slots = torch.arange(5, dtype=torch.int64)
    page, c, R, err = _run(lay, dec, pinv, Knew, V, slots, 8, v_dtype=torch.bfloat16)
    v_slots = encode.v_slots_from(lay, encode.encode_v(V, lay))
    assert torch.equal(page[slots, lay.v_offset:], v_slots)


def test_ties_and_zero_rows_follow_the_lowest_lane_rule():
    """Three-value alphabet (most lanes tie) and all-zero rows: the oracle uses the same
    tie rule (lowest lane index), so bytes must be identical, and zero rows carry the ruler
    fp16(1 / (2^(b-1)-1)) (test_encode_triton.py:256-325 in the reference)."""
    lay, dec, pinv, Knew, _ = _setup("safe", 6, seed=13)
    g = torch.Generator().manual_seed(14)
    V = torch.randint(0, 3, (H, 6, D), generator=g).float() - 1.0
    V[:, 4] = 0.0
    slots = torch.arange(6, dtype=torch.int64)
    page, _, _, err = _run(lay, dec, pinv, Knew, V, slots, 8)
    want = encode.v_slots_from(lay, encode.encode_v(V, lay))
    assert torch.equal(page[slots, lay.v_offset:], want)
    sc = unpack_v_slots(lay, page[slots, lay.v_offset:])[2].reshape(H, 6)
    assert torch.all(sc[:, 4] == torch.tensor(1.0 / 3, dtype=torch.float16))
    dense = attend.dense_v_from_slots(lay, page[slots, lay.v_offset:])
    assert float(dense[:, 4].abs().max()) == 0.0


def test_fit_coefficients_path():
    """A first chunk is written with its fit's own coefficients (encode.py:257-298)."""
    cfg = codec.CONFIGS["safe"]
    lay = layout_for_config(cfg, r1=110)
    K = synth.keys(40, seed=3)
    V = synth.values(40, seed=4)
    fk = encode.fit_into_budget(K, lay, cfg)
    dec = fk["decoder_f"]
    # fp32 coefficient ruler of the fit (build_k_layer keeps it fp32 for the residual)
    cs32 = fk["coeff_scale"].float()
    slots = torch.arange(40, dtype=torch.int64)
    page, _, R, err = _run(lay, dec, encode.pinv(dec), K, V, slots, 40,
                           cq_in=fk["coeff_q"], cs_in=cs32)
    assert err == 0
    R_k = R.reshape(-1, H, D).permute(1, 0, 2).reshape(H * 40, D)
    R_ref = encode.residual(K, fk["coeff_q"], cs32.unsqueeze(1), dec)
    assert (R_k - R_ref).abs().max() <= 1e-4
    k_slots = encode.k_slots_from(lay, fk["coeff_q"], cs32.to(torch.float16),
                                  codec.build_rows(R_k, lay.res_k, lay.res_bits))
    assert torch.equal(page[:, :lay.k_slot_bytes], k_slots)


def test_slot_refusals_set_the_error_word_and_write_nothing():
    """A slot id past the cache is refused (error bit 4) and writes nothing; a negative id is
    vLLM's PAD_SLOT_ID (padded tokens of a replayed graph): skipped silently, as vLLM's own cache
    writers do, while the other tokens are written."""
    lay, dec, pinv, Knew, V = _setup("safe", 3, seed=5)
    for bad, want_err in (([0, -1, 2], 0), ([0, 1, 99], 4)):
        page, _, _, err = _run(lay, dec, pinv, Knew, V, torch.tensor(bad, dtype=torch.int64), 8)
        assert err == want_err, f"{bad}: error word {err}"
        bad_i = 1 if bad[1] == -1 else 2
        ok_rows = [j for j in range(3) if j != bad_i]
        assert all(int(page[bad[j]].abs().sum()) > 0 for j in ok_rows)
        written = {bad[j] for j in ok_rows}
        assert all(int(page[s].abs().sum()) == 0 for s in range(8) if s not in written)


@pytest.mark.parametrize("case", ["ref_encode_safe_r16", "ref_encode_campaign4x_r64"])
def test_frozen_write_against_reference_vectors(case):
    """K3 on the reference's own inputs (tests/golden/, written by the reference's
    `encode_frozen` / `encode_v` on the CPU). The reference's CPU rulers are divisions and its
    CPU lane selection on a magnitude tie is `torch.topk`'s, so bytes may differ in a few places;
    the stores must agree byte-for-byte almost everywhere. Decoded K agrees within a coefficient
    step; decoded V within a residual step, or a tied lane's own magnitude where the two
    selections keep different lanes."""
    import pathlib
    import numpy as np
    z = np.load(pathlib.Path(__file__).parent / "golden" / f"{case}.npz")
    name = str(z["config"])
    lay = layout_for_config(codec.CONFIGS[name], r1=int(z["r1"]))
    dec = torch.from_numpy(z["fit_decoder_f"])
    pinv = torch.from_numpy(z["pinv"])
    K1 = torch.from_numpy(z["K1"]).float()
    n = K1.shape[1]
    V = torch.from_numpy(z["V0"]).float()[:, :n].contiguous()
    slots = torch.arange(n, dtype=torch.int64)
    page, _, _, err = _run(lay, dec, pinv, K1, V, slots, n)
    assert err == 0
    want = torch.cat([torch.from_numpy(z["frozen_k_slots"]),
                      torch.from_numpy(z["v_slots"])[:n]], dim=1)
    frac = float((page != want).float().mean())
    assert frac < 0.01, f"{case}: {frac:.4f} of bytes differ"
    kg = attend.dense_k_from_slots(lay, page[:, :lay.k_slot_bytes], dec)
    kr = attend.dense_k_from_slots(lay, want[:, :lay.k_slot_bytes], dec)
    assert float((kg - kr).abs().max()) <= 0.05 * float(K1.abs().max())
    vg = attend.dense_v_from_slots(lay, page[:, lay.v_offset:])
    vr = attend.dense_v_from_slots(lay, want[:, lay.v_offset:])
    assert float((vg - vr).abs().max()) <= 0.3 * float(V.abs().max())


@pytest.mark.parametrize("case", ["ref_encode_safe_r16", "ref_encode_campaign4x_r64"])
def test_device_pinv_against_reference_vectors(case):
    """The product's pinv (`vllm_ttkv.encode.KDecoder.pinv`, torch.linalg.pinv on the device, as
    the reference's encode.py:197-211 on its CUDA path) against the pinv the reference wrote on the
    CPU for the same decoder. The campaign4x decoder has rank 26 of 64 rows (the rest exactly
    zero), so the zero rows' pinv columns must come out exactly zero. Then the Moore-Penrose
    identities on the device result, and a frozen write driven by the device pinv against the
    reference's bytes, at the bar of the reference-pinv test above."""
    import pathlib
    import numpy as np
    from vllm_ttkv.encode import KDecoder
    z = np.load(pathlib.Path(__file__).parent / "golden" / f"{case}.npz")
    dec = torch.from_numpy(z["fit_decoder_f"])
    want = torch.from_numpy(z["pinv"]).double()
    got = KDecoder(dec.to(DEV)).pinv.cpu()
    assert got.shape == want.shape and got.dtype == torch.float32
    scale = float(want.abs().max())
    err = float((got.double() - want).abs().max())
    assert err <= 1e-4 * scale, f"{case}: pinv off by {err:.3e} (max |pinv| {scale:.3e})"
    zero_rows = (dec.abs().sum(dim=1) == 0).nonzero().flatten()
    if case.startswith("ref_encode_campaign4x"):
        assert len(zero_rows) == 64 - 26
    assert torch.equal(got[:, zero_rows], torch.zeros(got.shape[0], len(zero_rows)))
    D64, P64 = dec.double(), got.double()
    assert float((D64 @ P64 @ D64 - D64).abs().max()) <= 1e-5 * float(D64.abs().max())
    assert float((P64 @ D64 @ P64 - P64).abs().max()) <= 1e-4 * scale
    # frozen write with the device pinv: the reference's bytes almost everywhere
    lay = layout_for_config(codec.CONFIGS[str(z["config"])], r1=int(z["r1"]))
    K1 = torch.from_numpy(z["K1"]).float()
    n = K1.shape[1]
    V = torch.from_numpy(z["V0"]).float()[:, :n].contiguous()
    page, _, _, e = _run(lay, dec, got, K1, V, torch.arange(n, dtype=torch.int64), n)
    assert e == 0
    ref = torch.cat([torch.from_numpy(z["frozen_k_slots"]), torch.from_numpy(z["v_slots"])[:n]],
                    dim=1)
    frac = float((page != ref).float().mean())
    assert frac < 0.01, f"{case}: {frac:.4f} of bytes differ with the device pinv"


def test_workspace_shared_across_token_counts():
    """One workspace serves writes of different sizes in turn (a serving loop's token count
    changes every step): each write's bytes equal those of the same write with a fresh
    workspace. The arrival counters sit at a fixed place that no call's partials overlap."""
    lay, dec, pinv, Knew, V = _setup("safe", 120, seed=51)
    C = lay.compressed_bytes_per_token()
    Kt = Knew.permute(1, 0, 2).contiguous().to(DEV)
    Vt = V.permute(1, 0, 2).contiguous().to(DEV)
    bt = torch.zeros(1, 1, dtype=torch.int32, device=DEV)
    dec_map = torch.zeros(1, dtype=torch.int32, device=DEV)
    shared = kernels.write_workspace(lay, 120, DEV)

    def write(lo, hi, ws):
        n = hi - lo
        page = torch.zeros(128, C, dtype=torch.uint8, device=DEV)
        err = torch.zeros(1, dtype=torch.int32, device=DEV)
        kernels.write_paged(lay, Kt[lo:hi], Vt[lo:hi], torch.arange(n, dtype=torch.int64, device=DEV),
                            torch.tensor([0, n], dtype=torch.int32, device=DEV), bt, dec_map,
                            dec_pool_of([dec], DEV), pinv.t().unsqueeze(0).contiguous().to(DEV), page,
                            error_word=err, workspace=ws)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        return page.cpu()

    for lo, hi in [(0, 50), (0, 100), (30, 50), (0, 120), (7, 8), (0, 100)]:
        got = write(lo, hi, shared)
        want = write(lo, hi, None)
        assert torch.equal(got, want), f"tokens {lo}:{hi} with a shared workspace"
    assert int(shared[:65536].abs().sum()) == 0, "counters left non-zero"


def test_write_flags_the_decoder_slots_it_uses():
    """`dec_used` receives 1 for the decoder slot of every request with a written token, and
    nothing for the others: the registry's last-use record (rope_store evicts by it)."""
    lay, dec, pinv, Knew, V = _setup("safe", 4, seed=9)
    C = lay.compressed_bytes_per_token()
    page = torch.zeros(16, C, dtype=torch.uint8, device=DEV)
    bt = torch.tensor([[3], [1]], dtype=torch.int32, device=DEV)   # request keys 3 and 1
    dec_map = torch.tensor([-1, 4, -1, 2, -1], dtype=torch.int32, device=DEV)
    pool = dec_pool_of([dec] * 6, DEV)
    pinvs = pinv.t().unsqueeze(0).repeat(6, 1, 1).contiguous().to(DEV)
    used = torch.zeros(6, dtype=torch.int32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.write_paged(lay, Knew.permute(1, 0, 2).contiguous().to(DEV),
                        V.permute(1, 0, 2).contiguous().to(DEV),
                        torch.tensor([0, 5, -1, 9], dtype=torch.int64, device=DEV),
                        torch.tensor([0, 3, 4], dtype=torch.int32, device=DEV), bt, dec_map,
                        pool, pinvs, page, error_word=err, dec_used=used)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert used.cpu().tolist() == [0, 0, 1, 0, 1, 0]


@pytest.mark.parametrize("Hk,r1", [(4, 110), (2, 40), (8, 7)])
def test_write_fewer_kv_heads_and_ranks(Hk, r1):
    """K3 at other shapes than the serving ones: 4 or 2 KV heads (the projection reads H*d = 512
    or 256 dims per rank row, so lanes past them stay idle) and a rank budget below one 4-rank
    slice per wave; bytes exact from the kernel's own c and R, every other slot untouched."""
    from oracle.layout import Layout
    lay = Layout(H=Hk, d=D, r1=r1, qbits=8, res_k=81, res_bits=3, v_lanes=81, v_bits=3)
    g = torch.Generator().manual_seed(100 + Hk + r1)
    q = torch.randint(-127, 128, (r1, Hk * D), generator=g).float()
    dec = q * ((torch.rand(r1, generator=g) * 0.02 + 0.005).half().float())[:, None]
    pinv = encode.pinv(dec)
    Knew = synth.keys(7, H=Hk, seed=r1)
    V = synth.values(7, H=Hk, seed=r1 + 1) * 0.3
    n = 7
    slots = torch.tensor([4, 0, 9, 2, 11, 6, 1], dtype=torch.int64)
    print(f"[k3] H={Hk} r1={r1}", flush=True)
    page = torch.zeros(12, lay.compressed_bytes_per_token(), dtype=torch.uint8, device=DEV)
    c_out = torch.zeros(n, r1, device=DEV)
    r_out = torch.zeros(n, Hk * D, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.write_paged(lay, Knew.permute(1, 0, 2).contiguous().to(DEV),
                        V.permute(1, 0, 2).contiguous().to(DEV), slots.to(DEV),
                        torch.tensor([0, n], dtype=torch.int32, device=DEV),
                        torch.zeros(1, 1, dtype=torch.int32, device=DEV),
                        torch.zeros(1, dtype=torch.int32, device=DEV), dec_pool_of([dec], DEV),
                        pinv.t().unsqueeze(0).contiguous().to(DEV), page, coeff_out=c_out,
                        resid_out=r_out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    page, c, R = page.cpu(), c_out.cpu(), r_out.cpu()
    c_ref = encode.project(Knew, pinv)
    assert (c - c_ref).abs().max() <= 1e-4 * c_ref.abs().max() + 1e-7
    cq, cs = encode.quantise_coeffs(c)
    R_k = R.reshape(n, Hk, D).permute(1, 0, 2).reshape(Hk * n, D)
    assert (R_k - encode.residual(Knew, cq, cs, dec)).abs().max() <= 1e-4
    want = torch.cat([encode.k_slots_from(lay, cq, cs.to(torch.float16).reshape(-1),
                                          codec.build_rows(R_k, lay.res_k, lay.res_bits)),
                      encode.v_slots_from(lay, encode.encode_v(V, lay))], dim=1)
    assert int((page[slots] != want).sum()) == 0
    untouched = torch.ones(12, dtype=torch.bool)
    untouched[slots] = False
    assert int(page[untouched].abs().sum()) == 0
