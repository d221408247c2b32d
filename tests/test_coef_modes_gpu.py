"""The fp16 and 4-bit (group-32) coefficient modes through the HIP kernels: K3 writes them, K1 and
K2 read them, against the CPU oracle (`oracle.coef_modes`).

The modes are this build's own (the reference writes int8 coefficients only), so parity is
"unpinned" against the reference; the oracle's definition of them is pinned on the CPU
(tests/test_coef_modes.py). Here, as for the int8 mode: the write's bytes are exact from the
kernel's own projection and residual, and the reads are within the path's tolerance
(2e-3 max-abs / 1e-3 mean-abs, float64 oracle) at the decode and continuation shapes."""
import pytest
import torch

from helpers import D, H, HQ, dec_pool_of, device_store, llama3_cache
from oracle import attend, codec, coef_modes, encode
from oracle.layout import layout_for_config
from vllm_ttkv import kernels, synth
from vllm_ttkv.layout import EXTENSION_CONFIGS

pytestmark = pytest.mark.gpu
DEV = "cuda"
MODES = sorted(EXTENSION_CONFIGS)
BASE = {"safe_fp16": "safe", "campaign4x_int4g32": "campaign4x"}
MAX_ABS, MEAN_ABS = 2e-3, 1e-3
SCALE = 128 ** -0.5
_CS = {}


def _cos_sin():
    if "cs" not in _CS:
        _CS["cs"] = llama3_cache(8200)
    return _CS["cs"]


@pytest.mark.parametrize("name", MODES)
def test_write_bytes_exact_from_kernel_projection(name):
    """Frozen writes of 9 tokens into scattered slots: the projection within fp32 tolerance of the
    oracle's, then every byte (coefficient field, residual rows, V rows, padding) exactly the
    oracle's from the kernel's own c and R; bytes outside the written slots untouched."""
    print(f"[coef-modes write] {name}", flush=True)
    lay = layout_for_config(EXTENSION_CONFIGS[name], 110)
    bcfg = codec.CONFIGS[BASE[name]]
    K = synth.keys(96 + 9, seed=21)
    dec = encode.fit_into_budget(K[:, :96].contiguous(), layout_for_config(bcfg, 110),
                                 bcfg)["decoder_f"]
    pinv = encode.pinv(dec)
    Knew = K[:, 96:].contiguous()
    V = synth.values(9, seed=22) * 0.3
    n = Knew.shape[1]
    slots = torch.tensor([5, 0, 17, 3, 30, 8, 11, 2, 25], dtype=torch.int64)
    C = lay.compressed_bytes_per_token()
    page = torch.zeros(32, C, dtype=torch.uint8, device=DEV)
    c_out = torch.zeros(n, lay.r1, device=DEV)
    r_out = torch.zeros(n, H * D, device=DEV)
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
    e = encode.encode_frozen_mode(Knew, dec, lay, pinv_m=pinv)
    assert (c - e["c"]).abs().max() <= 1e-4 * e["c"].abs().max() + 1e-7
    vals, q, s = coef_modes.quantise(c, lay.qbits)          # from the kernel's own c
    want_R = (Knew.permute(1, 0, 2).reshape(n, H * D) - vals @ dec)
    assert (R - want_R).abs().max() <= 1e-4
    R_k = R.reshape(n, H, D).permute(1, 0, 2).reshape(H * n, D)
    k_slots = encode.k_slots_from(lay, q, s, codec.build_rows(R_k, lay.res_k, lay.res_bits))
    v_slots = encode.v_slots_from(lay, encode.encode_v(V, lay))
    want = torch.cat([k_slots, v_slots], dim=1)
    got = page[slots]
    nbad = int((got != want).sum())
    assert nbad == 0, f"{name}: {nbad} of {want.numel()} bytes differ"
    untouched = torch.ones(32, dtype=torch.bool)
    untouched[slots] = False
    assert int(page[untouched].abs().sum()) == 0


def _decode(st, q):
    B = st["seq_lens"].numel()
    out = torch.zeros(B, HQ, D, dtype=torch.float16, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.decode_paged(st["play"], q.to(DEV), st["page"], st["block_size"], st["block_table"],
                         st["seq_lens"], torch.arange(B + 1, dtype=torch.int32, device=DEV),
                         int(st["seq_lens"].max()), st["dec_map"], st["dec_pool"],
                         _cos_sin().to(DEV), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    return out.float().cpu()


def _check(got, want, what):
    assert torch.isfinite(got).all(), what
    e = (got.double() - want).abs()
    print(f"{what}: max-abs {e.max():.3e} mean-abs {e.mean():.3e}", flush=True)
    assert e.max() <= MAX_ABS and e.mean() <= MEAN_ABS, f"{what}: {e.max():.3e} / {e.mean():.3e}"


@pytest.mark.parametrize("name", MODES)
def test_decode_read_matches_oracle(name):
    """K1 over a 3-request ragged batch (one short request, split-K chunks on the long ones),
    stores fitted and written on the device in the mode, against the float64 oracle reading the
    same slot bytes."""
    torch.set_num_threads(16)
    lens = [3000, 700, 8100]
    print(f"[coef-modes decode] {name} {lens}", flush=True)
    st = device_store(name, lens, seed=31, fit_on=1024)
    q = synth.queries(3, seed=32)
    got = _decode(st, q)
    want = attend.paged_decode(st["lay"], st["page"].cpu(), st["block_table"].cpu(),
                               st["seq_lens"].cpu(), torch.arange(4), q.float(), st["decoders"],
                               _cos_sin(), st["block_size"], SCALE, dtype=torch.float64)
    for r in range(3):
        _check(got[r:r + 1], want[r:r + 1], f"{name} request {r} (n={lens[r]})")


@pytest.mark.parametrize("name", MODES)
@pytest.mark.parametrize("Q", [16, 128])
def test_continuation_read_matches_oracle(name, Q):
    """K2 attention mode over 2 requests whose last Q tokens are the chunk (causal, p0 = n - Q):
    Q = 16 runs the fused short-chunk kernel, Q = 128 the expand + attend pair."""
    torch.set_num_threads(16)
    lens = [2100, 1500]
    print(f"[coef-modes continuation] {name} Q={Q}", flush=True)
    st = device_store(name, lens, seed=41, fit_on=1024)
    q = synth.queries(2 * Q, seed=42)
    qsl = torch.arange(0, 2 * Q + 1, Q, dtype=torch.int32)
    out = torch.zeros(2 * Q, HQ, D, dtype=torch.float32, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.prefill_paged(st["play"], q.to(DEV), st["page"], 16, st["block_table"],
                          st["seq_lens"], qsl.to(DEV), Q, max(lens), st["dec_map"],
                          st["dec_pool"], _cos_sin().to(DEV), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(st["lay"], st["page"].cpu(), st["block_table"].cpu(),
                                     st["seq_lens"].cpu(), qsl, q.float(), st["decoders"],
                                     _cos_sin(), 16, SCALE, dtype=torch.float64)
    got = out.cpu()
    for r in range(2):
        _check(got[r * Q:(r + 1) * Q], want[r], f"{name} Q={Q} request {r}")


@pytest.mark.parametrize("name", MODES)
@pytest.mark.parametrize("Q", [5, 200])
def test_scores_mode_matches_oracle(name, Q):
    """K2 scores mode (`[HQ, Q, n]`, causal -inf pattern exact) over one request's store in the
    mode: Q = 5 through the fused kernel, Q = 200 through the expand + scores pair."""
    from oracle.rope import cos_sin_from_cache
    torch.set_num_threads(16)
    n = 1900
    print(f"[coef-modes scores] {name} Q={Q}", flush=True)
    st = device_store(name, [n], seed=51, fit_on=1024)
    q = synth.queries(Q, seed=52)
    qsl = torch.tensor([0, Q], dtype=torch.int32)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = kernels.multi_scores_paged(st["play"], q.to(DEV), st["page"], 16, st["block_table"],
                                     st["seq_lens"], qsl.to(DEV), Q, n, st["dec_map"],
                                     st["dec_pool"], _cos_sin().to(DEV), SCALE, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    ks, _ = attend.gather_request(st["lay"], st["page"].cpu(), st["block_table"][0].cpu(), n, 16)
    cos, sin = cos_sin_from_cache(_cos_sin(), torch.arange(n), D)
    want = attend.raw_scores_multi(st["lay"], ks, st["decoders"][0],
                                   q.permute(1, 0, 2).double(), cos, sin, SCALE, p0=n - Q,
                                   dtype=torch.float64)
    got = got.double().cpu()
    assert torch.equal(torch.isneginf(got), torch.isneginf(want)), "mask pattern"
    fin = torch.isfinite(want)
    _check(got[fin], want[fin], f"{name} scores Q={Q}")
