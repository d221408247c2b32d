"""Parity at the benchmark's full sizes, HIP path vs the float64 oracle.

The stores are full size and built the way serving builds them (`helpers.device_store`: fit of the
first chunk on the device, every token packed by K3); the oracle then reads the SAME slot bytes
through the reference's own request loop (`oracle.attend.paged_decode` / `paged_continuation`,
vllm_ttkv/impl.py:452-540, 725-778). These are the shapes where the approximations that grow with
context would show: fp16-rounded P' weights over 14k-16k keys, the lazy max rescaling, the
split-K combine over many chunks (reference test pattern: tests/test_impl_decode.py:259-329).

Tolerance (north star): 2e-3 max-abs / 1e-3 mean-abs on the fp16 outputs (and on the scores of
the multi-query kernel), against float64."""
import pytest
import torch

from helpers import HQ, config3_lens, device_store, llama3_cache
from oracle import attend
from vllm_ttkv import kernels, synth

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-3, 1e-3
SCALE = 128 ** -0.5
_CACHE = {}


def _cos_sin():
    if "cs" not in _CACHE:
        _CACHE["cs"] = llama3_cache(16400)
    return _CACHE["cs"]


def _k1(st, q, out_dtype=torch.float16):
    B = st["seq_lens"].numel()
    out = torch.zeros(B, HQ, 128, dtype=out_dtype, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.decode_paged(st["play"], q.cuda(), st["page"], st["block_size"], st["block_table"],
                         st["seq_lens"], torch.arange(B + 1, dtype=torch.int32, device="cuda"),
                         int(st["seq_lens"].max()), st["dec_map"], st["dec_pool"],
                         _cos_sin().cuda(), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0, f"device error word {int(err.item())}"
    return out.float().cpu()


def _oracle_decode(st, q):
    return attend.paged_decode(st["lay"], st["page"].cpu(), st["block_table"].cpu(),
                               st["seq_lens"].cpu(), torch.arange(q.shape[0] + 1), q.float(),
                               st["decoders"], _cos_sin(), st["block_size"], SCALE,
                               dtype=torch.float64)


def _check(got, want, what):
    assert torch.isfinite(got).all(), what
    e = (got.double() - want).abs()
    print(f"{what}: max-abs {e.max():.3e} mean-abs {e.mean():.3e}", flush=True)
    assert e.max() <= MAX_ABS and e.mean() <= MEAN_ABS, f"{what}: {e.max():.3e} / {e.mean():.3e}"


@pytest.mark.parametrize("n", [1082, 4322, 8642, 14402])
def test_config2_batch1_contexts(n):
    """Config 2: B = 1 at each context, four layers (independent stores and queries)."""
    torch.set_num_threads(16)
    for layer in range(4):
        print(f"config2 n={n} layer={layer}", flush=True)
        st = device_store("safe", [n], seed=200 + 10 * layer + n % 97)
        q = synth.queries(1, seed=layer + n)
        _check(_k1(st, q), _oracle_decode(st, q), f"config2 n={n} layer {layer}")


@pytest.mark.parametrize("layer", range(3))
def test_config3_batch8_random_contexts(layer):
    """Config 3: 8 requests, contexts seeded U[1000, 14400], shuffled block table, one launch;
    three layers (independent stores and queries over the same contexts)."""
    torch.set_num_threads(16)
    lens = config3_lens()
    print(f"config3 contexts {lens} layer {layer}", flush=True)
    st = device_store("safe", lens, seed=3 + 100 * layer)
    q = synth.queries(8, seed=5 + layer)
    got = _k1(st, q)
    want = _oracle_decode(st, q)
    for r in range(8):
        _check(got[r:r + 1], want[r:r + 1], f"config3 layer {layer} request {r} (n={lens[r]})")


def test_headline_batch8_at_14402():
    """The bench's headline shape: 8 requests of 14,402 tokens in one launch (8 chunks per
    (request, head), the in-launch combine of each), against the oracle."""
    torch.set_num_threads(16)
    lens = [14402] * 8
    st = device_store("safe", lens, seed=77)
    q = synth.queries(8, seed=78)
    got = _k1(st, q)
    want = _oracle_decode(st, q)
    for r in range(8):
        _check(got[r:r + 1], want[r:r + 1], f"headline request {r}")


def _config4_store():
    if "c4" not in _CACHE:
        torch.set_num_threads(16)
        _CACHE["c4"] = device_store("safe", [7656] * 4, seed=4)
    return _CACHE["c4"]


def test_config4_continuation_attention():
    """Config 4: 4 requests, 7,400 cached + a 256-query chunk (the chunk is in the store,
    p0 = 7,400), causal; every chunk in ONE K2 launch, against the continuation oracle."""
    st = _config4_store()
    Q, n = 256, 7656
    q = synth.queries(4 * Q, seed=44)
    qsl = torch.arange(0, 4 * Q + 1, Q, dtype=torch.int32)
    out = torch.zeros(4 * Q, HQ, 128, dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.prefill_paged(st["play"], q.cuda(), st["page"], 16, st["block_table"],
                          st["seq_lens"], qsl.cuda(), Q, n, st["dec_map"], st["dec_pool"],
                          _cos_sin().cuda(), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    got = out.float().cpu()
    want = attend.paged_continuation(st["lay"], st["page"].cpu(), st["block_table"].cpu(),
                                     st["seq_lens"].cpu(), qsl, q.float(), st["decoders"],
                                     _cos_sin(), 16, SCALE, dtype=torch.float64)
    for r in range(4):
        _check(got[r * Q:(r + 1) * Q], want[r], f"config4 attention request {r}")


@pytest.mark.parametrize("r", [0, 3])
def test_config4_continuation_scores(r):
    """Config 4, score mode (`krt_multi_from_slots`): [HQ, 256, 7656] with the causal -inf
    pattern compared exactly."""
    st = _config4_store()
    Q, n = 256, 7656
    q = synth.queries(Q, seed=45 + r)
    qsl = torch.tensor([0, Q], dtype=torch.int32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = kernels.multi_scores_paged(st["play"], q.cuda(), st["page"], 16,
                                     st["block_table"][r:r + 1].contiguous(),
                                     st["seq_lens"][r:r + 1].contiguous(), qsl, Q, n,
                                     st["dec_map"], st["dec_pool"], _cos_sin().cuda(), SCALE,
                                     error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    got = got.double().cpu()
    k, v = attend.gather_request(st["lay"], st["page"].cpu(), st["block_table"][r].cpu(), n, 16)
    from oracle.rope import cos_sin_from_cache
    cos, sin = cos_sin_from_cache(_cos_sin(), torch.arange(n), 128)
    want = attend.raw_scores_multi(st["lay"], k, st["decoders"][r], q.permute(1, 0, 2), cos, sin,
                                   SCALE, p0=n - Q, dtype=torch.float64)
    assert torch.equal(torch.isneginf(got), torch.isneginf(want)), "causal mask pattern"
    fin = torch.isfinite(want)
    _check(got[fin], want[fin], f"config4 scores request {r}")


def test_config5_campaign4x_write_then_read():
    """Config 5: campaign4x (4-bit codes), 8 requests at 16k context. K3 encodes and packs one
    new K/V per request (decoder projection, bitmap select, quantise, slot write); its bytes must
    equal the oracle's packing of K3's own projection and residual exactly; then K1 reads all
    8 x 16,385 tokens in one launch against the oracle."""
    from oracle import codec, encode
    torch.set_num_threads(16)
    n, B, H, D = 16384, 8, 8, 128
    # one block of headroom per request so the new token has a slot
    st = device_store("campaign4x", [n + 1] * B, seed=5)
    lay, play = st["lay"], st["play"]
    # the step's new token of each request: position n, written over its slot
    Knew = synth.keys(B, seed=555)                            # [H, B, d]: one per request
    Vnew = synth.values(B, seed=556)
    bt = st["block_table"].cpu()
    slots = torch.tensor([int(bt[r, n // 16]) * 16 + n % 16 for r in range(B)], dtype=torch.int64)
    c_out = torch.zeros(B, lay.r1, device="cuda")
    r_out = torch.zeros(B, H * D, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.write_paged(play, Knew.permute(1, 0, 2).contiguous().cuda(),
                        Vnew.permute(1, 0, 2).contiguous().cuda(), slots.cuda(),
                        torch.arange(B + 1, dtype=torch.int32, device="cuda"), st["block_table"],
                        st["dec_map"], st["dec_pool"], st["pinv_pool"], st["page"],
                        coeff_out=c_out, resid_out=r_out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    c, R = c_out.cpu(), r_out.cpu()
    # float stages at fp32 tolerance against each request's own decoder
    for r in range(B):
        pinv = st["pinv_pool"][r].cpu().t()
        c_ref = encode.project(Knew[:, r:r + 1].contiguous(), pinv)
        assert (c[r:r + 1] - c_ref).abs().max() <= 1e-4 * c_ref.abs().max() + 1e-7
    cq, cs = encode.quantise_coeffs(c)
    R_k = R.reshape(B, H, D).permute(1, 0, 2).reshape(H * B, D)
    for r in range(B):
        R_ref = encode.residual(Knew[:, r:r + 1].contiguous(), cq[r:r + 1], cs[r:r + 1],
                                st["decoders"][r])                      # [H, d]
        assert (R_k.reshape(H, B, D)[:, r] - R_ref).abs().max() <= 1e-4
    k_slots = encode.k_slots_from(lay, cq, cs.to(torch.float16).reshape(-1),
                                  codec.build_rows(R_k, lay.res_k, lay.res_bits))
    v_slots = encode.v_slots_from(lay, encode.encode_v(Vnew, lay))
    want_bytes = torch.cat([k_slots, v_slots], dim=1)
    got_bytes = st["page"][slots.cuda()].cpu()
    nbad = int((got_bytes != want_bytes).sum())
    assert nbad == 0, f"config5 write: {nbad} of {want_bytes.numel()} bytes differ"
    # then the read over the whole store, the new token included
    q = synth.queries(B, seed=57)
    got = _k1(st, q)
    want = _oracle_decode(st, q)
    for r in range(B):
        _check(got[r:r + 1], want[r:r + 1], f"config5 request {r} (n={n + 1})")
