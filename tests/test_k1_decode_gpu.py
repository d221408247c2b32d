"""K1 (fused paged decode read) on the GPU against the CPU oracle.

Tolerance (north star): attention outputs within 2e-3 max-abs and 1e-3 mean-abs against the
fp32 (here float64) oracle, with the kernel writing fp16."""
import pytest
import torch

from helpers import HQ, dec_pool_of, fitted_store, llama3_cache, paged
from oracle import attend, rope as orope
from vllm_ttkv import kernels, synth

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-3, 1e-3


def _run_k1(stores, q, cache, block_size=16, seed=0, out_dtype=torch.float16, workspace=None):
    pg = paged(stores, block_size, seed)
    dev = "cuda"
    lay = stores[0]["lay"]
    B = len(stores)
    dec_pool = dec_pool_of([s["decoder"] for s in stores], dev)
    dec_map = torch.full((pg["num_blocks"],), -1, dtype=torch.int32)
    for r in range(B):
        dec_map[pg["block_table"][r, 0]] = r
    qsl = torch.arange(B + 1, dtype=torch.int32)
    out = torch.zeros(B, q.shape[1], 128, dtype=out_dtype, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.decode_paged(lay, q.to(dev), pg["page"].to(dev), block_size,
                         pg["block_table"].to(dev), pg["seq_lens"].to(dev), qsl.to(dev),
                         int(pg["seq_lens"].max()), dec_map.to(dev), dec_pool,
                         cache.to(dev), 128 ** -0.5, out=out, error_word=err,
                         workspace=workspace)
    torch.cuda.synchronize()
    assert int(err.item()) == 0, f"device error word {int(err.item())}"
    return out.float().cpu(), pg


def _oracle(stores, q, cache, pg, block_size=16):
    lay = stores[0]["lay"]
    flat = pg["page"]
    return attend.paged_decode(lay, flat, pg["block_table"], pg["seq_lens"],
                               torch.arange(len(stores) + 1), q.float(),
                               [s["decoder"] for s in stores], cache, block_size, 128 ** -0.5,
                               dtype=torch.float64)


def _check(got, want, what):
    e = (got.double() - want).abs()
    print(f"{what}: max-abs {e.max():.3e} mean-abs {e.mean():.3e}")
    assert torch.isfinite(got).all(), what
    assert e.max() <= MAX_ABS and e.mean() <= MEAN_ABS, f"{what}: {e.max():.3e} / {e.mean():.3e}"


def test_config1_single_request_safe():
    """one request, 1082 tokens, Llama-3.2-3B shapes, safe, r1=110."""
    st = fitted_store("safe", 1082, seed=1)
    q = synth.queries(1, seed=1)
    cache = llama3_cache(16384)
    got, pg = _run_k1([st], q, cache)
    _check(got, _oracle([st], q, cache, pg), "config1")


@pytest.mark.parametrize("cfg", ["safe", "campaign4x", "tight"])
def test_ragged_batch_per_request_decoders(cfg):
    """Ragged lengths (incl. sub-tile and multi-chunk), each request with its own decoder."""
    lens = [1, 64, 100, 129, 700, 2500]
    stores = [fitted_store(cfg, n, seed=10 + i) for i, n in enumerate(lens)]
    q = synth.queries(len(lens), seed=3)
    cache = llama3_cache(4096)
    got, pg = _run_k1(stores, q, cache, seed=5)
    _check(got, _oracle(stores, q, cache, pg), f"ragged {cfg}")


def test_bf16_query_and_output():
    st = fitted_store("safe", 300, seed=2)
    q = synth.queries(1, seed=4, dtype=torch.bfloat16)
    cache = llama3_cache(512)
    got, pg = _run_k1([st], q, cache, out_dtype=torch.bfloat16)
    e = (got.double() - _oracle([st], q, cache, pg)).abs()
    assert e.max() <= 1e-2 and e.mean() <= 2e-3  # bf16 output rounding (8-bit mantissa)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_queries_in_rows_that_are_not_16_byte_aligned(dtype):
    """Query rows at a stride of HQ*d + 2 elements (a view into a wider buffer) are not 16-byte
    aligned, so the kernel loads them element by element instead of in wide loads: same result."""
    lens = [300, 130, 64]
    stores = [fitted_store("safe", n, seed=90 + i) for i, n in enumerate(lens)]
    q = synth.queries(len(lens), seed=15).to(dtype)
    wide = torch.zeros(len(lens), q.shape[1] * 128 + 2, dtype=dtype)
    wide[:, :q.shape[1] * 128] = q.reshape(len(lens), -1)
    qv = wide.to("cuda")[:, :q.shape[1] * 128].view(len(lens), q.shape[1], 128)
    assert qv.stride(0) == q.shape[1] * 128 + 2
    cache = llama3_cache(512)
    got, pg = _run_k1(stores, qv, cache, seed=16)
    _check(got, _oracle(stores, q, cache, pg), f"strided {dtype} queries")


def test_rotation_is_applied_per_row():
    """Negative control (test_reference.py:81-113 restated on the kernel): rotating every row by
    its neighbour's position must change the output by far more than the tolerance."""
    st = fitted_store("safe", 200, seed=6)
    q = synth.queries(1, seed=6)
    cache = llama3_cache(400)
    got, pg = _run_k1([st], q, cache)
    rolled = torch.cat([cache[1:], cache[:1]])          # row t holds t+1's angles
    want_rolled = _oracle([st], q, rolled, pg)
    assert (got.double() - want_rolled).abs().max() > 10 * MAX_ABS


def test_write_then_read_loop():
    """K3 writes a request's tokens (first chunk with its fit, the rest by frozen projection),
    then K1 reads them back; the oracle decodes the same (kernel-written) bytes."""
    from oracle import codec, encode
    from oracle.layout import layout_for_config
    cfg = codec.CONFIGS["safe"]
    lay = layout_for_config(cfg, r1=110)
    T, fit_on, bs = 300, 128, 16
    K = synth.keys(T, seed=31)
    V = synth.values(T, seed=31)
    fk = encode.fit_into_budget(K[:, :fit_on].contiguous(), lay, cfg)
    dec = fk["decoder_f"]
    dev = "cuda"
    bt, nblk = synth.shuffled_block_table([T], bs, seed=2, extra_blocks=2)
    pos = torch.arange(T)
    slots = (bt[0, pos // bs].long() * bs + pos % bs)
    C = lay.compressed_bytes_per_token()
    page = torch.zeros(nblk * bs, C, dtype=torch.uint8, device=dev)
    dec_map = torch.full((nblk,), -1, dtype=torch.int32)
    dec_map[bt[0, 0]] = 0
    args = dict(block_table=bt.to(dev), dec_slot_of_block=dec_map.to(dev),
                dec_pool=dec_pool_of([dec], dev), pinv_pool=encode.pinv(dec).t().unsqueeze(0).contiguous().to(dev),
                page=page)
    Kt = K.permute(1, 0, 2).contiguous()
    Vt = V.permute(1, 0, 2).contiguous()
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.write_paged(lay, Kt[:fit_on].to(dev), Vt[:fit_on].to(dev), slots[:fit_on].to(dev),
                        torch.tensor([0, fit_on], dtype=torch.int32, device=dev),
                        coeff_q_in=fk["coeff_q"].to(dev),
                        coeff_scale_in=fk["coeff_scale"].float().to(dev), error_word=err, **args)
    for t in range(fit_on, T, 50):                      # decode-style appends, several per call
        e = min(T, t + 50)
        kernels.write_paged(lay, Kt[t:e].to(dev), Vt[t:e].to(dev), slots[t:e].to(dev),
                            torch.tensor([0, e - t], dtype=torch.int32, device=dev),
                            error_word=err, **args)
    q = synth.queries(1, seed=32)
    cache = llama3_cache(512)
    out = torch.zeros(1, HQ, 128, dtype=torch.float16, device=dev)
    kernels.decode_paged(lay, q.to(dev), page, bs, bt.to(dev),
                         torch.tensor([T], dtype=torch.int32, device=dev),
                         torch.tensor([0, 1], dtype=torch.int32, device=dev), T,
                         dec_map.to(dev), args["dec_pool"], cache.to(dev), 128 ** -0.5,
                         out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_decode(lay, page.cpu(), bt, torch.tensor([T]), torch.arange(2),
                               q.float(), [dec], cache, bs, 128 ** -0.5, dtype=torch.float64)
    _check(out.float().cpu(), want, "write->read")
    # and the store approximates attention over the raw keys. A loose fidelity sanity check,
    # not parity: the decoder is fitted on 128 tokens of rank-768 synthetic keys and frozen.
    from oracle import rope as orope
    cos, sin = orope.cos_sin_from_cache(cache, pos, 128)
    Kpost = orope.rope_apply(K.permute(1, 0, 2).double(), cos.double().unsqueeze(1),
                             sin.double().unsqueeze(1))
    p_all = torch.arange(HQ) // 3
    s = torch.einsum("npd,pd->np", Kpost[:, p_all], q[0].double()) * 128 ** -0.5
    dense_v = attend.dense_v_from_slots(lay, page.cpu()[slots, lay.v_offset:C], torch.float64)
    ref = torch.einsum("np,npd->pd", torch.softmax(s, 0), dense_v.permute(1, 0, 2)[:, p_all])
    cosim = torch.nn.functional.cosine_similarity(out.float().cpu().double().reshape(1, -1),
                                                   ref.reshape(1, -1)).item()
    assert cosim > 0.95, cosim


@pytest.mark.parametrize("hq,r1,bs", [(8, 64, 16), (16, 110, 32), (32, 160, 24), (64, 110, 16)])
def test_head_groups_ranks_and_block_sizes(hq, r1, bs):
    """Every built instantiation family: 1/2/4/8 query heads per KV head, rank budgets that take
    2, 4 and 5 MFMA k-steps, and block sizes including one that is not a power of two."""
    lens = [37, 300, 1025]
    stores = [fitted_store("safe", n, seed=40 + i, r1=r1) for i, n in enumerate(lens)]
    q = synth.queries(len(lens), HQ=hq, seed=7)
    cache = llama3_cache(2048)
    got, pg = _run_k1(stores, q, cache, block_size=bs, seed=9)
    _check(got, _oracle(stores, q, cache, pg, block_size=bs), f"hq={hq} r1={r1} bs={bs}")


@pytest.mark.parametrize("kvh,hq", [(4, 12), (2, 8)])
def test_fewer_kv_heads(kvh, hq):
    """4 and 2 KV heads (a K slot of 4 or 2 residual rows, a plan with fewer heads per request)
    with 3 and 4 query heads each, against the oracle."""
    lens = [300, 1100, 70]
    stores = [fitted_store("safe", n, seed=60 + i, H_=kvh) for i, n in enumerate(lens)]
    q = synth.queries(len(lens), HQ=hq, seed=8)
    cache = llama3_cache(2048)
    got, pg = _run_k1(stores, q, cache, seed=3)
    _check(got, _oracle(stores, q, cache, pg), f"H={kvh} HQ={hq}")


def test_empty_context_and_missing_decoder():
    """A request with no cached tokens reads as zeros (the reference's einsum over zero rows); a
    request whose first block has no registered decoder sets error bit 1 and reads as NaN, and
    neither disturbs the other requests of the launch."""
    stores = [fitted_store("safe", n, seed=60 + i) for i, n in enumerate([200, 1, 500])]
    q = synth.queries(3, seed=8)
    cache = llama3_cache(1024)
    pg = paged(stores, 16, 3)
    dev = "cuda"
    lay = stores[0]["lay"]
    seq_lens = pg["seq_lens"].clone()
    seq_lens[1] = 0                                      # request 1: empty
    dec_pool = dec_pool_of([s["decoder"] for s in stores], dev)
    dec_map = torch.full((pg["num_blocks"],), -1, dtype=torch.int32)
    dec_map[pg["block_table"][0, 0]] = 0                 # request 2 left unregistered
    dec_map[pg["block_table"][1, 0]] = 1
    out = torch.full((3, HQ, 128), 7.0, dtype=torch.float16, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.decode_paged(lay, q.to(dev), pg["page"].to(dev), 16, pg["block_table"].to(dev),
                         seq_lens.to(dev), torch.arange(4, dtype=torch.int32).to(dev),
                         int(seq_lens.max()), dec_map.to(dev), dec_pool, cache.to(dev),
                         128 ** -0.5, out=out, error_word=err)
    torch.cuda.synchronize()
    got = out.float().cpu()
    assert int(err.item()) == 1
    assert torch.all(got[1] == 0)
    assert torch.isnan(got[2]).all()
    want = _oracle(stores[:1], q[:1], cache, dict(pg, block_table=pg["block_table"][:1],
                                                  seq_lens=pg["seq_lens"][:1]))
    _check(got[:1], want, "request 0 beside an empty and an undecodable request")


def test_one_long_request_among_short_ones():
    """The work plan splits by the batch's total length, not by its longest request: one long
    context beside sub-tile ones is cut into many chunks, the short ones into one each."""
    lens = [6000, 1, 2, 3, 64, 65, 127, 128]
    stores = [fitted_store("safe", n, seed=70 + i) for i, n in enumerate(lens)]
    q = synth.queries(len(lens), seed=11)
    cache = llama3_cache(6144)
    got, pg = _run_k1(stores, q, cache, seed=12)
    _check(got, _oracle(stores, q, cache, pg), "one long among short")


def test_more_requests_than_one_launch_plans():
    """300 requests: past the 256 a launch's work plan holds, so the call runs as two launches
    over consecutive request ranges sharing one workspace."""
    base = [fitted_store("safe", n, seed=80 + i) for i, n in enumerate([1, 17, 64, 65, 130, 257])]
    stores = [base[i % len(base)] for i in range(300)]
    q = synth.queries(len(stores), seed=13)
    cache = llama3_cache(512)
    got, pg = _run_k1(stores, q, cache, seed=14)
    _check(got, _oracle(stores, q, cache, pg), "300 requests")


def test_workspace_shared_across_batch_shapes():
    """One workspace serves decode calls of different batch shapes in turn (a serving loop's
    batch changes every step); each call's output equals the same call with a fresh workspace,
    bit for bit (same work plan, same combine order)."""
    from vllm_ttkv import kernels as K
    batches = [[3000, 40, 900], [5000], [200] * 6 + [64], [3000, 40, 900], [70, 2000]]
    stores = {n: fitted_store("safe", n, seed=90 + i)
              for i, n in enumerate(sorted({n for b in batches for n in b}))}
    cache = llama3_cache(5120)
    lay = stores[5000]["lay"]
    need = max(K.decode_workspace(lay, HQ, len(b), max(b), "cuda").numel() for b in batches)
    shared = torch.zeros(need, dtype=torch.uint8, device="cuda")
    for i, b in enumerate(batches):
        st = [stores[n] for n in b]
        q = synth.queries(len(b), seed=20 + i)
        got, _ = _run_k1(st, q, cache, seed=30 + i, workspace=shared)
        want, _ = _run_k1(st, q, cache, seed=30 + i)
        assert torch.equal(got, want), f"batch {b} with a shared workspace"
    assert int(shared[:65536].abs().sum()) == 0, "counters left non-zero"


def test_length_past_max_seq_len_is_flagged_and_clamped():
    """A seq_lens entry beyond the max_seq_len the call was sized with sets error bit 8 and is
    read over its first max_seq_len tokens; the other requests are unaffected."""
    stores = [fitted_store("safe", n, seed=100 + i) for i, n in enumerate([300, 500])]
    q = synth.queries(2, seed=15)
    cache = llama3_cache(1024)
    pg = paged(stores, 16, 4)
    dev = "cuda"
    lay = stores[0]["lay"]
    dec_pool = dec_pool_of([s["decoder"] for s in stores], dev)
    dec_map = torch.full((pg["num_blocks"],), -1, dtype=torch.int32)
    for r in range(2):
        dec_map[pg["block_table"][r, 0]] = r
    out = torch.zeros(2, HQ, 128, dtype=torch.float16, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.decode_paged(lay, q.to(dev), pg["page"].to(dev), 16, pg["block_table"].to(dev),
                         pg["seq_lens"].to(dev), torch.arange(3, dtype=torch.int32).to(dev), 400,
                         dec_map.to(dev), dec_pool, cache.to(dev), 128 ** -0.5, out=out,
                         error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 8
    want = _oracle(stores, q, cache, dict(pg, seq_lens=torch.tensor([300, 400])))
    _check(out.float().cpu(), want, "clamped at max_seq_len")
