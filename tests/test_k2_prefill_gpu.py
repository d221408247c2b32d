"""K2 (multi-query continuation read) on the GPU against the CPU oracle.

Scores mode vs `raw_scores_multi` (reference.py:112-146) and attention mode vs the reference's
continuation (impl.py:725-778: scores, softmax over the store, V readout), both with the causal
rule key t visible to query j iff t <= p0 + j, p0 = seq_len - q_len.

Tolerance (north star): scores and outputs within 2e-3 max-abs / 1e-3 mean-abs against the
float64 oracle; the masked pattern is compared exactly."""
import pytest
import torch

from helpers import HQ, dec_pool_of, fitted_store, llama3_cache, paged
from oracle import attend
from oracle.rope import cos_sin_from_cache
from vllm_ttkv import kernels, synth

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-3, 1e-3
SCALE = 128 ** -0.5


def _dev_inputs(stores, block_size=16, seed=0):
    pg = paged(stores, block_size, seed)
    B = len(stores)
    dec_pool = dec_pool_of([s["decoder"] for s in stores])
    dec_map = torch.full((pg["num_blocks"],), -1, dtype=torch.int32)
    for r in range(B):
        dec_map[pg["block_table"][r, 0]] = r
    return pg, dec_pool, dec_map.cuda()


def _check(got, want, what, exact_inf=True):
    got = got.double().cpu()
    if exact_inf:
        assert torch.equal(torch.isneginf(got), torch.isneginf(want)), f"{what}: mask pattern"
        fin = torch.isfinite(want)
        assert torch.isfinite(got[fin]).all(), what
        e = (got[fin] - want[fin]).abs()
    else:
        assert torch.isfinite(got).all(), what
        e = (got - want).abs()
    print(f"{what}: max-abs {e.max():.3e} mean-abs {e.mean():.3e}")
    assert e.max() <= MAX_ABS and e.mean() <= MEAN_ABS, f"{what}: {e.max():.3e} / {e.mean():.3e}"


@pytest.mark.parametrize("cfg,n,Q", [("safe", 1000, 100), ("safe", 2100, 256), ("safe", 77, 5),
                                     ("campaign4x", 900, 130), ("tight", 700, 64)])
def test_scores_mode_vs_raw_scores_multi(cfg, n, Q):
    st = fitted_store(cfg, n, seed=n + Q)
    cache = llama3_cache(4096)
    pg, dec_pool, dec_map = _dev_inputs([st])
    q = synth.queries(Q, seed=Q).reshape(Q, HQ, 128)
    qsl = torch.tensor([0, Q], dtype=torch.int32)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = kernels.multi_scores_paged(st["lay"], q.cuda(), pg["page"].cuda(), 16,
                                     pg["block_table"].cuda(), pg["seq_lens"].cuda(), qsl.cuda(),
                                     Q, n, dec_map, dec_pool, cache.cuda(), SCALE,
                                     error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    cos, sin = cos_sin_from_cache(cache, torch.arange(n), 128)
    want = attend.raw_scores_multi(st["lay"], st["k_slots"], st["decoder"],
                                   q.permute(1, 0, 2).double(), cos, sin, SCALE, p0=n - Q,
                                   dtype=torch.float64)
    _check(got, want, f"scores {cfg} n={n} Q={Q}")


@pytest.mark.parametrize("cfg,n,Q", [("safe", 2100, 257), ("campaign4x", 1030, 200)])
def test_scores_from_expanded_keys_equal_the_fused_kernel(cfg, n, Q):
    """A chunk of two or more queries with a workspace is scored from every stored key expanded
    once (expand launch + scores kernel); without one, by the fused kernel. Both reconstruct and
    rotate with the same fp32 arithmetic (up to the compiler's fma contraction, an ulp) and take
    the same fp16 MFMA operands, so the -inf pattern is identical and the finite scores agree to
    fp32 rounding. Rows past the tensor's n keys and Q queries stay untouched."""
    st = fitted_store(cfg, n, seed=3 * n + Q)
    cache = llama3_cache(4096)
    pg, dec_pool, dec_map = _dev_inputs([st], seed=9)
    q = synth.queries(Q, seed=Q + 1).reshape(Q, HQ, 128)
    qsl = torch.tensor([0, Q], dtype=torch.int32).cuda()
    args = (st["lay"], q.cuda(), pg["page"].cuda(), 16, pg["block_table"].cuda(),
            pg["seq_lens"].cuda(), qsl, Q, n, dec_map, dec_pool, cache.cuda(), SCALE)
    outs = []
    for ws in (None, False):
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        sc = torch.full((HQ, Q + 3, n + 5), 7.0, dtype=torch.float32, device="cuda")
        kernels.multi_scores_paged(*args, scores=sc, error_word=err, workspace=ws)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        outs.append(sc.cpu())
    expanded, fused = outs
    assert torch.equal(torch.isneginf(expanded), torch.isneginf(fused))
    fin = torch.isfinite(fused)
    assert torch.isfinite(expanded[fin]).all()
    d = (expanded[fin].double() - fused[fin].double()).abs().max()
    print(f"expanded vs fused scores {cfg} n={n} Q={Q}: max-abs {d:.3e}")
    assert d <= 1e-5 * float(fused[fin].abs().max())
    assert (expanded[:, Q:, :] == 7.0).all() and (expanded[:, :, n:] == 7.0).all()
    assert torch.isneginf(expanded[:, :Q, :n]).any()


def test_attend_mode_ragged_batch_with_splits():
    """Three continuation requests of different lengths in one launch (several key splits per
    query block, so the in-launch combine runs), fp16 queries and output."""
    shapes = [(300, 40), (1000, 128), (2100, 257)]
    stores = [fitted_store("safe", n, seed=7 + i) for i, (n, _) in enumerate(shapes)]
    cache = llama3_cache(4096)
    pg, dec_pool, dec_map = _dev_inputs(stores, seed=3)
    qs = [synth.queries(Q, seed=100 + i).reshape(Q, HQ, 128) for i, (_, Q) in enumerate(shapes)]
    q = torch.cat(qs)
    qsl = torch.tensor([0] + list(torch.tensor([Q for _, Q in shapes]).cumsum(0)),
                       dtype=torch.int32)
    out = torch.zeros_like(q, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.prefill_paged(st_lay := stores[0]["lay"], q.cuda(), pg["page"].cuda(), 16,
                          pg["block_table"].cuda(), pg["seq_lens"].cuda(), qsl.cuda(),
                          max(Q for _, Q in shapes), max(n for n, _ in shapes), dec_map, dec_pool,
                          cache.cuda(), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(st_lay, pg["page"], pg["block_table"], pg["seq_lens"], qsl,
                                     q.double(), [s["decoder"] for s in stores], cache, 16, SCALE,
                                     dtype=torch.float64)
    for r in range(len(shapes)):
        s, e = int(qsl[r]), int(qsl[r + 1])
        _check(out[s:e].float(), want[r], f"attend req {r} {shapes[r]}", exact_inf=False)


@pytest.mark.parametrize("r1", [64, 160])
def test_attend_mode_rank_budgets(r1):
    """Rank budgets of 2 and 5 reconstruction k-steps: r1 = 64 through the two-launch path
    (expand + attend) and r1 = 160 through the fused kernel (r1 > 128), each with a chunk of
    several queries and a single query, against the oracle. The output is fp32 here: an fp16
    output row of magnitude 4 or more is rounded by up to 2^-9 by its format alone, which would
    leave no room for the kernel's own error under the 2e-3 bound."""
    shapes = [(700, 70), (1200, 1)]
    stores = [fitted_store("safe", n, seed=60 + i, r1=r1) for i, (n, _) in enumerate(shapes)]
    cache = llama3_cache(2048)
    pg, dec_pool, dec_map = _dev_inputs(stores, seed=4)
    q = torch.cat([synth.queries(Q, seed=200 + i).reshape(Q, HQ, 128)
                   for i, (_, Q) in enumerate(shapes)])
    qsl = torch.tensor([0] + list(torch.tensor([Q for _, Q in shapes]).cumsum(0)),
                       dtype=torch.int32)
    out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    print(f"[k2] r1={r1}", flush=True)
    lay = stores[0]["lay"]
    kernels.prefill_paged(lay, q.cuda(), pg["page"].cuda(), 16, pg["block_table"].cuda(),
                          pg["seq_lens"].cuda(), qsl.cuda(), max(Q for _, Q in shapes),
                          max(n for n, _ in shapes), dec_map, dec_pool, cache.cuda(), SCALE,
                          out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(lay, pg["page"], pg["block_table"], pg["seq_lens"], qsl,
                                     q.double(), [s["decoder"] for s in stores], cache, 16, SCALE,
                                     dtype=torch.float64)
    for r in range(len(shapes)):
        s, e = int(qsl[r]), int(qsl[r + 1])
        _check(out[s:e].float(), want[r], f"r1={r1} req {r} {shapes[r]}", exact_inf=False)


def test_attend_mode_queries_in_rows_that_are_not_16_byte_aligned():
    """Query rows at a stride of HQ*d + 2 elements (a view into a wider buffer): the kernel loads
    them element by element instead of in wide loads, with the same result."""
    shapes = [(500, 70), (900, 130)]
    stores = [fitted_store("safe", n, seed=17 + i) for i, (n, _) in enumerate(shapes)]
    cache = llama3_cache(2048)
    pg, dec_pool, dec_map = _dev_inputs(stores, seed=5)
    q = torch.cat([synth.queries(Q, seed=200 + i).reshape(Q, HQ, 128)
                   for i, (_, Q) in enumerate(shapes)])
    wide = torch.zeros(q.shape[0], HQ * 128 + 2, dtype=q.dtype)
    wide[:, :HQ * 128] = q.reshape(q.shape[0], -1)
    qv = wide.cuda()[:, :HQ * 128].view(q.shape[0], HQ, 128)
    assert qv.stride(0) == HQ * 128 + 2
    qsl = torch.tensor([0] + list(torch.tensor([Q for _, Q in shapes]).cumsum(0)),
                       dtype=torch.int32)
    out = torch.zeros_like(q, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    lay = stores[0]["lay"]
    kernels.prefill_paged(lay, qv, pg["page"].cuda(), 16, pg["block_table"].cuda(),
                          pg["seq_lens"].cuda(), qsl.cuda(), max(Q for _, Q in shapes),
                          max(n for n, _ in shapes), dec_map, dec_pool, cache.cuda(), SCALE,
                          out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(lay, pg["page"], pg["block_table"], pg["seq_lens"], qsl,
                                     q.double(), [s["decoder"] for s in stores], cache, 16, SCALE,
                                     dtype=torch.float64)
    for r in range(len(shapes)):
        s, e = int(qsl[r]), int(qsl[r + 1])
        _check(out[s:e].float(), want[r], f"strided queries req {r}", exact_inf=False)


def test_attend_mode_req_index_subset_bf16():
    """`req_index` selects batch rows (decodes at the front are skipped); bf16 in and out."""
    shapes = [(50, 1), (600, 70), (1200, 200)]
    stores = [fitted_store("safe", n, seed=20 + i) for i, (n, _) in enumerate(shapes)]
    cache = llama3_cache(2048)
    pg, dec_pool, dec_map = _dev_inputs(stores, seed=5)
    q = torch.cat([synth.queries(Q, seed=200 + i).reshape(Q, HQ, 128)
                   for i, (_, Q) in enumerate(shapes)]).to(torch.bfloat16)
    qsl = torch.tensor([0, 1, 71, 271], dtype=torch.int32)
    out = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device="cuda")
    kernels.prefill_paged(stores[0]["lay"], q.cuda(), pg["page"].cuda(), 16,
                          pg["block_table"].cuda(), pg["seq_lens"].cuda(), qsl.cuda(), 200, 1200,
                          dec_map, dec_pool, cache.cuda(), SCALE,
                          req_index=torch.tensor([1, 2], dtype=torch.int32, device="cuda"),
                          out=out)
    torch.cuda.synchronize()
    assert torch.all(out[0].float() == 7.0), "row of an unselected request was written"
    want = attend.paged_continuation(stores[0]["lay"], pg["page"], pg["block_table"],
                                     pg["seq_lens"], qsl, q.double(),
                                     [s["decoder"] for s in stores], cache, 16, SCALE,
                                     rows=[1, 2], dtype=torch.float64)
    for r in (1, 2):
        s, e = int(qsl[r]), int(qsl[r + 1])
        e_ = (out[s:e].double().cpu() - want[r]).abs()
        print(f"bf16 req {r}: max-abs {e_.max():.3e} mean-abs {e_.mean():.3e}")
        # bf16 output rounding alone is up to 2^-9 relative; the tolerance is on the math
        assert e_.max() <= 2e-2 and e_.mean() <= 2e-3


def test_single_query_continuation_equals_decode_read():
    """Q = 1: the multi-query read of one query equals K1's decode read of it."""
    st = fitted_store("safe", 777, seed=31)
    cache = llama3_cache(1024)
    pg, dec_pool, dec_map = _dev_inputs([st])
    q = synth.queries(1, seed=31).reshape(1, HQ, 128).cuda()
    qsl = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    args = (pg["page"].cuda(), 16, pg["block_table"].cuda(), pg["seq_lens"].cuda(), qsl)
    k2 = kernels.prefill_paged(st["lay"], q, *args, 1, 777, dec_map, dec_pool, cache.cuda(),
                               SCALE, out=torch.zeros(1, HQ, 128, device="cuda"))
    k1 = kernels.decode_paged(st["lay"], q, *args, 777, dec_map, dec_pool, cache.cuda(), SCALE,
                              out=torch.zeros(1, HQ, 128, device="cuda"))
    torch.cuda.synchronize()
    e = (k1 - k2).abs().max().item()
    print(f"Q=1 K2 vs K1: {e:.3e}")
    assert e <= 1e-3


def test_missing_decoder_sets_error_and_nan():
    st = fitted_store("safe", 200, seed=41)
    cache = llama3_cache(1024)
    pg, dec_pool, _ = _dev_inputs([st])
    dec_map = torch.full((pg["num_blocks"],), -1, dtype=torch.int32, device="cuda")
    q = synth.queries(10, seed=1).reshape(10, HQ, 128).cuda()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = kernels.prefill_paged(st["lay"], q, pg["page"].cuda(), 16, pg["block_table"].cuda(),
                                pg["seq_lens"].cuda(),
                                torch.tensor([0, 10], dtype=torch.int32, device="cuda"), 10, 200,
                                dec_map, dec_pool, cache.cuda(), SCALE, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    assert torch.isnan(out).all()


@pytest.mark.parametrize("cfg", ["campaign4x", "tight"])
def test_attend_mode_other_allocations(cfg):
    """Attention mode on the 4-bit (campaign4x) and the narrow 3-bit (tight) allocations, two
    requests with key splits, fp16 in and out."""
    shapes = [(700, 64), (1500, 130)]
    stores = [fitted_store(cfg, n, seed=50 + i) for i, (n, _) in enumerate(shapes)]
    cache = llama3_cache(2048)
    pg, dec_pool, dec_map = _dev_inputs(stores, seed=6)
    q = torch.cat([synth.queries(Q, seed=300 + i).reshape(Q, HQ, 128)
                   for i, (_, Q) in enumerate(shapes)])
    qsl = torch.tensor([0, 64, 194], dtype=torch.int32)
    out = torch.zeros_like(q, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.prefill_paged(stores[0]["lay"], q.cuda(), pg["page"].cuda(), 16,
                          pg["block_table"].cuda(), pg["seq_lens"].cuda(), qsl.cuda(), 130, 1500,
                          dec_map, dec_pool, cache.cuda(), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(stores[0]["lay"], pg["page"], pg["block_table"],
                                     pg["seq_lens"], qsl, q.double(),
                                     [s["decoder"] for s in stores], cache, 16, SCALE,
                                     dtype=torch.float64)
    for r in range(2):
        s, e = int(qsl[r]), int(qsl[r + 1])
        _check(out[s:e].float(), want[r], f"attend {cfg} req {r}", exact_inf=False)


def test_workspace_shared_across_batch_shapes():
    """One workspace serves continuation calls of different shapes in turn; each call's output
    equals the same call with a fresh workspace, bit for bit."""
    calls = [[(1000, 128), (300, 40)], [(2100, 257)], [(700, 64), (1000, 128), (300, 40)],
             [(1000, 128), (300, 40)]]
    stores = {n: fitted_store("safe", n, seed=200 + n) for n in {n for c in calls for n, _ in c}}
    cache = llama3_cache(4096)
    lay = stores[1000]["lay"]
    need = max(kernels.prefill_workspace(lay, HQ, len(c), max(Q for _, Q in c),
                                         max(n for n, _ in c), "cuda").numel() for c in calls)
    shared = torch.zeros(need, dtype=torch.uint8, device="cuda")

    def run(shapes, ws, i):
        st = [stores[n] for n, _ in shapes]
        pg, dec_pool, dec_map = _dev_inputs(st, seed=40 + i)
        q = torch.cat([synth.queries(Q, seed=300 + i + j).reshape(Q, HQ, 128)
                       for j, (_, Q) in enumerate(shapes)])
        qsl = torch.tensor([0] + list(torch.tensor([Q for _, Q in shapes]).cumsum(0)),
                           dtype=torch.int32)
        out = torch.zeros_like(q, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        kernels.prefill_paged(lay, q.cuda(), pg["page"].cuda(), 16, pg["block_table"].cuda(),
                              pg["seq_lens"].cuda(), qsl.cuda(), max(Q for _, Q in shapes),
                              max(n for n, _ in shapes), dec_map, dec_pool, cache.cuda(), SCALE,
                              out=out, error_word=err, workspace=ws)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        return out.cpu()

    for i, shapes in enumerate(calls):
        assert torch.equal(run(shapes, shared, i), run(shapes, None, i)), f"call {shapes}"
    assert int(shared[:65536].abs().sum()) == 0, "counters left non-zero"


@pytest.mark.parametrize("hq", [8, 16])
def test_attend_and_scores_at_one_and_two_query_heads_per_kv_head(hq):
    """G = 1 and G = 2 (HQ = 8, 16 over 8 KV heads) build their own attend and scores kernels
    (and the attend's split-K combine over G * 128 rows): a two-request launch with key splits
    against the oracle, and the scores mode from expanded keys against raw_scores_multi."""
    shapes = [(2100, 257), (700, 64)]
    stores = [fitted_store("safe", n, seed=60 + hq + i) for i, (n, _) in enumerate(shapes)]
    cache = llama3_cache(4096)
    pg, dec_pool, dec_map = _dev_inputs(stores, seed=8)
    q = torch.cat([synth.queries(Q, HQ=hq, seed=600 + hq + i) for i, (_, Q) in enumerate(shapes)])
    qsl = torch.tensor([0] + list(torch.tensor([Q for _, Q in shapes]).cumsum(0)),
                       dtype=torch.int32)
    lay = stores[0]["lay"]
    out = torch.zeros_like(q, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.prefill_paged(lay, q.cuda(), pg["page"].cuda(), 16, pg["block_table"].cuda(),
                          pg["seq_lens"].cuda(), qsl.cuda(), 257, 2100, dec_map, dec_pool,
                          cache.cuda(), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(lay, pg["page"], pg["block_table"], pg["seq_lens"], qsl,
                                     q.double(), [s["decoder"] for s in stores], cache, 16, SCALE,
                                     dtype=torch.float64)
    for r in range(len(shapes)):
        s, e = int(qsl[r]), int(qsl[r + 1])
        _check(out[s:e].float(), want[r], f"attend HQ={hq} req {r}", exact_inf=False)

    n, Q = shapes[0]
    st = stores[0]
    pg1, dec_pool1, dec_map1 = _dev_inputs([st], seed=9)
    q1 = q[:Q]
    got = kernels.multi_scores_paged(lay, q1.cuda(), pg1["page"].cuda(), 16,
                                     pg1["block_table"].cuda(), pg1["seq_lens"].cuda(),
                                     torch.tensor([0, Q], dtype=torch.int32, device="cuda"), Q, n,
                                     dec_map1, dec_pool1, cache.cuda(), SCALE, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    cos, sin = cos_sin_from_cache(cache, torch.arange(n), 128)
    want_s = attend.raw_scores_multi(lay, st["k_slots"], st["decoder"], q1.permute(1, 0, 2).double(),
                                     cos, sin, SCALE, p0=n - Q, dtype=torch.float64)
    _check(got, want_s, f"scores HQ={hq}")


@pytest.mark.parametrize("kvh,hq", [(4, 12), (2, 8)])
def test_attend_mode_fewer_kv_heads(kvh, hq):
    """4 and 2 KV heads (3 and 4 query heads each): a 70-query chunk through the expand + attend
    pair and single queries through the fused kernel, against the oracle (fp32 output)."""
    shapes = [(700, 70), (1200, 1), (300, 5)]
    stores = [fitted_store("safe", n, seed=80 + i, H_=kvh) for i, (n, _) in enumerate(shapes)]
    cache = llama3_cache(2048)
    pg, dec_pool, dec_map = _dev_inputs(stores, seed=6)
    q = torch.cat([synth.queries(Q, HQ=hq, seed=300 + i) for i, (_, Q) in enumerate(shapes)])
    qsl = torch.tensor([0] + list(torch.tensor([Q for _, Q in shapes]).cumsum(0)),
                       dtype=torch.int32)
    out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    print(f"[k2] H={kvh} HQ={hq}", flush=True)
    lay = stores[0]["lay"]
    kernels.prefill_paged(lay, q.cuda(), pg["page"].cuda(), 16, pg["block_table"].cuda(),
                          pg["seq_lens"].cuda(), qsl.cuda(), max(Q for _, Q in shapes),
                          max(n for n, _ in shapes), dec_map, dec_pool, cache.cuda(), SCALE,
                          out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(lay, pg["page"], pg["block_table"], pg["seq_lens"], qsl,
                                     q.double(), [s["decoder"] for s in stores], cache, 16, SCALE,
                                     dtype=torch.float64)
    for r in range(len(shapes)):
        s, e = int(qsl[r]), int(qsl[r + 1])
        _check(out[s:e].float(), want[r], f"H={kvh} req {r} {shapes[r]}", exact_inf=False)
