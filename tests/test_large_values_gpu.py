"""V rows of large magnitude through every P.V readout (K1, K2's two-launch and fused paths, the
container v_out), against the float64 oracle.

The readouts multiply each softmax weight by its V row's fp16 ruler and round the product to fp16
for the MFMA (the V codes are exact integers). Weights reach 2^8 under the lazy softmax rescale,
so an unscaled product overflows fp16 once a ruler passes ~256 (|v| ~ 770 at 3 bits, ~1,800 at 4
bits). The kernels carry the product at a power-of-two scale that grows with the largest ruler
seen. Here the rulers run to ~10^4: outputs must be finite and, relative to the values' scale,
within the north star's 2e-3 max-abs / 1e-3 mean-abs (fp32 outputs, so output rounding does not
enter). A request of ordinary values rides in the same launch and keeps the absolute bound."""
import pytest
import torch

from helpers import HQ, dec_pool_of, fitted_store, llama3_cache, paged
from oracle import attend, codec, container as ocont
from vllm_ttkv import container, kernels, synth

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-3, 1e-3
SCALE = 128 ** -0.5


def _scales(T, seed):
    """Per-token value factors 10^U(0, 4): rulers from ~1 to ~10^4 in one request."""
    g = torch.Generator().manual_seed(seed)
    return 10.0 ** (4.0 * torch.rand(T, generator=g))


def _check(got, want, vs, what):
    got = got.double().cpu()
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    e = (got - want).abs() / vs
    print(f"{what}: max-abs {e.max():.3e} mean-abs {e.mean():.3e} (relative to {vs:.3g})")
    assert e.max() <= MAX_ABS and e.mean() <= MEAN_ABS, f"{what}: {e.max():.3e} / {e.mean():.3e}"


def _dev(stores, seed):
    pg = paged(stores, 16, seed)
    dec_pool = dec_pool_of([s["decoder"] for s in stores])
    dec_map = torch.full((pg["num_blocks"],), -1, dtype=torch.int32)
    for r in range(len(stores)):
        dec_map[pg["block_table"][r, 0]] = r
    return pg, dec_pool, dec_map.cuda()


@pytest.mark.parametrize("cfg", ["safe", "campaign4x"])
def test_k1_large_value_rows(cfg):
    lens = [700, 1300, 2100]
    vsc = [1.0, 2048.0, None]   # ordinary, uniform x2^11, per-token 10^U(0,4)
    stores = [fitted_store(cfg, n, seed=90 + i,
                           v_scale=_scales(n, 5 + i) if s is None else (s if s != 1.0 else None))
              for i, (n, s) in enumerate(zip(lens, vsc))]
    q = synth.queries(len(lens), seed=9)
    cache = llama3_cache(4096)
    pg, dec_pool, dec_map = _dev(stores, 3)
    out = torch.zeros(len(lens), HQ, 128, dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.decode_paged(stores[0]["lay"], q.cuda(), pg["page"].cuda(), 16,
                         pg["block_table"].cuda(), pg["seq_lens"].cuda(),
                         torch.arange(len(lens) + 1, dtype=torch.int32, device="cuda"), max(lens),
                         dec_map, dec_pool, cache.cuda(), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_decode(stores[0]["lay"], pg["page"], pg["block_table"], pg["seq_lens"],
                               torch.arange(len(lens) + 1), q.float(),
                               [s["decoder"] for s in stores], cache, 16, SCALE,
                               dtype=torch.float64)
    for r in range(len(lens)):
        vs = 1.0 if vsc[r] == 1.0 else float(stores[r]["V"].abs().max() / 4.0)
        _check(out[r], want[r], vs, f"K1 {cfg} request {r}")


@pytest.mark.parametrize("cfg", ["safe", "campaign4x"])
def test_k2_two_launch_large_value_rows(cfg):
    """Chunks of two or more queries at G = 3: the expand + attend path."""
    shapes = [(600, 40), (1500, 130)]
    stores = [fitted_store(cfg, shapes[0][0], seed=120),
              fitted_store(cfg, shapes[1][0], seed=121, v_scale=_scales(shapes[1][0], 12))]
    cache = llama3_cache(2048)
    pg, dec_pool, dec_map = _dev(stores, 4)
    q = torch.cat([synth.queries(Q, seed=400 + i) for i, (_, Q) in enumerate(shapes)])
    qsl = torch.tensor([0, shapes[0][1], shapes[0][1] + shapes[1][1]], dtype=torch.int32)
    out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
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
        vs = 1.0 if r == 0 else float(stores[r]["V"].abs().max() / 4.0)
        _check(out[s:e], want[r], vs, f"K2 {cfg} request {r}")


@pytest.mark.parametrize("hq,Q", [(32, 50), (24, 1)])
def test_k2_fused_large_value_rows(hq, Q):
    """The fused continuation kernel: G = 4 (any chunk) and single queries."""
    n = 1200
    st = fitted_store("safe", n, seed=130 + Q, v_scale=2048.0)
    cache = llama3_cache(2048)
    pg, dec_pool, dec_map = _dev([st], 6)
    q = synth.queries(Q, HQ=hq, seed=500 + Q)
    qsl = torch.tensor([0, Q], dtype=torch.int32)
    out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.prefill_paged(st["lay"], q.cuda(), pg["page"].cuda(), 16, pg["block_table"].cuda(),
                          pg["seq_lens"].cuda(), qsl.cuda(), Q, n, dec_map, dec_pool,
                          cache.cuda(), SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    want = attend.paged_continuation(st["lay"], pg["page"], pg["block_table"], pg["seq_lens"],
                                     qsl, q.double(), [st["decoder"]], cache, 16, SCALE,
                                     dtype=torch.float64)
    _check(out, want[0], 2048.0, f"K2 fused HQ={hq} Q={Q}")


@pytest.mark.parametrize("vbits_cfg", ["safe", "campaign4x"])
def test_container_v_out_large_weights(vbits_cfg):
    """Container v_out with products p * ruler up to ~10^4 (the former fixed 2^8 scaling
    overflowed above 256), over several tiles per workgroup."""
    cfg = codec.CONFIGS[vbits_cfg]
    H, D, n, hq = 8, 128, 3000, 24
    g = torch.Generator().manual_seed(77)
    V = torch.randn(H, n, D, generator=g) * _scales(n, 13).reshape(1, n, 1)
    vr = codec.build_v_layer(V, cfg["k_lanes"], cfg["vbits"])
    logits = torch.randn(hq, n, generator=g) * 3.0
    p = torch.softmax(logits, -1) * 40.0          # weights need not sum to one
    rows = container.PackedRows(*(x.cuda() for x in vr), cfg["vbits"])
    o = container.v_out(p.cuda(), rows, n, hq, hq // H, D)
    torch.cuda.synchronize()
    want = ocont.v_out(p, vr, n, H, D, cfg["k_lanes"], cfg["vbits"])
    assert torch.isfinite(o).all()
    rel = float((o.double().cpu() - want).abs().max() / want.abs().max())
    print(f"container v_out {vbits_cfg}: rel {rel:.2e}")
    assert rel < 1e-5
