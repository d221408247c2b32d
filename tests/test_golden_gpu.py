"""K1 and K2 on the GPU against attention vectors written by the reference implementation itself
(tests/golden/ref_attend_safe.npz, from reference.py:94-176 on a fitted safe store, n = 96 rows,
HQ = 24, r1 = 32, llama-style RoPE at theta 500000 in the HF (j, j + d/2) pairing).

The reference's cos/sin tables [n, d] become vLLM's cos_sin_cache [n, d] (cosine half, sine half)
for the kernels. Tolerance (north star): 2e-3 max-abs, 1e-3 mean-abs; the causal mask pattern of
the scores is compared exactly."""
import pathlib

import numpy as np
import pytest
import torch

from helpers import dec_pool_of
from oracle import attend
from oracle.codec import CONFIGS
from vllm_ttkv import kernels, synth
from vllm_ttkv.layout import layout_for_config

pytestmark = pytest.mark.gpu
MAX_ABS, MEAN_ABS = 2e-3, 1e-3
FIX = pathlib.Path(__file__).parent / "golden" / "ref_attend_safe.npz"


def _load():
    z = np.load(FIX)
    f = {k: torch.from_numpy(np.ascontiguousarray(z[k])) for k in z.files if z[k].dtype.kind != "U"}
    lay = layout_for_config(CONFIGS[str(z["config"])], int(z["r1"]))
    n = f["k_slots"].shape[0]
    blob = torch.cat([f["k_slots"], f["v_slots"]], dim=1).contiguous()
    assert blob.shape[1] == lay.compressed_bytes_per_token()
    bs = 16
    bt, nblk = synth.shuffled_block_table([n], bs, seed=4, extra_blocks=2)
    page = torch.zeros(nblk * bs, blob.shape[1], dtype=torch.uint8)
    pos = torch.arange(n)
    page[(bt[0, pos // bs].long() * bs + pos % bs)] = blob
    cache = torch.cat([f["cos"][:, :64], f["sin"][:, :64]], dim=1).float().contiguous()
    dec_map = torch.full((nblk,), -1, dtype=torch.int32)
    dec_map[bt[0, 0]] = 0
    return z, f, lay, n, bs, bt, page, cache, dec_map


def _check(got, want, what):
    e = (got.double() - want.double()).abs()
    print(f"{what}: max-abs {e.max():.3e} mean-abs {e.mean():.3e}")
    assert e.max() <= MAX_ABS and e.mean() <= MEAN_ABS, f"{what}: {e.max():.3e} / {e.mean():.3e}"


def test_k1_matches_reference_attend_raw_store():
    z, f, lay, n, bs, bt, page, cache, dec_map = _load()
    q = f["q"].half().reshape(1, 24, 128)
    out = torch.zeros(1, 24, 128, dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.decode_paged(lay, q.cuda(), page.cuda(), bs, bt.cuda(),
                         torch.tensor([n], dtype=torch.int32).cuda(),
                         torch.tensor([0, 1], dtype=torch.int32).cuda(), n, dec_map.cuda(),
                         dec_pool_of([f["decoder_f"]]), cache.cuda(), 128 ** -0.5,
                         out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    _check(out[0].float().cpu(), f["attend_raw_store"], "K1 vs reference attend_raw_store")


def test_k2_scores_match_reference_raw_scores_multi_causal():
    z, f, lay, n, bs, bt, page, cache, dec_map = _load()
    qm = f["qm"]                                             # [HQ, Q, d]
    Q = qm.shape[1]
    p0 = int(z["p0"])
    assert p0 == n - Q
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = kernels.multi_scores_paged(lay, qm.permute(1, 0, 2).half().contiguous().cuda(),
                                     page.cuda(), bs, bt.cuda(),
                                     torch.tensor([n], dtype=torch.int32).cuda(),
                                     torch.tensor([0, Q], dtype=torch.int32).cuda(), Q, n,
                                     dec_map.cuda(), dec_pool_of([f["decoder_f"]]),
                                     cache.cuda(), 128 ** -0.5, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    got = got.cpu()
    want = f["raw_scores_multi_causal"]
    assert torch.equal(torch.isneginf(got), torch.isneginf(want))
    fin = torch.isfinite(want)
    _check(got[fin], want[fin], "K2 scores vs reference raw_scores_multi(p0)")


def test_k2_attention_matches_reference_scores_softmax_readout():
    """K2 attention mode against softmax over the reference's causal scores and the V rows the
    store decodes to (dense_v_from_slots, itself pinned by the byte fixtures)."""
    z, f, lay, n, bs, bt, page, cache, dec_map = _load()
    qm = f["qm"]
    Q = qm.shape[1]
    q = qm.permute(1, 0, 2).half().contiguous()
    out = torch.zeros(Q, 24, 128, dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.prefill_paged(lay, q.cuda(), page.cuda(), bs, bt.cuda(),
                          torch.tensor([n], dtype=torch.int32).cuda(),
                          torch.tensor([0, Q], dtype=torch.int32).cuda(), Q, n, dec_map.cuda(),
                          dec_pool_of([f["decoder_f"]]), cache.cuda(), 128 ** -0.5,
                          out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    from oracle.layout import layout_for_config as oracle_layout
    V = attend.dense_v_from_slots(oracle_layout(CONFIGS["safe"], int(z["r1"])), f["v_slots"],
                                  dtype=torch.float64)     # [H, n, d]
    p = torch.softmax(f["raw_scores_multi_causal"].double(), dim=-1)   # [HQ, Q, n]
    want = torch.einsum("hqn,hnd->qhd", p, V[torch.arange(24) // 3])
    _check(out.float().cpu(), want, "K2 attention vs reference scores + softmax + V")
