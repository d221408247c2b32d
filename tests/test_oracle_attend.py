"""Pins for the oracle's read path (oracle/attend.py, oracle/rope.py): two index orders, float64
brute force, negative controls on rotation, causal pattern, RoPE conventions.

Reference: vllm_ttkv/reference.py:47-181, tests/test_reference.py:69-113,
tests/test_decode_conventions.py:38-168, tests/test_krt_multi.py:108-172."""
import math

import pytest
import torch

from helpers import fitted_store, llama3_cache
from oracle import attend, codec, encode, rope
from oracle.layout import Layout, layout_for_config, pack_k_slots, pack_v_slots


def _tiny_store(seed=0, n=6, H=2, d=16, r1=8):
    lay = Layout(H=H, d=d, r1=r1, qbits=8, res_k=5, res_bits=3, v_lanes=7, v_bits=3)
    g = torch.Generator().manual_seed(seed)
    cq = torch.randint(-127, 128, (n, r1), generator=g, dtype=torch.int8)
    cs = (torch.rand(n, generator=g) * 0.02 + 0.001).to(torch.float16)
    dec = torch.randn(r1, H * d, generator=g)
    R = torch.randn(H * n, d, generator=g) * 0.1
    V = torch.randn(H * n, d, generator=g)
    ks = pack_k_slots(lay, cq, cs, *codec.build_rows(R, 5, 3))
    vs = pack_v_slots(lay, *codec.build_rows(V, 7, 3))
    return lay, ks, vs, dec


def test_brute_force_float64_loops():
    """Every step written out element by element in float64."""
    lay, ks, vs, dec = _tiny_store()
    n, H, d, HQ = ks.shape[0], 2, 16, 4
    g = torch.Generator().manual_seed(3)
    q = torch.randn(HQ, d, generator=g)
    pos = torch.arange(n)
    inv = rope.inv_freq_theta(d)
    cos, sin = rope.cos_sin_from_cache(rope.vllm_cos_sin_cache(inv, 16), pos, d)
    Kd = attend.dense_k_from_slots(lay, ks, dec, torch.float64)
    Vd = attend.dense_v_from_slots(lay, vs, torch.float64)
    cq, cs, _ = __import__("oracle.layout", fromlist=["x"]).unpack_k_slots(lay, ks)
    out = torch.zeros(HQ, d, dtype=torch.float64)
    scale = d ** -0.5
    for p in range(HQ):
        h = p // (HQ // H)
        s = []
        for t in range(n):
            k = [sum(float(cq[t, a]) * float(cs[t]) * float(dec[a, h * d + j]) for a in range(lay.r1))
                 for j in range(d)]
            rres = Kd[h, t] - torch.tensor(k, dtype=torch.float64)      # residual lanes
            kv = [k[j] + float(rres[j]) for j in range(d)]
            half = d // 2
            y = [0.0] * d
            for j in range(half):
                c, sn = math.cos(t * float(inv[j])), math.sin(t * float(inv[j]))
                y[j] = kv[j] * c - kv[j + half] * sn
                y[j + half] = kv[j + half] * c + kv[j] * sn
            s.append(scale * sum(float(q[p, j]) * y[j] for j in range(d)))
        m = max(s)
        w = [math.exp(x - m) for x in s]
        Z = sum(w)
        for t in range(n):
            out[p] += (w[t] / Z) * Vd[h, t]
    got = attend.attend_raw_store(lay, ks, vs, dec, q, cos, sin, dtype=torch.float64)
    assert (got - out).abs().max() < 1e-6


def test_two_index_orders_agree():
    st = fitted_store("campaign4x", 96, seed=0)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(24, 128, generator=g) * 0.1
    cos, sin = rope.cos_sin_from_cache(llama3_cache(128), torch.arange(96), 128)
    a = attend.attend_raw_store(st["lay"], st["k_slots"], st["v_slots"], st["decoder"], q, cos, sin)
    b = attend.oracle_attend(st["lay"], st["k_slots"], st["v_slots"], st["decoder"], q, cos, sin)
    assert ((a - b).abs().max() / b.abs().max()) < 1e-5


def test_rotation_negative_controls():
    st = fitted_store("safe", 96, seed=2)
    q = torch.randn(24, 128, generator=torch.Generator().manual_seed(2))
    cos, sin = rope.cos_sin_from_cache(llama3_cache(128), torch.arange(96), 128)
    kw = dict(lay=st["lay"], k_slots=st["k_slots"], decoder_f=st["decoder"], query=q)
    good = attend.raw_scores(cos=cos, sin=sin, **kw)
    unrot = attend.raw_scores(cos=torch.ones_like(cos), sin=torch.zeros_like(sin), **kw)
    rolled = attend.raw_scores(cos=cos.roll(1, 0), sin=sin.roll(1, 0), **kw)
    assert ((good - unrot).abs().max() / good.abs().max()) > 0.5
    assert ((good - rolled).abs().max() / good.abs().max()) > 1e-2


def test_multi_query_causal_and_q1_equivalence():
    st = fitted_store("safe", 40, seed=4)
    g = torch.Generator().manual_seed(5)
    Q, p0 = 6, 34
    q = torch.randn(24, Q, 128, generator=g)
    cos, sin = rope.cos_sin_from_cache(llama3_cache(64), torch.arange(40), 128)
    s = attend.raw_scores_multi(st["lay"], st["k_slots"], st["decoder"], q, cos, sin, p0=p0)
    allow = torch.arange(40)[None, :] <= (p0 + torch.arange(Q))[:, None]
    assert torch.equal(torch.isfinite(s), allow[None].expand_as(s))
    assert torch.isfinite(s[:, -1]).all()                              # last query sees all rows
    single = attend.raw_scores(st["lay"], st["k_slots"], st["decoder"], q[:, 0], cos, sin)
    multi = attend.raw_scores_multi(st["lay"], st["k_slots"], st["decoder"], q[:, :1], cos, sin)
    assert torch.allclose(multi[:, 0].T, single, atol=1e-5)


def test_vllm_half_layout_translation():
    """test_decode_conventions.py:38-74 restated: the duplicated table reproduces vLLM's
    rotate-half on the cache halves; a mis-built table moves the result a lot."""
    d, n = 128, 24
    cache = rope.vllm_cos_sin_cache(rope.inv_freq_theta(d), n)
    cos, sin = rope.cos_sin_from_cache(cache, torch.arange(n), d)
    x = torch.randn(n, d, generator=torch.Generator().manual_seed(0))
    c, s = cache[:, :64], cache[:, 64:]
    want = torch.cat([x[:, :64] * c - x[:, 64:] * s, x[:, 64:] * c + x[:, :64] * s], -1)
    assert (rope.rope_apply(x, cos, sin) - want).abs().max() < 1e-6
    assert (rope.rope_apply(x, cache, cache) - want).abs().max() / want.abs().max() > 0.1
    with pytest.raises(IndexError):
        rope.cos_sin_from_cache(cache, torch.tensor([n]), d)
    with pytest.raises(NotImplementedError):
        rope.cos_sin_from_cache(cache[:, :64], torch.arange(2), d)


def test_llama3_frequencies_match_transformers():
    tr = pytest.importorskip("transformers.modeling_rope_utils")
    from transformers import LlamaConfig
    cfg = LlamaConfig(hidden_size=3072, num_attention_heads=24, num_key_value_heads=8,
                      head_dim=128, max_position_embeddings=131072, rope_theta=500000.0,
                      rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                    "high_freq_factor": 4.0,
                                    "original_max_position_embeddings": 8192})
    fn = tr.ROPE_INIT_FUNCTIONS["llama3"]
    inv_ref, _ = fn(cfg, "cpu")
    ours = rope.inv_freq_llama3(128, **rope.LLAMA32_3B_ROPE)
    assert torch.allclose(ours, inv_ref.float(), rtol=1e-6, atol=0)
    from vllm_ttkv import rope as prope
    assert torch.equal(prope.llama3_inv_freq(128), ours)


def test_block_slots_flat_indexing():
    """test_decode_conventions.py:152-168 restated."""
    bt = torch.tensor([3, 7, 11], dtype=torch.int32)
    s = attend.block_slots(bt, 40, 16)
    assert s.tolist()[:17] == [48 + i for i in range(16)] + [112]
    assert s.tolist()[-1] == 11 * 16 + 7 and len(s) == 40
    with pytest.raises(IndexError):
        attend.block_slots(bt, 49, 16)
