"""Direct CPU pins for the oracle's composite read functions, `attend_multi`, `paged_decode` and
`paged_continuation` (oracle/attend.py), on the vectors the REFERENCE wrote
(tests/golden/ref_attend_safe.npz: its `raw_scores_multi_causal` with p0 = 91 and its
`attend_raw_store` output, on a fitted 96-token store).

- `attend_multi` = softmax over keys of the reference's causal scores, times the V rows of each
  query head's KV head (impl.py:770-777).
- `paged_decode` over a shuffled paged cache holding two requests = the reference's
  `attend_raw_store` per request (the 96-token request is compared with the reference's own
  output; the 57-token one with the oracle on its contiguous slots).
- `paged_continuation` with p0 = seq_len - q_len = 91 = the same causal attention.
Planted mistakes (softmax over the wrong axis, two block ids swapped, p0 off by one) must fail."""
import pathlib

import numpy as np
import torch

from oracle import attend, codec
from oracle.layout import layout_for_config

Z = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "ref_attend_safe.npz")


def t(x):
    return torch.from_numpy(np.asarray(x))


def _fixture():
    lay = layout_for_config(codec.CONFIGS[str(Z["config"])], int(Z["r1"]), H=int(Z["H"]),
                            d=int(Z["d"]))
    return (lay, t(Z["k_slots"]), t(Z["v_slots"]), t(Z["decoder_f"]), t(Z["cos"]), t(Z["sin"]),
            t(Z["q"]), t(Z["qm"]), int(Z["p0"]))


def _cache_from(cos, sin):
    """vLLM's cos_sin_cache [max_pos, d] (cos | sin halves) that yields the fixture's rotate-half
    tables, whose two halves are equal."""
    h = cos.shape[1] // 2
    assert torch.equal(cos[:, :h], cos[:, h:]) and torch.equal(sin[:, :h], sin[:, h:])
    return torch.cat([cos[:, :h], sin[:, :h]], dim=1).contiguous()


def _want_causal(lay, vs, HQ):
    """softmax over keys of the reference's causal scores, then the V readout."""
    s = t(Z["raw_scores_multi_causal"]).double()                 # [HQ, Q, n], -inf masked
    V = attend.dense_v_from_slots(lay, vs, torch.float64)        # [H, n, d]
    p_all = torch.arange(HQ) // (HQ // lay.H)
    return torch.einsum("hqn,hnd->hqd", torch.softmax(s, dim=-1), V[p_all])


def test_attend_multi_against_reference_causal_scores():
    lay, ks, vs, dec, cos, sin, q, qm, p0 = _fixture()
    HQ = qm.shape[0]
    got = attend.attend_multi(lay, ks, vs, dec, qm, cos, sin, p0=p0, dtype=torch.float64)
    want = _want_causal(lay, vs, HQ)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    # planted mistake: softmax over the query axis instead of the keys
    s = t(Z["raw_scores_multi_causal"]).double()
    wrong = torch.einsum("hqn,hnd->hqd", torch.softmax(s.masked_fill(torch.isinf(s), -1e30), 1),
                         attend.dense_v_from_slots(lay, vs, torch.float64)[
                             torch.arange(HQ) // (HQ // lay.H)])
    assert (wrong - got).abs().max() > 1e-2


def _paged_two(ks, vs, n1, bs=16, swap=False):
    """Two requests over one shuffled paged cache: request 0 = all 96 fixture tokens, request 1 =
    the first n1 of them, in separately owned blocks."""
    blob = torch.cat([ks, vs], dim=1)
    n0 = blob.shape[0]
    need = [-(-n0 // bs), -(-n1 // bs)]
    g = torch.Generator().manual_seed(11)
    perm = torch.randperm(sum(need) + 2, generator=g).to(torch.int32)
    bt = torch.full((2, max(need)), -1, dtype=torch.int32)
    bt[0, :need[0]] = perm[:need[0]]
    bt[1, :need[1]] = perm[need[0]:need[0] + need[1]]
    flat = torch.zeros((sum(need) + 2) * bs, blob.shape[1] + 6, dtype=torch.uint8)  # wider rows
    for r, n in enumerate((n0, n1)):
        p = torch.arange(n)
        flat[bt[r, p // bs].long() * bs + p % bs, :blob.shape[1]] = blob[:n]
    if swap:
        bt[0, [1, 3]] = bt[0, [3, 1]]
    return flat, bt, torch.tensor([n0, n1], dtype=torch.int32)


def test_paged_decode_two_requests_against_reference():
    lay, ks, vs, dec, cos, sin, q, qm, p0 = _fixture()
    csc = _cache_from(cos, sin)
    n1 = 57
    flat, bt, lens = _paged_two(ks, vs, n1)
    query = torch.stack([q, q.flip(0)])                          # [N=2, HQ, d]
    got = attend.paged_decode(lay, flat, bt, lens, torch.arange(3), query, [dec, dec], csc, 16,
                              128 ** -0.5, dtype=torch.float64)
    torch.testing.assert_close(got[0].float(), t(Z["attend_raw_store"]), rtol=1e-5, atol=1e-5)
    want1 = attend.attend_raw_store(lay, ks[:n1], vs[:n1], dec, q.flip(0), cos[:n1], sin[:n1],
                                    dtype=torch.float64)
    torch.testing.assert_close(got[1], want1, rtol=1e-9, atol=1e-9)
    # planted mistake: two block ids of request 0 swapped
    flat_s, bt_s, _ = _paged_two(ks, vs, n1, swap=True)
    bad = attend.paged_decode(lay, flat, bt_s, lens, torch.arange(3), query, [dec, dec], csc, 16,
                              128 ** -0.5, dtype=torch.float64)
    assert (bad[0].float() - t(Z["attend_raw_store"])).abs().max() > 1e-3


def test_paged_continuation_against_reference_causal_scores():
    lay, ks, vs, dec, cos, sin, q, qm, p0 = _fixture()
    csc = _cache_from(cos, sin)
    HQ, Q, d = qm.shape
    flat, bt, lens = _paged_two(ks, vs, 40)
    assert int(lens[0]) - Q == p0                                 # p0 = seq_len - q_len
    query = torch.cat([qm.permute(1, 0, 2), torch.zeros(3, HQ, d)])  # request 1: 3 queries
    qsl = torch.tensor([0, Q, Q + 3])
    got = attend.paged_continuation(lay, flat, bt, lens, qsl, query, [dec, dec], csc, 16,
                                    128 ** -0.5, rows=[0], dtype=torch.float64)
    want = _want_causal(lay, vs, HQ)                              # [HQ, Q, d]
    torch.testing.assert_close(got[0], want.permute(1, 0, 2), rtol=1e-5, atol=1e-5)
    # planted mistake: p0 one too large (each query sees one more key)
    wrong = attend.attend_multi(lay, ks, vs, dec, qm, cos, sin, p0=p0 + 1, dtype=torch.float64)
    assert (wrong.permute(1, 0, 2) - got[0]).abs().max() > 1e-4
