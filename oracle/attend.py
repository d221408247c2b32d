"""Read path: the reference's dense oracle plus its paged addressing (TEST INFRASTRUCTURE ONLY).

Reference: `vllm_ttkv/reference.py:63-181` (dense reconstruction, per-row RoPE, scores, softmax,
V readout, two index orders), `vllm_ttkv/decode.py:160-197, 307-339` (slot ids from a block table,
gather), `vllm_ttkv/impl.py:511-540` (decode: UNSCALED scores * scale -> softmax -> V),
`:725-778` (continuation: `p0 = seq_len - q_len`, causal `row <= p0 + j`).

`dtype` selects the arithmetic (float32 mirrors the reference; float64 gives a tighter checker).
"""
from __future__ import annotations

import torch

from . import codec
from .layout import Layout, split_blob, unpack_k_slots, unpack_v_slots
from .rope import rope_apply


def dense_k_from_slots(lay: Layout, k_slots, decoder_f, dtype=torch.float32):
    """reference.py:63-76 -> RAW K [H, n, d]."""
    n, H, d = k_slots.shape[0], lay.H, lay.d
    cq, cs, (bm, pk, sc) = unpack_k_slots(lay, k_slots)
    if lay.qbits == 8:
        kflat = (cq.to(dtype) * cs.to(dtype).unsqueeze(1)) @ decoder_f.to(dtype)
    else:  # this build's fp16 / 4-bit coefficient modes: cq holds the stored values themselves
        kflat = cq.to(dtype) @ decoder_f.to(dtype)
    R = codec.packed_rows_materialise(bm, pk, sc, d, lay.res_k, lay.res_bits).to(dtype)
    return (kflat.reshape(n, H, d).permute(1, 0, 2) + R.reshape(H, n, d)).contiguous()


def dense_v_from_slots(lay: Layout, v_slots, dtype=torch.float32):
    """reference.py:79-85 -> V [H, n, d]."""
    n, H, d = v_slots.shape[0], lay.H, lay.d
    bm, pk, sc = unpack_v_slots(lay, v_slots)
    return codec.packed_rows_materialise(bm, pk, sc, d, lay.v_lanes, lay.v_bits).to(dtype) \
        .reshape(H, n, d).contiguous()


def raw_scores(lay, k_slots, decoder_f, query, cos, sin, scale=None, dtype=torch.float32):
    """reference.py:94-109 -> [n, HQ], scaled, each row rotated by its own position."""
    K_pre = dense_k_from_slots(lay, k_slots, decoder_f, dtype)
    HQ, d = query.shape
    scale = d ** -0.5 if scale is None else scale
    K_post = rope_apply(K_pre.permute(1, 0, 2), cos.to(dtype).unsqueeze(1),
                        sin.to(dtype).unsqueeze(1))
    p_all = torch.arange(HQ) // (HQ // lay.H)
    return torch.einsum("npd,pd->np", K_post[:, p_all, :], query.to(dtype)) * scale


def raw_scores_multi(lay, k_slots, decoder_f, query, cos, sin, scale=None, p0=None,
                     dtype=torch.float32):
    """reference.py:112-146. query [HQ, Q, d] post-RoPE -> [HQ, Q, n], -inf where row > p0+j."""
    K_pre = dense_k_from_slots(lay, k_slots, decoder_f, dtype)
    H, n, d = K_pre.shape
    HQ, Q, _ = query.shape
    scale = d ** -0.5 if scale is None else scale
    K_post = rope_apply(K_pre.permute(1, 0, 2), cos.to(dtype).unsqueeze(1),
                        sin.to(dtype).unsqueeze(1))
    p_all = torch.arange(HQ) // (HQ // H)
    s = torch.einsum("hqd,phd->hqp", query.to(dtype), K_post[:, p_all, :]) * scale
    if p0 is not None:
        pos = p0 + torch.arange(Q)
        allow = torch.arange(n)[None, :] <= pos[:, None]
        s = s.masked_fill(~allow[None, :, :], float("-inf"))
    return s


def attend_raw_store(lay, k_slots, v_slots, decoder_f, query, cos, sin, scale=None,
                     dtype=torch.float32):
    """reference.py:149-163. query [HQ, d] -> [HQ, d]."""
    HQ = query.shape[0]
    s = raw_scores(lay, k_slots, decoder_f, query, cos, sin, scale, dtype)
    p = torch.softmax(s, dim=0)
    V = dense_v_from_slots(lay, v_slots, dtype)
    p_all = torch.arange(HQ) // (HQ // lay.H)
    return torch.einsum("np,npd->pd", p, V.permute(1, 0, 2)[:, p_all, :])


def oracle_attend(lay, k_slots, v_slots, decoder_f, query, cos, sin, scale=None,
                  dtype=torch.float32):
    """reference.py:166-181: same attention in [head, group, dim] order."""
    K_pre = dense_k_from_slots(lay, k_slots, decoder_f, dtype)
    V = dense_v_from_slots(lay, v_slots, dtype)
    H, n, d = K_pre.shape
    HQ = query.shape[0]
    G = HQ // H
    scale = d ** -0.5 if scale is None else scale
    K_post = rope_apply(K_pre, cos.to(dtype).unsqueeze(0), sin.to(dtype).unsqueeze(0))
    q = query.to(dtype).reshape(H, G, d)
    p = torch.softmax(torch.einsum("hgd,hnd->hgn", q, K_post) * scale, dim=-1)
    return torch.einsum("hgn,hnd->hgd", p, V).reshape(HQ, d)


def attend_multi(lay, k_slots, v_slots, decoder_f, query, cos, sin, scale=None, p0=None,
                 dtype=torch.float32):
    """impl.py:770-777: continuation attention. query [HQ, Q, d] -> [HQ, Q, d]."""
    s = raw_scores_multi(lay, k_slots, decoder_f, query, cos, sin, scale, p0, dtype)
    p = torch.softmax(s, dim=-1)
    V = dense_v_from_slots(lay, v_slots, dtype)                            # [H, n, d]
    HQ = query.shape[0]
    p_all = torch.arange(HQ) // (HQ // lay.H)
    return torch.einsum("hqn,hnd->hqd", p, V[p_all])


# ------------------------------------------------------------------ paged addressing
def block_slots(block_row: torch.Tensor, seq_len: int, block_size: int) -> torch.Tensor:
    """decode.py:307-339: slot id = block_table[r, p // bs] * bs + p % bs."""
    if seq_len == 0:
        return torch.zeros(0, dtype=torch.long)
    pos = torch.arange(seq_len)
    idx = pos // block_size
    if int(idx.max()) >= block_row.shape[0]:
        raise IndexError("seq_len needs more blocks than the block table row holds")
    return block_row[idx].to(torch.long) * block_size + pos % block_size


def gather_request(lay: Layout, flat: torch.Tensor, block_row, seq_len: int, block_size: int):
    """decode.py:160-197 + 286-304 -> (k_slots [n,k], v_slots [n,v])."""
    slots = block_slots(block_row, seq_len, block_size)
    blob = flat[slots, :lay.compressed_bytes_per_token()].contiguous()
    return split_blob(lay, blob)


def paged_decode(lay: Layout, flat, block_table, seq_lens, query_start_loc, query, decoders,
                 cos_sin_cache, block_size: int, scale: float, dtype=torch.float32):
    """impl.py:452-493 + 511-540: the reference's per-request decode loop over a paged batch.

    flat [n_slots, W] uint8; query [N, HQ, d] post-RoPE; decoders: list of [r1, H*d] per request.
    Returns [B, HQ, d] in `dtype` (one row per decode request, at query_start_loc[r])."""
    from .rope import cos_sin_from_cache
    out = []
    for r in range(block_table.shape[0]):
        n = int(seq_lens[r])
        k, v = gather_request(lay, flat, block_table[r], n, block_size)
        cos, sin = cos_sin_from_cache(cos_sin_cache, torch.arange(n), lay.d)
        q = query[int(query_start_loc[r])]
        out.append(attend_raw_store(lay, k, v, decoders[r], q, cos, sin, scale, dtype))
    return torch.stack(out)


def paged_continuation(lay: Layout, flat, block_table, seq_lens, query_start_loc, query,
                       decoders, cos_sin_cache, block_size: int, scale: float, rows=None,
                       dtype=torch.float32):
    """impl.py:725-778: `_prefill_continuation` for each request in `rows` (default: all).

    Request r's queries are rows query_start_loc[r]..[r+1] of query [N, HQ, d] (post-RoPE); they
    attend over the seq_lens[r] stored keys with p0 = seq_len - q_len. Returns {r: [Q, HQ, d]}."""
    from .rope import cos_sin_from_cache
    rows = range(block_table.shape[0]) if rows is None else rows
    out = {}
    for r in rows:
        n = int(seq_lens[r])
        s, e = int(query_start_loc[r]), int(query_start_loc[r + 1])
        k, v = gather_request(lay, flat, block_table[r], n, block_size)
        cos, sin = cos_sin_from_cache(cos_sin_cache, torch.arange(n), lay.d)
        q = query[s:e].permute(1, 0, 2)
        o = attend_multi(lay, k, v, decoders[r], q, cos, sin, scale, p0=n - (e - s), dtype=dtype)
        out[r] = o.permute(1, 0, 2)
    return out
