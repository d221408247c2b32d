"""Shared test fixtures: seeded compressed stores built by the CPU oracle, and paged caches.

Test infrastructure only (imports the oracle as the checker)."""
from __future__ import annotations

import torch

from oracle import codec, encode, rope as orope
from oracle.layout import layout_for_config
from vllm_ttkv import synth

H, D, HQ = 8, 128, 24


def fitted_store(cfg_name: str, T: int, seed: int, r1: int = 110, HQ_: int = HQ):
    """One request's store: fit on the whole context (fit_into_budget), then slots."""
    cfg = codec.CONFIGS[cfg_name]
    lay = layout_for_config(cfg, r1=r1)
    K = synth.keys(T, seed=seed)
    V = synth.values(T, seed=seed)
    fk = encode.fit_into_budget(K, lay, cfg)
    ks = encode.k_slots_from(lay, fk["coeff_q"], fk["coeff_scale"], fk["resid"])
    vs = encode.v_slots_from(lay, encode.encode_v(V, lay))
    return dict(lay=lay, cfg=cfg, K=K, V=V, decoder=fk["decoder_f"], k_slots=ks, v_slots=vs,
                blob=torch.cat([ks, vs], dim=1).contiguous())


def paged(stores, block_size: int = 16, seed: int = 0, width_pad: int = 0):
    """Scatter per-request blobs into one shuffled paged cache (CPU tensors).

    Returns dict(page [num_blocks*bs, C+width_pad] u8, block_table, seq_lens, num_blocks)."""
    lens = [s["blob"].shape[0] for s in stores]
    bt, nblk = synth.shuffled_block_table(lens, block_size, seed=seed, extra_blocks=3)
    C = stores[0]["blob"].shape[1]
    page = torch.zeros(nblk * block_size, C + width_pad, dtype=torch.uint8)
    for r, s in enumerate(stores):
        n = lens[r]
        pos = torch.arange(n)
        slots = bt[r, pos // block_size].long() * block_size + pos % block_size
        page[slots, :C] = s["blob"]
    return dict(page=page, block_table=bt, seq_lens=torch.tensor(lens, dtype=torch.int32),
                num_blocks=nblk)


def llama3_cache(max_pos: int):
    inv = orope.inv_freq_llama3(D, **orope.LLAMA32_3B_ROPE)
    return orope.vllm_cos_sin_cache(inv, max_pos)
