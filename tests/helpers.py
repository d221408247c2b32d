"""Shared test fixtures: seeded compressed stores built by the CPU oracle, and paged caches.

Test infrastructure only (imports the oracle as the checker)."""
from __future__ import annotations

import torch

from oracle import codec, encode, rope as orope
from oracle.layout import layout_for_config
from vllm_ttkv import synth

H, D, HQ = 8, 128, 24


def fitted_store(cfg_name: str, T: int, seed: int, r1: int = 110, HQ_: int = HQ,
                 v_scale=None, H_: int = H):
    """One request's store of H_ KV heads: fit on the whole context (fit_into_budget), then
    slots. `v_scale` (a number or a [T] tensor of per-token factors) multiplies the values before
    encoding."""
    cfg = codec.CONFIGS[cfg_name]
    lay = layout_for_config(cfg, r1=r1, H=H_)
    K = synth.keys(T, H=H_, seed=seed)
    V = synth.values(T, H=H_, seed=seed)
    if v_scale is not None:
        V = V * (v_scale if not torch.is_tensor(v_scale) else v_scale.reshape(1, T, 1))
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


def dec_pool_of(decoders, dev: str = "cuda"):
    """The product's decoder pool (`DecoderPool`, int8 + rank rulers) holding fp32 `decoders`
    ([r1, H*d] each, fitted, so exactly int8 x ruler), one slot per decoder, on `dev`."""
    from vllm_ttkv.decoder_pool import pack_decoders
    return pack_decoders(torch.stack([d.to(torch.float32) for d in decoders]).to(dev))


def llama3_cache(max_pos: int):
    inv = orope.inv_freq_llama3(D, **orope.LLAMA32_3B_ROPE)
    return orope.vllm_cos_sin_cache(inv, max_pos)


def device_store(cfg_name: str, lens, seed: int, r1: int = 110, block_size: int = 16,
                 fit_on: int = 2048, dev: str = "cuda"):
    """A paged store for requests of `lens` tokens, built the way serving builds it: each
    request's first `fit_on` tokens fitted on the device (`vllm_ttkv.encode.fit_into_budget`) and
    every token packed by the K3 write kernel (the first chunk from the fit's coefficients, the
    rest by frozen projection; in the fp16 / 4-bit coefficient modes every token is projected). Full-size stores in seconds, where the CPU oracle's fit would take
    minutes; the oracle then reads the SAME slot bytes, so K1/K2 are checked against it exactly
    as on a store the oracle built.

    Returns dict(lay (oracle Layout), play (product TTKLayout), page [n_slots, C] u8 (device),
    block_table, seq_lens, dec_map, dec_pool (DecoderPool), pinv_pool (device), decoders (CPU
    fp32 list), num_blocks).
    """
    from vllm_ttkv import encode as penc, kernels
    from vllm_ttkv.layout import config_named, layout_for_config as play_for

    pcfg = config_named(cfg_name)  # a shipped allocation or a coefficient-mode extension
    lay = layout_for_config(pcfg, r1=r1)
    play = play_for(pcfg, r1)
    B = len(lens)
    bt, nblk = synth.shuffled_block_table(lens, block_size, seed=seed, extra_blocks=3)
    C = lay.compressed_bytes_per_token()
    page = torch.zeros(nblk * block_size, C, dtype=torch.uint8, device=dev)
    from vllm_ttkv.decoder_pool import empty_pool
    dec_pool = empty_pool(B, r1, H, D, dev)
    dec_f = torch.zeros(B, r1, H * D, dtype=torch.float32, device=dev)
    pinv_pool = torch.zeros(B, r1, H * D, dtype=torch.float32, device=dev)
    dec_map = torch.full((nblk,), -1, dtype=torch.int32)
    for r in range(B):
        dec_map[bt[r, 0]] = r
    bt_d, dec_map_d = bt.to(dev), dec_map.to(dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    fk_all, rest = [], []
    for r, n in enumerate(lens):
        s = seed * 1000003 + r
        K = synth.keys(n, seed=s, device=dev).permute(1, 0, 2)      # [n, H, d]
        V = synth.values(n, seed=s, device=dev).permute(1, 0, 2)
        f = min(fit_on, n)
        fk = penc.fit_into_budget(K[:f].permute(1, 0, 2).contiguous(), play, pcfg)
        dec_f[r] = fk.decoder.decoder_f
        dec_pool.q[r].copy_(fk.decoder.packed.q)
        dec_pool.scale[r].copy_(fk.decoder.packed.scale)
        pinv_pool[r] = fk.decoder.pinv.t()
        p = torch.arange(n)
        slot = (bt[r, p // block_size].long() * block_size + p % block_size).to(dev)
        fk_all.append((K[:f], V[:f], slot[:f], fk.coeff_q, fk.coeff_scale))
        rest.append((K[f:], V[f:], slot[f:]))

    def _write(parts, cq=None, cs=None):
        ln = [x[0].shape[0] for x in parts]
        if not sum(ln):
            return
        reqs = [i for i, l in enumerate(ln) if l]
        qsl = torch.tensor([0] + list(torch.tensor([ln[i] for i in reqs]).cumsum(0)),
                           dtype=torch.int32, device=dev)
        kernels.write_paged(play, torch.cat([parts[i][0] for i in reqs]).contiguous(),
                            torch.cat([parts[i][1] for i in reqs]).contiguous(),
                            torch.cat([parts[i][2] for i in reqs]), qsl,
                            bt_d[torch.tensor(reqs, device=dev)].contiguous(), dec_map_d,
                            dec_pool, pinv_pool, page,
                            coeff_q_in=None if cq is None else torch.cat([cq[i] for i in reqs]),
                            coeff_scale_in=None if cs is None else torch.cat([cs[i] for i in reqs]),
                            error_word=err)

    if play.qbits == 8:
        _write(fk_all, [x[3] for x in fk_all], [x[4] for x in fk_all])
    else:  # fp16 / 4-bit coefficients: the first chunk is projected too
        _write(fk_all)
    _write(rest)
    torch.cuda.synchronize()
    if int(err.item()):
        raise RuntimeError(f"store build: device error word {int(err.item())}")
    return dict(lay=lay, play=play, page=page, block_table=bt_d, seq_lens=torch.tensor(
        lens, dtype=torch.int32, device=dev), dec_map=dec_map_d, dec_pool=dec_pool,
        pinv_pool=pinv_pool, decoders=[dec_f[r].cpu() for r in range(B)], num_blocks=nblk,
        block_size=block_size)


def config3_lens(seed: int = 3, B: int = 8):
    """BASELINE config 3's contexts: 8 lengths drawn uniformly from [1000, 14400], seeded."""
    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(1000, 14401, (B,), generator=g)]
