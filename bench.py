"""Benchmark: the fused compressed-KV decode read (K1) on one MI355X.

Headline workload: Llama-3.2-3B attention geometry (24 q heads, 8 KV heads,
head dim 128, 28 layers), `safe` allocation at r1 = 110, block size 16, 8 concurrent requests at
14,402 cached tokens each, one decode query per request per step. One step = 28 K1 launches (one
per layer, each over the whole batch). `value` = decode tokens/s of the attention read alone
(8 tokens per step / step time); inputs are resident in HBM before timing starts.

Stores are built the way serving builds them, with this package's own code (never the oracle):
keys/values from the seeded synthetic generator, each request's first chunk fitted on the GPU
(`encode.fit_into_budget`), every token packed by the K3 write kernel (first chunk from the fit's
coefficients, the rest by frozen projection).

Extra fields: the batch-1 context sweep (1082/4322/8642/14402), batch 8 with seeded random
contexts U[1000, 14400] (config 3), the multi-query continuation score (config 4) and the
4-bit store with one write per request per layer (config 5) when their kernels are built, the
dense fp16 paged-attention comparator, the container-layout reads, first-chunk timings, K1 over
this package's fp16 and 4-bit group-32 coefficient modes at the headline shape, the K1 roofline
(HBM bytes per launch / measured launch time vs 8 TB/s) and the CPU baseline (the torch-CPU
oracle timed on a bounded sample on this host). `--*-only` flags run one extra alone.

Timing: the headline's K steps (and config 3's, and the dense comparator's launches) run back to
back with HIP events only around the timed region, so a launch's time includes the gap to the
next launch but no per-launch event packets; the per-launch event-pair figure is reported beside
it. The batch-1 sweep flushes the caches between launches (its layers would otherwise stay in
the Infinity Cache) and so is timed per launch. Config 5's K3 / K1 split comes from HIP-graph
replays of one step's writes alone and reads alone.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ttkv-vllm_amd"))

HBM_PEAK_GBPS = 8000.0
L_LAYERS, HQ, H, D, BS = 28, 24, 8, 128, 16
R1, FIT_ON = 110, 2048


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_store(torch, lay, cfg, lens, n_layers, seed, dev, fit_on=FIT_ON, distinct=4):
    """Per-layer paged caches for requests of `lens` tokens. Returns a dict of device tensors."""
    from vllm_ttkv import encode, kernels, synth
    from vllm_ttkv.decoder_pool import DecoderPool, empty_pool
    bt, nblk = synth.shuffled_block_table(lens, BS, seed=seed, extra_blocks=4)
    B = len(lens)
    C = lay.compressed_bytes_per_token()
    dec_map = torch.full((nblk,), -1, dtype=torch.int32)
    for r in range(B):
        dec_map[bt[r, 0]] = r
    bt_d, dec_map_d = bt.to(dev), dec_map.to(dev)
    pos_slot = []
    for r, n in enumerate(lens):
        p = torch.arange(n)
        pos_slot.append((bt[r, p // BS].long() * BS + p % BS).to(dev))
    layers = []
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    t_fit = t_write = 0.0
    for li in range(n_layers):
        if li >= distinct:
            # replicate a built layer into this layer's own pages (distinct HBM addresses)
            src = layers[li % distinct]
            layers.append(dict(page=src["page"].clone(),
                               dec_pool=DecoderPool(src["dec_pool"].q.clone(),
                                                    src["dec_pool"].scale.clone()),
                               pinv_pool=src["pinv_pool"].clone(), dec_f=src["dec_f"]))
            continue
        page = torch.zeros(nblk * BS, C, dtype=torch.uint8, device=dev)
        dec_pool = empty_pool(B, lay.r1, H, D, dev)
        dec_f = torch.zeros(B, lay.r1, H * D, dtype=torch.float32, device=dev)  # CPU baselines
        pinv_pool = torch.zeros(B, lay.r1, H * D, dtype=torch.float32, device=dev)
        first_k, first_v, first_cq, first_cs, first_slot, rest = [], [], [], [], [], []
        for r, n in enumerate(lens):
            s = seed * 1000003 + li * 1009 + r
            K = synth.keys(n, seed=s, device=dev)
            V = synth.values(n, seed=s, device=dev)
            f = min(fit_on, n)
            t0 = time.perf_counter()
            fk = encode.fit_into_budget(K[:, :f], lay, cfg)
            dec_f[r] = fk.decoder.decoder_f
            dec_pool.q[r].copy_(fk.decoder.packed.q)
            dec_pool.scale[r].copy_(fk.decoder.packed.scale)
            pinv_pool[r] = fk.decoder.pinv.t()
            torch.cuda.synchronize()
            t_fit += time.perf_counter() - t0
            Kt, Vt = K.permute(1, 0, 2), V.permute(1, 0, 2)
            first_k.append(Kt[:f]); first_v.append(Vt[:f])
            first_cq.append(fk.coeff_q); first_cs.append(fk.coeff_scale)
            first_slot.append(pos_slot[r][:f])
            rest.append((Kt[f:], Vt[f:], pos_slot[r][f:]))
        t0 = time.perf_counter()
        fl = [x.shape[0] for x in first_k]
        qsl = torch.tensor([0] + list(torch.tensor(fl).cumsum(0)), dtype=torch.int32, device=dev)
        kernels.write_paged(lay, torch.cat(first_k).contiguous(), torch.cat(first_v).contiguous(),
                            torch.cat(first_slot), qsl, bt_d, dec_map_d, dec_pool, pinv_pool,
                            page,
                            coeff_q_in=torch.cat(first_cq) if lay.qbits == 8 else None,
                            coeff_scale_in=torch.cat(first_cs) if lay.qbits == 8 else None,
                            error_word=err)
        rl = [x[0].shape[0] for x in rest]
        if sum(rl):
            qsl = torch.tensor([0] + list(torch.tensor(rl).cumsum(0)), dtype=torch.int32,
                               device=dev)
            kernels.write_paged(lay, torch.cat([x[0] for x in rest]).contiguous(),
                                torch.cat([x[1] for x in rest]).contiguous(),
                                torch.cat([x[2] for x in rest]), qsl, bt_d, dec_map_d, dec_pool,
                                pinv_pool, page, error_word=err)
        torch.cuda.synchronize()
        t_write += time.perf_counter() - t0
        del first_k, first_v, rest
        layers.append(dict(page=page, dec_pool=dec_pool, pinv_pool=pinv_pool, dec_f=dec_f))
    if int(err.item()):
        raise RuntimeError(f"store build: device error word {int(err.item())}")
    return dict(layers=layers, bt=bt_d, dec_map=dec_map_d, nblk=nblk, B=B,
                seq_lens=torch.tensor(lens, dtype=torch.int32, device=dev), max_len=max(lens),
                t_fit=t_fit, t_write=t_write)


def bench_coef_modes(torch, cache, dev, steps=10, warmup=3, n_layers=L_LAYERS):
    """K1 at the headline shape (8 x 14,402, 28 layers back to back) over stores in this
    library's own coefficient modes (`EXTENSION_CONFIGS`: fp16 coefficients on the safe
    geometry, 4-bit group-32 coefficients on campaign4x's), each fitted and written on the device
    like the headline store."""
    from vllm_ttkv import synth
    from vllm_ttkv.layout import EXTENSION_CONFIGS, layout_for_config
    lens = [14402] * 8
    q = synth.queries(8, seed=5, device=dev)
    res = {}
    for name, mcfg in EXTENSION_CONFIGS.items():
        mlay = layout_for_config(mcfg, R1)
        st = build_store(torch, mlay, mcfg, lens, n_layers, seed=9, dev=dev)
        _, ml = time_k1(torch, mlay, st, q, cache, steps, warmup, n_layers, per_launch=False)
        b = k1_bytes(mlay, lens, R1, max(lens))
        res[name] = dict(slot_bytes=mlay.compressed_bytes_per_token(), qbits=mlay.qbits,
                         us_per_layer=ml * 1e3, algorithmic_bytes=b,
                         hbm_gbps=b / (ml * 1e-3) / 1e9,
                         roofline_frac=b / (ml * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                         ns_per_cached_token=ml * 1e6 / sum(lens))
        log(f"K1 B=8x14402 {name} ({mlay.compressed_bytes_per_token()} B/token): "
            f"{ml * 1e3:.1f} us/launch back to back")
        del st
    return res


def batch1_sweep(torch, lay, cfg, cache, dev, flush):
    """K1 at batch 1 (BASELINE config 2's contexts), 28 layers of distinct pages cycled, the
    caches flushed between launches (cold HBM), an event pair around each launch."""
    from vllm_ttkv import synth
    sweep = []
    for n in (1082, 4322, 8642, 14402):
        st = build_store(torch, lay, cfg, [n], L_LAYERS, seed=2, dev=dev)
        q1 = synth.queries(1, seed=6, device=dev)
        _, ml = time_k1(torch, lay, st, q1, cache, 3, 1, L_LAYERS, flush=flush)
        b = k1_bytes(lay, [n], R1, n)
        log(f"K1 B=1x{n}: {ml * 1e3:.1f} us/launch (cold)")
        sweep.append(dict(context=n, us_per_layer=ml * 1e3,
                          hbm_gbps=b / (ml * 1e-3) / 1e9,
                          tokens_per_s=1.0 / (ml * 1e-3 * L_LAYERS), cold_hbm=True,
                          layers_cycled=L_LAYERS))
        del st
    return sweep


def config3_lens(seed=3, B=8):
    """BASELINE config 3's contexts: 8 lengths drawn uniformly from [1000, 14400], seeded."""
    import torch
    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(1000, 14401, (B,), generator=g)]


def k1_bytes(lay, lens, r1, cs_rows):
    """Algorithmic HBM bytes of one K1 launch: every slot once, each request's decoder once in
    the pool's form (r1 x H*d int8 values and r1 fp32 rank rulers), the angle table rows once, q
    and out once (fp16)."""
    B = len(lens)
    return (sum(lens) * lay.compressed_bytes_per_token() + B * r1 * (H * D + 4)
            + cs_rows * D * 4 + 2 * B * HQ * D * 2)


def cache_flusher(torch, dev, mib=768):
    """A callable that streams a 768 MiB buffer through the memory hierarchy (read + write),
    evicting the 256 MB Infinity Cache and every XCD's L2, so the next launch reads cold HBM."""
    buf = torch.zeros(mib << 20, dtype=torch.uint8, device=dev)
    return lambda: buf.add_(1)


def time_k1(torch, lay, store, q, cache, steps, warmup, n_layers, flush=None, per_launch=True):
    """Time `steps` decode steps (n_layers K1 launches each, layer li reading its own pages).
    Returns (ms/step, ms/launch). With `flush`, the caches are flushed between launches (outside
    the per-launch events), so every launch reads cold HBM; ms/step then includes the flushes
    and only ms/launch is meaningful. With per_launch=False the steps run back to back with events
    only around the whole timed region (per-launch event pairs add ~8 us of packet processing
    per launch between kernels), and ms/launch is ms/step / n_layers."""
    from vllm_ttkv import kernels
    dev = q.device
    B = store["B"]
    qsl = torch.arange(B + 1, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    ws = kernels.decode_workspace(lay, HQ, B, store["max_len"], dev, BS)
    err = torch.zeros(1, dtype=torch.int32, device=dev)

    def step(evs=None):
        for li in range(n_layers):
            L = store["layers"][li % len(store["layers"])]
            if flush is not None:
                flush()
            if evs is not None:
                evs[li][0].record()
            kernels.decode_paged(lay, q, L["page"], BS, store["bt"], store["seq_lens"], qsl,
                                 store["max_len"], store["dec_map"], L["dec_pool"], cache,
                                 D ** -0.5, out=out, workspace=ws, error_word=err)
            if evs is not None:
                evs[li][1].record()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if not per_launch:
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            step()
        t1.record()
        torch.cuda.synchronize()
        if int(err.item()):
            raise RuntimeError(f"K1: device error word {int(err.item())}")
        ms_step = t0.elapsed_time(t1) / steps
        return ms_step, ms_step / n_layers
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(n_layers)] for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for s in range(steps):
        step(evs[s])
    t1.record()
    torch.cuda.synchronize()
    if int(err.item()):
        raise RuntimeError(f"K1: device error word {int(err.item())}")
    ms_step = t0.elapsed_time(t1) / steps
    per = [a.elapsed_time(b) for st in evs for (a, b) in st]
    return ms_step, sum(per) / len(per)


def time_back_to_back(torch, fn, steps, warmup):
    """Average ms per call of `fn` with the calls back to back and events only around the whole
    timed region (the calls' own launch gaps included, no per-call event packets)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def time_launches(torch, fn, steps, warmup):
    """Average ms per call of `fn` (one kernel launch on torch's current stream), HIP events."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / steps


def k2_flops(lens, qlens, r1):
    """Algorithmic FLOPs of one K2 attention launch: causal-visible scores and P.V
    (2*HQ*d each per visible (query, key)), and each stored key reconstructed once
    (2*H*r1*d)."""
    f = 0
    for n, Q in zip(lens, qlens):
        p0 = n - Q
        vis = Q * p0 + Q * (Q + 1) // 2
        f += 2 * 2 * HQ * D * vis + 2 * H * r1 * D * n
    return f


def _oracle_layout(lay):
    sys.path.insert(0, str(ROOT))
    from oracle.layout import Layout
    return Layout(lay.H, lay.d, lay.r1, lay.qbits, lay.res_k, lay.res_bits, lay.v_lanes, lay.v_bits)


def cpu_k2_sample(torch, lay, st, L, q_chunk, cache, n, Q):
    """The torch-CPU oracle's continuation (impl.py:770-777 restated: scores, softmax, V readout)
    for ONE request's chunk of config 4, all host threads: ms per chunk-layer."""
    from oracle import attend, rope as orope
    olay = _oracle_layout(lay)
    torch.set_num_threads(os.cpu_count() or 1)
    bt = st["bt"].cpu()
    p = torch.arange(n)
    slots = (bt[0, p // BS].long() * BS + p % BS)
    blob = L["page"][slots.to(L["page"].device)].cpu()
    k_s, v_s = blob[:, :olay.k_slot_bytes].contiguous(), blob[:, olay.k_slot_bytes:].contiguous()
    dec = L["dec_f"][0].cpu()
    cos, sin = orope.cos_sin_from_cache(cache.cpu(), p, D)
    qq = q_chunk.float().cpu().permute(1, 0, 2).contiguous()                # [HQ, Q, d]
    t0 = time.perf_counter()
    attend.attend_multi(olay, k_s, v_s, dec, qq, cos, sin, D ** -0.5, p0=n - Q)
    return (time.perf_counter() - t0) * 1e3, torch.get_num_threads()


def cpu_k3_sample(torch, lay, k_new, v_new, dec_f, pinv_pool):
    """The torch-CPU oracle's write (encode.py:301-443 restated: projection, quantisation,
    residual, top-k select and pack of K and V rows) for the B new tokens of one config-5
    step-layer, each against its own request's decoder as the reference's request loop does
    (impl.py:543-653), all host threads: ms per step-layer write."""
    from oracle import encode as oenc
    olay = _oracle_layout(lay)
    torch.set_num_threads(os.cpu_count() or 1)
    K = k_new.float().cpu().permute(1, 0, 2).contiguous()                  # [H, B, d]
    V = v_new.float().cpu().permute(1, 0, 2).contiguous()
    dec, pinv = dec_f.cpu(), pinv_pool.cpu().transpose(1, 2)   # [B, H*d, r1]
    t0 = time.perf_counter()
    for r in range(K.shape[1]):
        ef = oenc.encode_frozen(K[:, r:r + 1].contiguous(), dec[r], olay, pinv[r])
        oenc.k_slots_from(olay, ef["coeff_q"], ef["coeff_scale"], ef["resid"])
        oenc.v_slots_from(olay, oenc.encode_v(V[:, r:r + 1].contiguous(), olay))
    return (time.perf_counter() - t0) * 1e3, torch.get_num_threads()


def bench_first_chunk(torch, lay, cfg, dev, lengths=(2048, 8192), reps=5):
    """A request's first chunk, per layer: the attention over the chunk's own post-RoPE q/k/v
    (the drop-in's `TTKVAttentionImpl._sdpa`: causal SDPA in fp32, as the reference runs it,
    impl.py:716-721), the fit of its keys on the device (`encode.fit_into_budget`) and the K3
    write of its tokens with the fit's coefficients. The fp16 SDPA (model dtype, not the
    reference's arithmetic) is timed beside it for scale."""
    from vllm_ttkv import encode, kernels, synth
    from vllm_ttkv.decoder_pool import DecoderPool
    from vllm_ttkv.impl import TTKVAttentionImpl
    im = TTKVAttentionImpl(HQ, D, D ** -0.5, H)
    out = []

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    for T in lengths:
        K = synth.keys(T, seed=T, device=dev)                     # [H, T, d] raw
        V = synth.values(T, seed=T, device=dev).permute(1, 0, 2).contiguous()
        q = synth.queries(T, seed=T, device=dev)                  # [T, HQ, d] fp16
        k = K.permute(1, 0, 2).reshape(T, H * D).half()           # stands in for post-RoPE k
        v = V.reshape(T, H * D).half()
        us_sdpa = timed(lambda: im._sdpa(q, k, v))
        qh = q.transpose(0, 1).unsqueeze(0)
        kh = k.view(T, H, D).repeat_interleave(HQ // H, 1).transpose(0, 1).unsqueeze(0)
        vh = v.view(T, H, D).repeat_interleave(HQ // H, 1).transpose(0, 1).unsqueeze(0)
        us_sdpa16 = timed(lambda: torch.nn.functional.scaled_dot_product_attention(
            qh, kh, vh, is_causal=True, scale=D ** -0.5))
        fk = [None]

        def fit():
            fk[0] = encode.fit_into_budget(K, lay, cfg)
        us_fit = timed(fit)
        nblk = (T + BS - 1) // BS
        page = torch.zeros(nblk * BS, lay.compressed_bytes_per_token(), dtype=torch.uint8,
                           device=dev)
        bt = torch.arange(nblk, dtype=torch.int32, device=dev).reshape(1, nblk)
        dec_map = torch.full((nblk,), -1, dtype=torch.int32, device=dev)
        dec_map[0] = 0
        dec_pool = DecoderPool(fk[0].decoder.packed.q.unsqueeze(0).contiguous(),
                               fk[0].decoder.packed.scale.unsqueeze(0).contiguous())
        # the decoder's registration (its pseudo-inverse, for the frozen projection of the
        # request's later tokens; rope_store.register)
        us_reg = timed(lambda: encode.KDecoder(fk[0].decoder.decoder_f).pinv)
        pinv_pool = fk[0].decoder.pinv.t().unsqueeze(0).contiguous()
        qsl = torch.tensor([0, T], dtype=torch.int32, device=dev)
        slots = torch.arange(T, dtype=torch.int64, device=dev)
        Kt = K.permute(1, 0, 2).contiguous()
        us_write = timed(lambda: kernels.write_paged(
            lay, Kt, V, slots, qsl, bt, dec_map, dec_pool, pinv_pool, page,
            coeff_q_in=fk[0].coeff_q, coeff_scale_in=fk[0].coeff_scale))
        row = dict(tokens=T, sdpa_fp32_us=us_sdpa, sdpa_fp16_us=us_sdpa16, fit_us=us_fit,
                   register_us=us_reg, write_us=us_write,
                   total_us=us_sdpa + us_fit + us_reg + us_write)
        log(f"first chunk {T}: SDPA fp32 {us_sdpa:.0f} us (fp16 {us_sdpa16:.0f}), fit "
            f"{us_fit:.0f} us, registration {us_reg:.0f} us, write {us_write:.0f} us per layer")
        out.append(row)
        del K, V, q, k, v, qh, kh, vh, page
    return dict(per_layer=out, note="one request's first chunk per layer: attention over the "
                "chunk (fp32 causal SDPA, the reference's precision), device fit, the decoder's "
                "registration (pseudo-inverse), K3 write")


def bench_config4(torch, lay, cfg, cache, dev, steps=10, warmup=3, cpu=False):
    """4 requests, 7400 cached tokens each plus a 256-query chunk whose keys
    are already written (n = 7656), causal over cached + chunk positions; one K2 launch per
    layer over the 4 chunks."""
    from vllm_ttkv import kernels, synth
    Q, n = 256, 7400 + 256
    lens = [n] * 4
    st = build_store(torch, lay, cfg, lens, 1, seed=4, dev=dev)
    L = st["layers"][0]
    q = synth.queries(4 * Q, seed=8, device=dev)
    qsl = torch.arange(0, 4 * Q + 1, Q, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    ws = kernels.prefill_workspace(lay, HQ, 4, Q, n, dev, BS)
    err = torch.zeros(1, dtype=torch.int32, device=dev)

    def attend():
        kernels.prefill_paged(lay, q, L["page"], BS, st["bt"], st["seq_lens"], qsl, Q, n,
                              st["dec_map"], L["dec_pool"], cache, D ** -0.5, out=out,
                              workspace=ws, error_word=err)

    ms = time_launches(torch, attend, steps, warmup)
    scores = torch.empty(HQ, Q, n, dtype=torch.float32, device=dev)
    from vllm_ttkv import _hip
    sws = torch.empty(max(1, _hip.lib().ttkv_multi_scores_workspace_bytes(_hip.Layout.of(lay), HQ,
                                                                           Q, n)),
                      dtype=torch.uint8, device=dev)

    def score1():
        kernels.multi_scores_paged(lay, q[:Q], L["page"], BS, st["bt"][:1], st["seq_lens"][:1],
                                   qsl[:2], Q, n, st["dec_map"], L["dec_pool"], cache,
                                   D ** -0.5, scores=scores, error_word=err, workspace=sws)

    ms_s = time_launches(torch, score1, steps, warmup)
    # a short chunk over the same store: 16 queries per request (the last 16 keys are the chunk's)
    Qs = 16
    qs = q[:4 * Qs].contiguous()
    qsl_s = torch.arange(0, 4 * Qs + 1, Qs, dtype=torch.int32, device=dev)
    outs = torch.empty_like(qs)
    ws_s = kernels.prefill_workspace(lay, HQ, 4, Qs, n, dev, BS)

    def attend_short():
        kernels.prefill_paged(lay, qs, L["page"], BS, st["bt"], st["seq_lens"], qsl_s, Qs, n,
                              st["dec_map"], L["dec_pool"], cache, D ** -0.5, out=outs,
                              workspace=ws_s, error_word=err)

    ms_q16 = time_launches(torch, attend_short, steps, warmup)
    torch.cuda.synchronize()
    if int(err.item()):
        raise RuntimeError(f"K2: device error word {int(err.item())}")
    fl = k2_flops(lens, [Q] * 4, lay.r1)
    tf = fl / (ms * 1e-3) / 1e12
    log(f"K2 config4: {ms * 1e3:.1f} us/launch (4 chunks), {tf:.1f} TFLOP/s; scores mode "
        f"{ms_s * 1e3:.1f} us per chunk; 16-query chunks {ms_q16 * 1e3:.1f} us/launch")
    res = dict(requests=4, cached=7400, chunk=Q, us_per_launch=ms * 1e3,
               us_per_chunk_layer=ms * 1e3 / 4, algorithmic_flop_per_launch=fl,
               tflops=tf, mfma_peak_tflops=2500.0, mfma_frac=tf / 2500.0,
               scores_mode_us_per_chunk_layer=ms_s * 1e3,
               scores_mode_gbps_written=HQ * Q * n * 4 / (ms_s * 1e-3) / 1e9,
               us_per_launch_16_query_chunks=ms_q16 * 1e3)
    if cpu:
        cms, cores = cpu_k2_sample(torch, lay, st, L, q[:Q], cache, n, Q)
        res["cpu_baseline"] = dict(value=cms, unit="ms per chunk-layer", cores=cores, kind="port",
                                   sample="one request's 256-query chunk over 7,656 keys through "
                                          "the torch-CPU oracle attend_multi")
        log(f"K2 config4 cpu baseline: {cms:.0f} ms per chunk-layer on {cores} threads")
    return res


def bench_dense(torch, lens, q, dev, steps=3, warmup=1, n_layers=L_LAYERS):
    """Dense fp16 paged attention of the same shapes (the per-cached-token comparison): this
    build's dense HIP comparator over a shuffled paged cache, one K/V cache per layer (28, so
    the cycled bytes far exceed the caches, as the compressed read's are), and torch SDPA over
    contiguous per-request K/V (no paging)."""
    from vllm_ttkv import kernels, synth
    B = len(lens)
    bt, nblk = synth.shuffled_block_table(lens, BS, seed=11, extra_blocks=2)
    g = torch.Generator(device=dev).manual_seed(12)
    kcs, vcs = [], []
    for _ in range(n_layers):
        kcs.append(torch.randn(nblk * BS, H, D, generator=g, device=dev).to(torch.float16))
        vcs.append(torch.randn(nblk * BS, H, D, generator=g, device=dev).to(torch.float16))
    bt_d = bt.to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    qsl = torch.arange(B + 1, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    n = kernels._hip.lib().ttkv_dense_workspace_bytes(H, HQ, B, max(lens), BS)
    ws = torch.zeros(max(int(n), 256), dtype=torch.uint8, device=dev)
    li = [0]

    def run():
        kernels.dense_decode_paged(q, kcs[li[0]], vcs[li[0]], BS, bt_d, sl, qsl, max(lens),
                                   D ** -0.5, out=out, workspace=ws)
        li[0] = (li[0] + 1) % n_layers

    ms = time_back_to_back(torch, run, steps * n_layers, warmup * n_layers)
    ms_ev = time_launches(torch, run, steps * n_layers, warmup * n_layers)
    del kcs, vcs
    gbps = sum(lens) * H * D * 2 * 2 / (ms * 1e-3) / 1e9
    res = dict(us_per_layer=ms * 1e3, hbm_gbps=gbps, hbm_frac=gbps / HBM_PEAK_GBPS,
               ns_per_cached_token=ms * 1e6 / sum(lens), layers_cycled=n_layers,
               us_per_layer_launch_events=ms_ev * 1e3)
    try:
        import torch.nn.functional as F
        kd = torch.randn(B, H, max(lens), D, generator=g, device=dev).to(torch.float16)
        vd = torch.randn(B, H, max(lens), D, generator=g, device=dev).to(torch.float16)
        q4 = q.reshape(B, HQ, 1, D)
        ms_s = time_launches(torch, lambda: F.scaled_dot_product_attention(
            q4, kd, vd, scale=D ** -0.5, enable_gqa=True), steps, warmup)
        res["torch_sdpa_contiguous_us_per_layer"] = ms_s * 1e3
        del kd, vd
    except Exception as e:  # noqa: BLE001 - report, do not fail the bench line
        res["torch_sdpa_contiguous_us_per_layer"] = f"unavailable: {type(e).__name__}"
    return res


def bench_container(torch, dev, B=8, n=14402, r1=R1, steps=10, warmup=3):
    """The container-layout reads (the codec's pooled container, not slots) at the headline shape:
    B sequences of n tokens, safe rows (81 lanes at 3 bits). The container is synthetic and
    structurally valid (every row has exactly k set lanes); timing does not depend on values."""
    from vllm_ttkv import container
    g = torch.Generator(device=dev).manual_seed(21)
    k, bits, pb = 81, 3, (81 * 3 + 7) // 8
    rows = B * H * n

    def synth_rows():
        bm = torch.empty(rows, 16, dtype=torch.uint8, device=dev)
        w = (2 ** torch.arange(7, -1, -1, device=dev)).to(torch.int32)
        for r0 in range(0, rows, 1 << 17):                       # bounded temporaries
            r1_ = min(rows, r0 + (1 << 17))
            idx = torch.rand(r1_ - r0, D, generator=g, device=dev).topk(k, dim=1).indices
            mask = torch.zeros(r1_ - r0, D, dtype=torch.int32, device=dev).scatter_(1, idx, 1)
            bm[r0:r1_] = (mask.view(-1, 16, 8) * w).sum(-1).to(torch.uint8)
        pk = torch.randint(0, 256, (rows, pb), generator=g, device=dev, dtype=torch.uint8)
        sc = torch.rand(rows, generator=g, device=dev) * 0.01
        return container.PackedRows(bm, pk, sc, bits)

    cq = torch.randint(-127, 128, (B * n, r1), generator=g, device=dev, dtype=torch.int8)
    cs = torch.rand(B * n, generator=g, device=dev) * 0.01
    dq = torch.randint(-127, 128, (B, r1, H * D), generator=g, device=dev, dtype=torch.int8)
    ds = torch.rand(B, r1, generator=g, device=dev) * 0.01
    kr, vr = synth_rows(), synth_rows()
    from vllm_ttkv import rope
    csc = rope.cos_sin_cache(n, D, device=dev)
    cos = torch.cat([csc[:, :D // 2]] * 2, -1).contiguous()
    sin = torch.cat([csc[:, D // 2:]] * 2, -1).contiguous()
    q = torch.randn(B, HQ, D, generator=g, device=dev)
    p = torch.softmax(torch.randn(B, HQ, n, generator=g, device=dev), -1)
    ms_k = time_launches(torch, lambda: container.krt(cq, cs, dq, ds, kr, cos, sin, q, n, HQ,
                                                      HQ // H, D), steps, warmup)
    ms_v = time_launches(torch, lambda: container.v_out(p, vr, n, HQ, HQ // H, D), steps, warmup)
    # algorithmic bytes: each array once (decoder as fp32 after the launcher's conversion)
    kb = (B * n * (r1 + 4) + rows * (16 + pb + 4) + B * r1 * H * D * 4 + 2 * n * D * 4
          + B * HQ * D * 4 + B * HQ * n * 4)
    vb = rows * (16 + pb + 4) + B * HQ * n * 4 + B * HQ * D * 4
    log(f"container krt B={B}x{n}: {ms_k * 1e3:.1f} us ({kb / (ms_k * 1e-3) / 1e9:.0f} GB/s); "
        f"v_out {ms_v * 1e3:.1f} us ({vb / (ms_v * 1e-3) / 1e9:.0f} GB/s)")
    return dict(B=B, n=n, r1=r1, krt_us=ms_k * 1e3, krt_bytes=kb,
                krt_gbps=kb / (ms_k * 1e-3) / 1e9, v_out_us=ms_v * 1e3, v_out_bytes=vb,
                v_out_gbps=vb / (ms_v * 1e-3) / 1e9)


def bench_config5(torch, cache, dev, steps=10, warmup=3, n_layers=L_LAYERS, cpu=False):
    """the reference's 4-bit store (`campaign4x`: 64 lanes of 4-bit codes for
    K residual and V, int8 coefficients, fp16 rulers), 8 requests at 16k context, 28 layers. Each
    step writes one new key/value per request per layer (K3: projection onto the decoder, bitmap
    select, quantise, pack, slot write) and then reads the layer (K1) -- both timed together."""
    from vllm_ttkv import kernels, synth
    from vllm_ttkv.layout import CONFIGS, layout_for_config
    cfg5 = CONFIGS["campaign4x"]
    lay5 = layout_for_config(cfg5, r1=R1)
    ctx, B, spare = 16384, 8, 16
    st = build_store(torch, lay5, cfg5, [ctx + spare] * B, n_layers, seed=6, dev=dev)
    bt_cpu = st["bt"].cpu()
    qsl_w = torch.arange(B + 1, dtype=torch.int32, device=dev)
    newk = [synth.keys(spare, seed=900 + r, device=dev).permute(1, 0, 2) for r in range(B)]
    newv = [synth.values(spare, seed=900 + r, device=dev).permute(1, 0, 2) for r in range(B)]
    q = synth.queries(B, seed=9, device=dev)
    out = torch.empty_like(q)
    ws = kernels.decode_workspace(lay5, HQ, B, ctx + spare, dev, BS)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    plans = []
    for j in range(spare):  # step j writes position ctx + j and reads ctx + j + 1 tokens
        pos = ctx + j
        slots = torch.tensor([int(bt_cpu[r, pos // BS]) * BS + pos % BS for r in range(B)],
                             dtype=torch.int64, device=dev)
        k_new = torch.stack([newk[r][j] for r in range(B)]).contiguous()
        v_new = torch.stack([newv[r][j] for r in range(B)]).contiguous()
        plans.append((slots, k_new, v_new, torch.full((B,), pos + 1, dtype=torch.int32,
                                                      device=dev)))
    wws = kernels.write_workspace(lay5, B, dev)

    def write(j, li):
        slots, k_new, v_new, _ = plans[j % spare]
        L = st["layers"][li]
        kernels.write_paged(lay5, k_new, v_new, slots, qsl_w, st["bt"], st["dec_map"],
                            L["dec_pool"], L["pinv_pool"], L["page"], error_word=err,
                            workspace=wws)

    def read(j, li):
        L = st["layers"][li]
        kernels.decode_paged(lay5, q, L["page"], BS, st["bt"], plans[j % spare][3], qsl_w,
                             ctx + spare, st["dec_map"], L["dec_pool"], cache, D ** -0.5, out=out,
                             workspace=ws, error_word=err)

    def step(j):
        for li in range(n_layers):
            write(j, li)
            read(j, li)

    def timed(fn, reps):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        for j in range(reps):
            fn(j)
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / reps

    for j in range(warmup):
        step(j)
    # the step time with the launches back to back (events only around the timed steps)
    ms_step = timed(lambda j: step(warmup + j), steps)
    # The K3 / K1 split from HIP graph replays of one step's 28 writes alone, its 28 reads alone
    # and both: no host work between launches (an event pair around each eager launch also times
    # the host's submission whenever the host, not the GPU, is behind). A write graph replays the
    # same token into the same slot, so its bytes do not change.
    graphs = {}
    for name, body in (("k3", lambda: [write(0, li) for li in range(n_layers)]),
                       ("k1", lambda: [read(0, li) for li in range(n_layers)]),
                       ("step", lambda: step(0))):
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            body()
        g.replay()
        graphs[name] = g
    ms_g = {name: timed(lambda j, g=g: g.replay(), steps) for name, g in graphs.items()}
    if int(err.item()):
        raise RuntimeError(f"config 5: device error word {int(err.item())}")
    k3, k1 = ms_g["k3"] / n_layers, ms_g["k1"] / n_layers
    nbytes = k1_bytes(lay5, [ctx + 1] * B, R1, ctx + 1)
    log(f"config5 campaign4x 8x16k: {ms_step * 1e3 / n_layers:.1f} us/layer back to back; graph "
        f"replays {ms_g['step'] * 1e3 / n_layers:.1f} (K3 {k3 * 1e3:.1f} + K1 {k1 * 1e3:.1f})")
    res = dict(allocation="campaign4x (4-bit residual/V codes, int8 coefficients)",
               requests=B, context=ctx, layers=n_layers, ms_per_step=ms_step,
               us_per_layer=ms_step * 1e3 / n_layers,
               us_per_layer_graph=ms_g["step"] * 1e3 / n_layers, k3_us_per_launch=k3 * 1e3,
               k1_us_per_launch=k1 * 1e3, tokens_per_s=B / (ms_step * 1e-3),
               k1_hbm_gbps=nbytes / (k1 * 1e-3) / 1e9)
    if cpu:
        L = st["layers"][0]
        slots, k_new, v_new, _ = plans[0]
        cms, cores = cpu_k3_sample(torch, lay5, k_new, v_new, L["dec_f"], L["pinv_pool"])
        res["k3_cpu_baseline"] = dict(value=cms, unit="ms per 8-token write", cores=cores,
                                      kind="port",
                                      sample="one step-layer's 8 new tokens through the "
                                             "torch-CPU oracle encode_frozen + row packing")
        log(f"config5 K3 cpu baseline: {cms:.1f} ms per 8-token write on {cores} threads")
    return res


def cpu_baseline(torch, lay, store, q, cache, n, budget_s=12.0):
    """The torch-CPU oracle (reference.py:149-163 restated, float32, the reference's request
    loop) on a bounded sample: request-layers of the headline workload, timed until `budget_s`."""
    sys.path.insert(0, str(ROOT))
    from oracle import attend, rope as orope
    from oracle.layout import Layout
    lay = Layout(lay.H, lay.d, lay.r1, lay.qbits, lay.res_k, lay.res_bits, lay.v_lanes, lay.v_bits)
    torch.set_num_threads(os.cpu_count() or 1)
    cores = torch.get_num_threads()
    bt = store["bt"].cpu()
    cos, sin = orope.cos_sin_from_cache(cache.cpu(), torch.arange(n), D)
    done, t_tot = 0, 0.0
    r, li = 0, 0
    while t_tot < budget_s and done < 64:
        L = store["layers"][li % len(store["layers"])]
        p = torch.arange(n, device=bt.device)
        slots = (bt[r, p // BS].long() * BS + p % BS)
        blob = L["page"][slots.to(L["page"].device)].cpu()
        dec = L["dec_f"][r].cpu()
        k_s, v_s = blob[:, :lay.k_slot_bytes].contiguous(), blob[:, lay.k_slot_bytes:].contiguous()
        qq = q[r].float().cpu()
        t0 = time.perf_counter()
        attend.attend_raw_store(lay, k_s, v_s, dec, qq, cos, sin, D ** -0.5)
        t_tot += time.perf_counter() - t0
        done += 1
        r = (r + 1) % store["B"]
        li += 1
    per_req_layer = t_tot / done
    step_s = per_req_layer * store["B"] * L_LAYERS
    return dict(value=store["B"] / step_s, unit="tokens/s", cores=cores, kind="port",
                sample=f"{done} request-layers of the headline workload (n={n}) through the "
                       f"torch-CPU oracle attend_raw_store, {t_tot:.1f} s; extrapolated x"
                       f"{store['B']} requests x {L_LAYERS} layers per step",
                ms_per_request_layer=per_req_layer * 1e3)


def read_traffic(path):
    """HBM bytes per K1 launch from a committed rocprofv3 --pmc summary, if one exists."""
    p = ROOT / "profiles" / path
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1].split()[0])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=L_LAYERS)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--config5-only", action="store_true",
                    help="only the 4-bit read+write workload (BASELINE config 5); prints its line")
    ap.add_argument("--config4-only", action="store_true",
                    help="only the continuation workload (BASELINE config 4, K2); prints its line")
    ap.add_argument("--container-only", action="store_true",
                    help="only the container-layout reads (krt + v_out at 8 x 14402); prints its line")
    ap.add_argument("--batch1-only", action="store_true",
                    help="only the batch-1 sweep (cold, 1082 / 4322 / 8642 / 14402 tokens)")
    ap.add_argument("--coef-modes-only", action="store_true",
                    help="only K1 over the fp16 / 4-bit coefficient-mode stores")
    ap.add_argument("--first-chunk-only", action="store_true",
                    help="only the first-chunk timings (attention, fit, write at 2048 / 8192)")
    ap.add_argument("--dense-only", action="store_true",
                    help="only the dense fp16 paged comparator (headline and config 3 shapes)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 1 GiB device copy (HBM-counter calibration for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} "
              f"requested). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    from vllm_ttkv import rope, synth
    from vllm_ttkv.layout import CONFIGS, layout_for_config
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    cfg = CONFIGS["safe"]
    lay = layout_for_config(cfg, r1=R1)
    cache = rope.cos_sin_cache(32768, D, device=dev)
    extra = {}

    if args.calib_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 1073741824 bytes read + written")
        del src, dst

    if args.config4_only:
        c4 = bench_config4(torch, lay, cfg, cache, dev, args.steps, args.warmup)
        print(json.dumps(dict(metric="continuation chunk us/layer (K2, BASELINE config 4)",
                              value=c4["us_per_chunk_layer"], unit="us", n_gpus=1,
                              higher_is_better=False,
                              dtype="f16 MFMA on exact hi+lo key splits (V readout: P*ruler_v "
                                    "rounded to fp16 once), fp32 accumulate",
                              data="synthetic", **c4)))
        return

    if args.container_only:
        cr = bench_container(torch, dev, steps=args.steps, warmup=args.warmup)
        print(json.dumps(dict(metric="container-layout reads us/launch (krt + v_out, 8 x 14402)",
                              value=cr["krt_us"] + cr["v_out_us"], unit="us", n_gpus=1,
                              higher_is_better=False,
                              dtype="fp32 in/out; fp16 MFMA on exact hi+lo splits, fp32 accumulate",
                              data="synthetic", **cr)))
        return

    if args.first_chunk_only:
        fc = bench_first_chunk(torch, lay, cfg, dev)
        print(json.dumps(dict(metric="first chunk us/layer (attention + fit + write)",
                              value=fc["per_layer"][-1]["total_us"], unit="us", n_gpus=1,
                              higher_is_better=False, data="synthetic", **fc)))
        return

    if args.dense_only:
        qd = synth.queries(8, seed=5, device=dev)
        dh = bench_dense(torch, [14402] * 8, qd, dev, args.steps, args.warmup)
        d3 = bench_dense(torch, config3_lens(), qd, dev, args.steps, args.warmup)
        print(json.dumps(dict(metric="dense fp16 paged decode us/layer (comparator)",
                              value=dh["us_per_layer"], unit="us", n_gpus=1,
                              higher_is_better=False, dtype="fp16 in/out, fp32 accumulate",
                              data="synthetic", headline=dh, config3=d3)))
        return

    if args.batch1_only:
        sw = batch1_sweep(torch, lay, cfg, cache, dev, cache_flusher(torch, dev))
        print(json.dumps(dict(metric="K1 us/layer at batch 1 (cold, per context)",
                              value=sw[0]["us_per_layer"], unit="us", n_gpus=1,
                              higher_is_better=False, data="synthetic", sweep=sw)))
        return

    if args.coef_modes_only:
        cm = bench_coef_modes(torch, cache, dev, args.steps, args.warmup)
        print(json.dumps(dict(metric="K1 us/layer at 8 x 14402, fp16 and 4-bit coefficient modes",
                              value=cm["safe_fp16"]["us_per_layer"], unit="us", n_gpus=1,
                              higher_is_better=False, data="synthetic", modes=cm)))
        return

    if args.config5_only:
        c5 = bench_config5(torch, cache, dev, args.steps, args.warmup)
        print(json.dumps(dict(metric="4-bit decode step us/layer, K3 write + K1 read (BASELINE "
                                     "config 5)", value=c5["us_per_layer"], unit="us",
                              n_gpus=1, higher_is_better=False,
                              dtype="fp16 in/out; fp16 MFMA on exact hi+lo splits (V "
                                    "readout: P*ruler_v rounded to fp16 once), fp32 "
                                    "accumulate and softmax",
                              data="synthetic", **c5)))
        return

    # ---------------------------------------------------------------- headline: B=8 @ 14402
    lens = [14402] * 8
    t0 = time.perf_counter()
    store = build_store(torch, lay, cfg, lens, args.layers, seed=1, dev=dev)
    log(f"build B=8x14402: {time.perf_counter() - t0:.1f}s (fit {store['t_fit']:.1f}s, "
        f"write {store['t_write']:.1f}s)")
    q = synth.queries(8, seed=5, device=dev)
    # the timed region: K steps back to back, events only around it; then the same steps with an
    # event pair around every launch, for the per-launch figure alone
    ms_step, ms_launch = time_k1(torch, lay, store, q, cache, args.steps, args.warmup,
                                 args.layers, per_launch=False)
    _, ms_launch_ev = time_k1(torch, lay, store, q, cache, args.steps, 1, args.layers)
    nbytes = k1_bytes(lay, lens, R1, max(lens))
    achieved = nbytes / (ms_launch * 1e-3) / 1e9
    step_ms = ms_step * L_LAYERS / args.layers
    log(f"K1 B=8x14402: {ms_launch * 1e3:.1f} us/launch back to back ({ms_launch_ev * 1e3:.1f} "
        f"with an event pair per launch), {achieved:.0f} GB/s")

    if not args.no_extra:
        # Cold-HBM extras: 28 layers of distinct pages each, and the caches flushed between
        # launches (a batch-1 layer of 1-13 MB would otherwise stay in the 256 MB Infinity Cache
        # across a 28-layer cycle; in serving, the model's weights pass between two reads of a
        # layer's cache)
        flush = cache_flusher(torch, dev)
        extra["batch1_sweep"] = batch1_sweep(torch, lay, cfg, cache, dev, flush)
        lens3 = config3_lens()
        st = build_store(torch, lay, cfg, lens3, L_LAYERS, seed=3, dev=dev)
        # 28 layers of ~42 MB each cycle far past the 256 MB Infinity Cache: timed back to back
        # like the headline (and the dense comparator below); the flushed per-launch figure too
        _, ml = time_k1(torch, lay, st, q, cache, 10, 3, L_LAYERS, per_launch=False)
        _, mlf = time_k1(torch, lay, st, q, cache, 3, 1, L_LAYERS, flush=flush)
        b = k1_bytes(lay, lens3, R1, max(lens3))
        log(f"K1 config3 ({sum(lens3)} tokens, longest {max(lens3)}): {ml * 1e3:.1f} us/layer "
            f"back to back ({mlf * 1e3:.1f} flushed, event pair per launch)")
        extra["config3_b8_random"] = dict(contexts=lens3, us_per_layer=ml * 1e3,
                                          hbm_gbps=b / (ml * 1e-3) / 1e9,
                                          tokens_per_s=8 / (ml * 1e-3 * L_LAYERS), cold_hbm=True,
                                          layers_cycled=L_LAYERS,
                                          us_per_layer_flushed_event_pairs=mlf * 1e3)
        del st
        dn = bench_dense(torch, lens3, q, dev)
        dn["compressed_ns_per_cached_token"] = ml * 1e6 / sum(lens3)
        extra["config3_dense_fp16_comparator"] = dn
        log(f"dense fp16 comparator (config 3 shapes): {dn['us_per_layer']:.1f} us/layer, "
            f"{dn['hbm_gbps']:.0f} GB/s ({100 * dn['hbm_frac']:.0f} % of HBM peak)")
        dh = bench_dense(torch, lens, q, dev)
        dh["compressed_ns_per_cached_token"] = ms_launch * 1e6 / sum(lens)
        extra["headline_dense_fp16_comparator"] = dh
        log(f"dense fp16 comparator (8x14402): {dh['us_per_layer']:.1f} us/layer, "
            f"{dh['hbm_gbps']:.0f} GB/s ({100 * dh['hbm_frac']:.0f} % of HBM peak)")
        extra["config4_continuation"] = bench_config4(torch, lay, cfg, cache, dev,
                                                      cpu=not args.no_cpu)
        extra["config5_4bit_read_write"] = bench_config5(torch, cache, dev, cpu=not args.no_cpu)
        extra["container_reads_b8_ctx14402"] = bench_container(torch, dev)
        extra["first_chunk"] = bench_first_chunk(torch, lay, cfg, dev)
        extra["coefficient_modes_b8_ctx14402"] = bench_coef_modes(torch, cache, dev)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, lay, store, q, cache, lens[0])
        log(f"cpu baseline: {cpu['ms_per_request_layer']:.0f} ms per request-layer on "
            f"{cpu['cores']} threads")

    line = {
        "metric": "decode step us/layer vs context at batch 1 & 8; achieved HBM GB/s; tokens/s",
        "value": 8 / (step_ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 in/out; fp16 MFMA: reconstruction and scores on exact hi+lo splits, V "
                 "readout on exact codes against P*ruler_v rounded to fp16 once (power-of-two "
                 "scaled below 2^15); fp32 accumulate and softmax",
        "data": "synthetic (seeded low-rank keys with outlier channels, N(0,1) values, fp16 "
                "queries; stores fitted and packed on the GPU by this package; 4 distinct layer "
                "stores, each copied into its own pages for the other 24 layers)",
        "config": {"workload": "llama-3.2-3b attention decode read, batch 8 x 14402 cached tokens, "
                               "28 layers, safe r1=110, block 16, one K1 launch per layer",
                   "global_batch": 8, "seq_len": 14402, "layers": L_LAYERS,
                   "layers_timed": args.layers, "parallelism": "single GPU"},
        "us_per_layer": ms_launch * 1e3,
        "us_per_launch_event_pairs": ms_launch_ev * 1e3,
        "hbm_gbps": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS,
                     "traffic": read_traffic("k1_decode_b8_ctx14402_pmc.txt"),
                     "algorithmic_bytes_per_launch": nbytes},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
