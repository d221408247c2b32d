"""The drop-in `TTKVAttentionImpl.forward` on the GPU: first-chunk fit + write, decode steps and a
mixed decode / continuation / first-chunk step, each checked against the CPU oracle reading the
cache bytes the step wrote (reference test: test_impl_decode.py:259-873 -- real forward vs
attend_raw_store, write->decode loop, continuation over the whole store, mixed batch)."""
from dataclasses import dataclass
from types import SimpleNamespace

import pytest
import torch

from helpers import HQ, H, D
from oracle import attend
from oracle.layout import layout_for_config as oracle_layout
from oracle.rope import cos_sin_from_cache, rope_apply
from vllm_ttkv import impl as impl_mod
from vllm_ttkv import patch, rope_store, synth
from vllm_ttkv.impl import TTKVAttentionImpl
from vllm_ttkv.layout import CONFIGS, config_named, layout_for_config
from vllm_ttkv.metadata import TTKVAttentionMetadata, TTKVAttentionMetadataBuilder
from vllm_ttkv.rope import cos_sin_cache

pytestmark = pytest.mark.gpu
SCALE = D ** -0.5
BS = 16
NAME = "model.layers.5.self_attn.attn"


@dataclass
class _Layer:
    layer_name: str
    ttkv_layout: object


class _Seq:
    """One request's raw K/V/q streams (positions 0..T-1)."""

    def __init__(self, T, seed, kvh=H, hq=HQ):
        self.K = synth.keys(T, H=kvh, seed=seed).permute(1, 0, 2).contiguous()   # [T, H, d]
        self.V = synth.values(T, H=kvh, seed=seed).permute(1, 0, 2).contiguous()
        self.Q = synth.queries(T, HQ=hq, seed=seed).float()                      # [T, HQ, d]


def _step(im, layer, cache, csc, bt, reqs):
    """reqs: list of (seq, start, end) -> positions [start, end) of each request this step."""
    qsl, rows_k, rows_v, rows_q, slots, seq_lens = [0], [], [], [], [], []
    for r, (sq, s, e) in enumerate(reqs):
        qsl.append(qsl[-1] + e - s)
        rows_k.append(sq.K[s:e])
        rows_v.append(sq.V[s:e])
        rows_q.append(sq.Q[s:e])
        pos = torch.arange(s, e)
        slots.append(bt[r, pos // BS].long() * BS + pos % BS)
        seq_lens.append(e)
    raw_k = torch.cat(rows_k)
    positions = torch.cat([torch.arange(s, e) for _, s, e in reqs])
    cos, sin = cos_sin_from_cache(csc, positions, D)
    k_post = rope_apply(raw_k, cos.unsqueeze(1), sin.unsqueeze(1)).to(torch.float16)
    N = qsl[-1]
    dev = "cuda"
    md = TTKVAttentionMetadata(
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32, device=dev),
        slot_mapping=torch.cat(slots).to(dev),
        block_table=bt[:len(reqs)].to(dev),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=dev),
        query_start_loc_cpu=torch.tensor(qsl, dtype=torch.int32), num_actual_tokens=N,
        max_query_len=max(e - s for _, s, e in reqs), max_seq_len=max(seq_lens))
    q = torch.cat(rows_q).to(torch.float16)
    kvh, hq = raw_k.shape[1], q.shape[1]
    patch.stash_raw_k(NAME, raw_k.reshape(N, kvh * D).to(dev), cos_sin_cache=csc.to(dev))
    out = torch.full((N, hq, D), float("nan"), dtype=torch.float16, device=dev)
    im.forward(layer, q.to(dev), k_post.reshape(N, kvh * D).to(dev),
               torch.cat(rows_v).reshape(N, kvh * D).to(torch.float16).to(dev), cache, md,
               output=out)
    torch.cuda.synchronize()
    assert int(im.error_word.item()) == 0
    return out.float().cpu(), q, k_post, qsl, seq_lens


def _check(got, want, what, max_abs=2e-3, mean_abs=1e-3):
    e = (got.double() - want.double()).abs()
    print(f"{what}: max-abs {e.max():.3e} mean-abs {e.mean():.3e}")
    assert torch.isfinite(got).all(), what
    assert e.max() <= max_abs and e.mean() <= mean_abs, f"{what}: {e.max():.3e} / {e.mean():.3e}"


def _sdpa_ref(q, k_post, v):
    """fp64 causal attention over the chunk's own (fp16) post-RoPE keys and values."""
    q, k_post, v = q.double(), k_post.double(), v.half().double()
    G = q.shape[1] // k_post.shape[1]
    T = q.shape[0]
    kk = k_post.repeat_interleave(G, dim=1).transpose(0, 1)
    vv = v.repeat_interleave(G, dim=1).transpose(0, 1)
    s = torch.einsum("htd,hsd->hts", q.transpose(0, 1), kk) * SCALE
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    return torch.einsum("hts,hsd->htd", torch.softmax(s, -1), vv).transpose(0, 1)


@pytest.mark.parametrize("kvh,hq", [(4, 12), (2, 8)])
def test_forward_with_fewer_kv_heads(kvh, hq):
    """The drop-in at 4 and 2 KV heads (3 and 4 query heads each): a first chunk (fit, write,
    SDPA), then decode steps against the oracle reading the bytes they wrote."""
    lay = layout_for_config(CONFIGS["safe"], 110, H=kvh)
    olay = oracle_layout(CONFIGS["safe"], 110, H=kvh)
    rope_store.clear_stores()
    csc = cos_sin_cache(2048)
    seqs = [_Seq(600, 11, kvh, hq), _Seq(500, 12, kvh, hq)]
    bt, nblk = synth.shuffled_block_table([600, 500], BS, seed=4, extra_blocks=2)
    C = lay.compressed_bytes_per_token()
    cache = torch.zeros(nblk, 1, BS, C // 2, dtype=torch.bfloat16, device="cuda")
    im = TTKVAttentionImpl(hq, D, SCALE, kvh)
    layer = _Layer(NAME, lay)
    out, q, k_post, qsl, _ = _step(im, layer, cache, csc, bt, [(seqs[0], 0, 400),
                                                                (seqs[1], 0, 300)])
    for r, (s, e) in enumerate([(0, 400), (0, 300)]):
        want = _sdpa_ref(q[qsl[r]:qsl[r + 1]], k_post[qsl[r]:qsl[r + 1]], seqs[r].V[s:e])
        _check(out[qsl[r]:qsl[r + 1]], want, f"H={kvh} first chunk {r}")
    for t in range(2):
        reqs = [(seqs[0], 400 + t, 401 + t), (seqs[1], 300 + t, 301 + t)]
        out, q, _, qsl, seq_lens = _step(im, layer, cache, csc, bt, reqs)
        flat = cache.view(torch.uint8).reshape(-1, C).cpu()
        store = rope_store.store_for_layer(NAME)
        decs = [store.decoders[int(bt[r, 0])].decoder_f.cpu() for r in range(2)]
        want = attend.paged_decode(olay, flat, bt[:2], torch.tensor(seq_lens), torch.tensor(qsl),
                                   q.float(), decs, csc, BS, SCALE, dtype=torch.float64)
        _check(out, want, f"H={kvh} decode step {t}")
    rope_store.clear_stores()


@pytest.mark.parametrize("alloc", ["safe", "safe_fp16", "campaign4x_int4g32"])
def test_forward_write_then_read_loop_and_mixed_batch(alloc, monkeypatch):
    """Also in this library's fp16 and 4-bit coefficient modes (selected like an allocation,
    by VLLM_TTKV_CONFIG), whose first chunks are written by projection onto the new decoder."""
    monkeypatch.setenv("VLLM_TTKV_CONFIG", alloc)
    lay = layout_for_config(config_named(alloc), 110)
    olay = oracle_layout(config_named(alloc), 110)
    rope_store.clear_stores()
    csc = cos_sin_cache(4096)
    seqs = [_Seq(1100, 1), _Seq(1000, 2), _Seq(400, 3)]
    bt, nblk = synth.shuffled_block_table([1100, 1000, 400], BS, seed=9, extra_blocks=2)
    C = lay.compressed_bytes_per_token()
    cache = torch.zeros(nblk, 1, BS, C // 2, dtype=torch.bfloat16, device="cuda")
    im = TTKVAttentionImpl(HQ, D, SCALE, H)
    layer = _Layer(NAME, lay)

    def oracle_inputs():
        flat = cache.view(torch.uint8).reshape(-1, C).cpu()
        store = rope_store.store_for_layer(NAME)
        decs = [store.decoders[int(bt[r, 0])].decoder_f.cpu() for r in range(len(store.decoders))]
        return flat, decs

    # step 1: two first chunks (fit + write; SDPA over the chunk's own q/k/v)
    out, q, k_post, qsl, _ = _step(im, layer, cache, csc, bt, [(seqs[0], 0, 700),
                                                                (seqs[1], 0, 500)])
    for r, (s, e) in enumerate([(0, 700), (0, 500)]):
        want = _sdpa_ref(q[qsl[r]:qsl[r + 1]], k_post[qsl[r]:qsl[r + 1]], seqs[r].V[s:e])
        _check(out[qsl[r]:qsl[r + 1]], want, f"first chunk {r}")
    assert len(rope_store.store_for_layer(NAME).decoders) == 2

    # steps 2-3: decode-only steps (K3 frozen write, then one K1 launch)
    for t in range(2):
        reqs = [(seqs[0], 700 + t, 701 + t), (seqs[1], 500 + t, 501 + t)]
        out, q, _, qsl, seq_lens = _step(im, layer, cache, csc, bt, reqs)
        flat, decs = oracle_inputs()
        want = attend.paged_decode(olay, flat, bt[:2], torch.tensor(seq_lens), torch.tensor(qsl),
                                   q.float(), decs, csc, BS, SCALE, dtype=torch.float64)
        _check(out, want, f"decode step {t}")

    # step 4: mixed -- a decode, a continuation chunk of 99, a new request's first chunk
    reqs = [(seqs[0], 702, 703), (seqs[1], 502, 601), (seqs[2], 0, 300)]
    out, q, k_post, qsl, seq_lens = _step(im, layer, cache, csc, bt, reqs)
    flat, decs = oracle_inputs()
    sl = torch.tensor(seq_lens)
    want_d = attend.paged_decode(olay, flat, bt[:1], sl[:1], torch.tensor(qsl[:2]), q.float(),
                                 decs[:1], csc, BS, SCALE, dtype=torch.float64)
    _check(out[0:1], want_d, "mixed: decode row")
    want_c = attend.paged_continuation(olay, flat, bt[:3], sl, torch.tensor(qsl), q.double(),
                                       decs, csc, BS, SCALE, rows=[1], dtype=torch.float64)
    _check(out[qsl[1]:qsl[2]], want_c[1], "mixed: continuation rows")
    want_f = _sdpa_ref(q[qsl[2]:qsl[3]], k_post[qsl[2]:qsl[3]], seqs[2].V[0:300])
    _check(out[qsl[2]:qsl[3]], want_f, "mixed: first chunk rows")
    rope_store.clear_stores()


def test_decode_steps_replayed_from_one_captured_graph(monkeypatch):
    """A decode-only `forward` (K3 write, then one K1 launch) captured once in a HIP graph and
    replayed for three steps, the inputs updated in place between replays (next token's q/k/v,
    slot ids, lengths). Each replay matches the oracle over the cache bytes it wrote: the step
    makes no host read-back and allocates nothing, and K1's work plan follows the new lengths on
    the device. The graph is sized with max_seq_len above every length it will see."""
    monkeypatch.delenv("VLLM_TTKV_CHECK", raising=False)
    lay = layout_for_config(CONFIGS["safe"], 110)
    olay = oracle_layout(CONFIGS["safe"], 110)
    rope_store.clear_stores()
    csc = cos_sin_cache(2048)
    csc_d = csc.cuda()
    seqs = [_Seq(900, 21), _Seq(600, 22)]
    bt, nblk = synth.shuffled_block_table([900, 600], BS, seed=23, extra_blocks=2)
    C = lay.compressed_bytes_per_token()
    cache = torch.zeros(nblk, 1, BS, C // 2, dtype=torch.bfloat16, device="cuda")
    im = TTKVAttentionImpl(HQ, D, SCALE, H)
    layer = _Layer(NAME, lay)
    _step(im, layer, cache, csc, bt, [(seqs[0], 0, 700), (seqs[1], 0, 400)])   # first chunks

    dev = "cuda"
    sq = torch.zeros(2, HQ, D, dtype=torch.float16, device=dev)
    sk = torch.zeros(2, H * D, dtype=torch.float16, device=dev)
    sv = torch.zeros(2, H * D, dtype=torch.float16, device=dev)
    sraw = torch.zeros(2, H * D, dtype=torch.float32, device=dev)
    out = torch.zeros(2, HQ, D, dtype=torch.float16, device=dev)
    md = TTKVAttentionMetadata(
        seq_lens=torch.zeros(2, dtype=torch.int32, device=dev),
        slot_mapping=torch.zeros(2, dtype=torch.int64, device=dev),
        block_table=bt[:2].to(dev), query_start_loc=torch.tensor([0, 1, 2], dtype=torch.int32,
                                                                   device=dev),
        query_start_loc_cpu=torch.tensor([0, 1, 2], dtype=torch.int32), num_actual_tokens=2,
        max_query_len=1, max_seq_len=900)

    def fill(t):
        pos = [700 + t, 400 + t]
        raw = torch.stack([seqs[r].K[p] for r, p in enumerate(pos)])            # [2, H, d]
        c, s = cos_sin_from_cache(csc, torch.tensor(pos), D)
        kp = rope_apply(raw, c.unsqueeze(1), s.unsqueeze(1))
        sq.copy_(torch.stack([seqs[r].Q[p] for r, p in enumerate(pos)]).to(torch.float16))
        sk.copy_(kp.reshape(2, H * D).to(torch.float16))
        sv.copy_(torch.stack([seqs[r].V[p] for r, p in enumerate(pos)]).reshape(2, H * D)
                 .to(torch.float16))
        sraw.copy_(raw.reshape(2, H * D))
        md.seq_lens.copy_(torch.tensor([p + 1 for p in pos], dtype=torch.int32))
        md.slot_mapping.copy_(torch.stack([bt[r, p // BS].long() * BS + p % BS
                                           for r, p in enumerate(pos)]))
        return pos

    # eager warm-up with the same static tensors (step 0), then capture
    fill(0)
    patch.stash_raw_k(NAME, sraw, cos_sin_cache=csc_d)
    im.forward(layer, sq, sk, sv, cache, md, output=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    patch.stash_raw_k(NAME, sraw, cos_sin_cache=csc_d)
    with torch.cuda.graph(graph):
        im.forward(layer, sq, sk, sv, cache, md, output=out)
    for t in range(3):
        pos = fill(t)
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert int(im.error_word.item()) == 0
        flat = cache.view(torch.uint8).reshape(-1, C).cpu()
        st = rope_store.store_for_layer(NAME)
        decs = [st.decoders[int(bt[r, 0])].decoder_f.cpu() for r in range(2)]
        want = attend.paged_decode(olay, flat, bt[:2], torch.tensor([p + 1 for p in pos]),
                                   torch.tensor([0, 1, 2]), sq.float().cpu(), decs, csc, BS,
                                   SCALE, dtype=torch.float64)
        _check(out.float().cpu(), want, f"graph replay {t}")
    rope_store.clear_stores()
    impl_mod.release_workspaces()


class _DecodeBatch:
    """A decode batch over rows `rows` of the block table, with static input buffers (as vLLM's
    runner keeps them for a captured graph) and metadata from the builder's capture path."""

    def __init__(self, rows, bt, builder, csc_d, dev="cuda"):
        n = len(rows)
        self.rows, self.bt, self.csc_d = rows, bt, csc_d
        self.q = torch.zeros(n, HQ, D, dtype=torch.float16, device=dev)
        self.k = torch.zeros(n, H * D, dtype=torch.float16, device=dev)
        self.v = torch.zeros(n, H * D, dtype=torch.float16, device=dev)
        self.raw = torch.zeros(n, H * D, dtype=torch.float32, device=dev)
        self.out = torch.zeros(n, HQ, D, dtype=torch.float16, device=dev)
        qsl = torch.arange(n + 1, dtype=torch.int32)
        cam = SimpleNamespace(
            seq_lens=torch.ones(n, dtype=torch.int32, device=dev),
            slot_mapping=torch.zeros(n, dtype=torch.int64, device=dev),
            block_table_tensor=bt[rows].to(torch.int32).to(dev), query_start_loc=qsl.to(dev),
            query_start_loc_cpu=qsl, num_actual_tokens=n, max_query_len=1, max_seq_len=1)
        self.md = builder.build_for_cudagraph_capture(cam)

    def fill(self, seqs, pos, csc):
        """Next token of each row's request at positions `pos` (one per row)."""
        raw = torch.stack([seqs[r].K[p] for r, p in zip(self.rows, pos)])      # [n, H, d]
        c, s_ = cos_sin_from_cache(csc, torch.tensor(pos), D)
        kp = rope_apply(raw, c.unsqueeze(1), s_.unsqueeze(1))
        n = len(self.rows)
        self.q.copy_(torch.stack([seqs[r].Q[p] for r, p in zip(self.rows, pos)]).half())
        self.k.copy_(kp.reshape(n, H * D).half())
        self.v.copy_(torch.stack([seqs[r].V[p] for r, p in zip(self.rows, pos)])
                     .reshape(n, H * D).half())
        self.raw.copy_(raw.reshape(n, H * D))
        self.md.seq_lens.copy_(torch.tensor([p + 1 for p in pos], dtype=torch.int32))
        self.md.slot_mapping.copy_(torch.stack([self.bt[r, p // BS].long() * BS + p % BS
                                                for r, p in zip(self.rows, pos)]))

    def stash(self):
        patch.stash_raw_k(NAME, self.raw, cos_sin_cache=self.csc_d)


def _oracle_decode(olay, cache, C, bt, rows, pos, q, csc):
    flat = cache.view(torch.uint8).reshape(-1, C).cpu()
    st = rope_store.store_for_layer(NAME)
    decs = [st.decoders[int(bt[r, 0])].decoder_f.cpu() for r in rows]
    n = len(rows)
    return attend.paged_decode(olay, flat, bt[rows], torch.tensor([p + 1 for p in pos]),
                               torch.arange(n + 1), q.float().cpu(), decs, csc, BS, SCALE,
                               dtype=torch.float64)


def test_graphs_at_two_batch_sizes_then_a_larger_eager_batch(monkeypatch):
    """vLLM's capture pattern for uniform decode: graphs captured at two batch sizes (2 and 4
    requests) from the builder's capture metadata (`max_seq_len` = the model's maximum), then a
    LARGER batch (all 6 requests) run eagerly, then both graphs replayed twice more. Every step is
    checked against the oracle over the cache bytes it wrote, and the decode-step workspaces are
    the same buffers before and after the larger batch (nothing a graph holds was replaced). The
    first chunks arrive in one prefill step whose fit decisions come from
    `num_computed_tokens_cpu` (no read of `seq_lens`)."""
    monkeypatch.delenv("VLLM_TTKV_CHECK", raising=False)
    monkeypatch.setenv("VLLM_TTKV_MAX_NUM_SEQS", "8")
    monkeypatch.setenv("VLLM_TTKV_MAX_MODEL_LEN", "2048")
    impl_mod.release_workspaces()
    lay = layout_for_config(CONFIGS["safe"], 110)
    olay = oracle_layout(CONFIGS["safe"], 110)
    rope_store.clear_stores()
    csc = cos_sin_cache(2048)
    csc_d = csc.cuda()
    lens = [700, 400, 900, 300, 520, 610]
    seqs = [_Seq(L + 8, 40 + i) for i, L in enumerate(lens)]
    bt0, nblk = synth.shuffled_block_table([L + 8 for L in lens], BS, seed=41, extra_blocks=2)
    # as vLLM's: ceil(max_model_len / block_size) columns, unused entries padded (-1 here, so a
    # read past a request's length would set the device error bit)
    bt = torch.full((6, 2048 // BS), -1, dtype=torch.int32)
    bt[:, :bt0.shape[1]] = bt0
    C = lay.compressed_bytes_per_token()
    cache = torch.zeros(nblk, 1, BS, C // 2, dtype=torch.bfloat16, device="cuda")
    im = TTKVAttentionImpl(HQ, D, SCALE, H)
    layer = _Layer(NAME, lay)
    builder = TTKVAttentionMetadataBuilder()
    assert builder.max_model_len == 2048

    # one prefill step: all six first chunks, planned from host metadata
    dev = "cuda"
    qsl = [0]
    for L in lens:
        qsl.append(qsl[-1] + L)
    N = qsl[-1]
    raw_k = torch.cat([sq.K[:L] for sq, L in zip(seqs, lens)])
    pos = torch.cat([torch.arange(L) for L in lens])
    c, s_ = cos_sin_from_cache(csc, pos, D)
    k_post = rope_apply(raw_k, c.unsqueeze(1), s_.unsqueeze(1)).half()
    slots = torch.cat([bt[r, torch.arange(L) // BS].long() * BS + torch.arange(L) % BS
                       for r, L in enumerate(lens)])
    md = TTKVAttentionMetadata(
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=dev), slot_mapping=slots.to(dev),
        block_table=bt[:6].to(dev), query_start_loc=torch.tensor(qsl, dtype=torch.int32,
                                                                 device=dev),
        query_start_loc_cpu=torch.tensor(qsl, dtype=torch.int32), num_actual_tokens=N,
        num_computed_tokens_cpu=torch.zeros(6, dtype=torch.int32),
        max_query_len=max(lens), max_seq_len=max(lens))
    patch.stash_raw_k(NAME, raw_k.reshape(N, H * D).to(dev), cos_sin_cache=csc_d)
    out = torch.zeros(N, HQ, D, dtype=torch.float16, device=dev)
    im.forward(layer, torch.cat([sq.Q[:L] for sq, L in zip(seqs, lens)]).half().to(dev),
               k_post.reshape(N, H * D).to(dev),
               torch.cat([sq.V[:L] for sq, L in zip(seqs, lens)]).reshape(N, H * D).half()
               .to(dev), cache, md, output=out)
    torch.cuda.synchronize()
    assert int(im.error_word.item()) == 0
    assert len(rope_store.store_for_layer(NAME).decoders) == 6
    nxt = list(lens)                       # next position of each request

    batches = {"A": _DecodeBatch([0, 1], bt, builder, csc_d),
               "B": _DecodeBatch([2, 3, 4, 5], bt, builder, csc_d)}
    assert batches["A"].md.max_seq_len == 2048
    graphs = {}
    for name, b in batches.items():        # eager warm-up step, then capture
        p = [nxt[r] for r in b.rows]
        b.fill(seqs, p, csc)
        b.stash()
        im.forward(layer, b.q, b.k, b.v, cache, b.md, output=b.out)
        torch.cuda.synchronize()
        _check(b.out.float().cpu(), _oracle_decode(olay, cache, C, bt, b.rows, p, b.q, csc),
               f"warm-up {name}")
        for r in b.rows:
            nxt[r] += 1
        g = torch.cuda.CUDAGraph()
        b.stash()
        with torch.cuda.graph(g):
            im.forward(layer, b.q, b.k, b.v, cache, b.md, output=b.out)
        graphs[name] = g
    ws = impl_mod.workspaces(dev)
    assert ws.frozen
    held = {k: v.data_ptr() for k, v in ws.bufs.items() if k.startswith("decode")}
    assert set(held) == {"decode", "decode_write"}

    # a larger batch, eagerly: all six requests
    rows = list(range(6))
    big = _DecodeBatch(rows, bt, builder, csc_d)
    big.md.max_seq_len = max(nxt) + 1      # an eager step carries the exact maximum
    p = [nxt[r] for r in rows]
    big.fill(seqs, p, csc)
    big.stash()
    im.forward(layer, big.q, big.k, big.v, cache, big.md, output=big.out)
    torch.cuda.synchronize()
    assert int(im.error_word.item()) == 0
    _check(big.out.float().cpu(), _oracle_decode(olay, cache, C, bt, rows, p, big.q, csc),
           "eager batch of 6")
    for r in rows:
        nxt[r] += 1
    assert {k: v.data_ptr() for k, v in ws.bufs.items() if k in held} == held

    # both graphs replayed, twice each, interleaved
    for t in range(2):
        for name in ("A", "B"):
            b = batches[name]
            p = [nxt[r] for r in b.rows]
            b.fill(seqs, p, csc)
            b.out.fill_(float("nan"))
            graphs[name].replay()
            torch.cuda.synchronize()
            assert int(im.error_word.item()) == 0
            _check(b.out.float().cpu(), _oracle_decode(olay, cache, C, bt, b.rows, p, b.q, csc),
                   f"replay {name} {t}")
            for r in b.rows:
                nxt[r] += 1
    rope_store.clear_stores()
    impl_mod.release_workspaces()


def test_recycled_first_block_gets_a_new_fit(monkeypatch):
    """A finished request's blocks, first block included, go to a new request (vLLM recycles
    them). The key (first block id) is the same, but the new request's first chunk is fitted
    and re-registered: its decoder is the fit of ITS keys, not the old request's basis, and its
    decode step matches the oracle."""
    from vllm_ttkv import encode as penc
    monkeypatch.delenv("VLLM_TTKV_CHECK", raising=False)
    lay = layout_for_config(CONFIGS["safe"], 110)
    olay = oracle_layout(CONFIGS["safe"], 110)
    rope_store.clear_stores()
    csc = cos_sin_cache(1024)
    old, new = _Seq(400, 51), _Seq(400, 52)
    bt, nblk = synth.shuffled_block_table([400], BS, seed=53, extra_blocks=1)
    C = lay.compressed_bytes_per_token()
    cache = torch.zeros(nblk, 1, BS, C // 2, dtype=torch.bfloat16, device="cuda")
    im = TTKVAttentionImpl(HQ, D, SCALE, H)
    layer = _Layer(NAME, lay)
    key = int(bt[0, 0])
    _step(im, layer, cache, csc, bt, [(old, 0, 300)])
    _step(im, layer, cache, csc, bt, [(old, 300, 301)])
    dec_old = rope_store.store_for_layer(NAME).decoders[key].decoder_f.clone()
    # the old request ends; a new one arrives on the same blocks
    _step(im, layer, cache, csc, bt, [(new, 0, 250)])
    st = rope_store.store_for_layer(NAME)
    dec_new = st.decoders[key].decoder_f
    want_dec = penc.fit_into_budget(new.K[:250].permute(1, 0, 2).contiguous().cuda(), lay,
                                    CONFIGS["safe"]).decoder.decoder_f
    assert torch.equal(dec_new, want_dec)
    assert not torch.equal(dec_new, dec_old)
    out, q, _, qsl, seq_lens = _step(im, layer, cache, csc, bt, [(new, 250, 251)])
    flat = cache.view(torch.uint8).reshape(-1, C).cpu()
    want = attend.paged_decode(olay, flat, bt[:1], torch.tensor(seq_lens), torch.tensor(qsl),
                               q.float(), [dec_new.cpu()], csc, BS, SCALE, dtype=torch.float64)
    _check(out, want, "decode after recycling")
    rope_store.clear_stores()


def test_running_request_outlives_short_requests_in_a_full_decoder_pool(monkeypatch):
    """A pool of 3 decoders. A running request decodes every other step and sits out the steps
    in between, where short requests arrive one at a time (first chunk only, then never seen
    again). Six of them register, more than the pool holds: eviction follows last use (the write
    kernel flags every decoder a step uses), so the short requests leave, oldest use first, and
    the running request keeps its decoder and decodes against the oracle after every one.
    (Registration order with `live` = the step's own requests evicted it at the third.)"""
    monkeypatch.delenv("VLLM_TTKV_CHECK", raising=False)
    monkeypatch.setenv("VLLM_TTKV_MAX_DECODERS", "3")
    lay = layout_for_config(CONFIGS["safe"], 110)
    olay = oracle_layout(CONFIGS["safe"], 110)
    rope_store.clear_stores()
    csc = cos_sin_cache(1024)
    run = _Seq(320, 61)
    shorts = [_Seq(96, 70 + i) for i in range(6)]
    bt, nblk = synth.shuffled_block_table([320] + [96] * 6, BS, seed=62, extra_blocks=1)
    C = lay.compressed_bytes_per_token()
    cache = torch.zeros(nblk, 1, BS, C // 2, dtype=torch.bfloat16, device="cuda")
    im = TTKVAttentionImpl(HQ, D, SCALE, H)
    layer = _Layer(NAME, lay)
    key = int(bt[0, 0])
    _step(im, layer, cache, csc, bt[[0]], [(run, 0, 300)])
    st = rope_store.store_for_layer(NAME)
    assert st.capacity == 3
    pos = 300
    for i, sq in enumerate(shorts):
        _step(im, layer, cache, csc, bt[[1 + i]], [(sq, 0, 96)])        # a short request
        out, q, _, qsl, seq_lens = _step(im, layer, cache, csc, bt[[0]], [(run, pos, pos + 1)])
        assert key in st.decoders and len(st.decoders) == min(3, 2 + i)
        flat = cache.view(torch.uint8).reshape(-1, C).cpu()
        want = attend.paged_decode(olay, flat, bt[[0]], torch.tensor(seq_lens), torch.tensor(qsl),
                                   q.float(), [st.decoders[key].decoder_f.cpu()], csc, BS, SCALE,
                                   dtype=torch.float64)
        _check(out, want, f"running request after short request {i}")
        pos += 1
    assert list(st.decoders) == [key, int(bt[5, 0]), int(bt[6, 0])]
    rope_store.clear_stores()


def test_padded_graph_replay_skips_pad_tokens(monkeypatch):
    """vLLM replays a graph captured for 4 decode requests with only 2 real ones: the 2 padded
    entries carry slot id -1 (PAD_SLOT_ID) and sequence length 0. The write skips the pad tokens
    without a refusal, the read returns zero rows for the empty requests, the error word stays 0
    (so a later checked step does not inherit a false refusal), and the real rows match the
    oracle."""
    monkeypatch.delenv("VLLM_TTKV_CHECK", raising=False)
    monkeypatch.setenv("VLLM_TTKV_MAX_NUM_SEQS", "8")
    monkeypatch.setenv("VLLM_TTKV_MAX_MODEL_LEN", "2048")
    impl_mod.release_workspaces()
    lay = layout_for_config(CONFIGS["safe"], 110)
    olay = oracle_layout(CONFIGS["safe"], 110)
    rope_store.clear_stores()
    csc = cos_sin_cache(2048)
    csc_d = csc.cuda()
    lens = [500, 700, 300, 420]
    seqs = [_Seq(L + 8, 80 + i) for i, L in enumerate(lens)]
    bt0, nblk = synth.shuffled_block_table([L + 8 for L in lens], BS, seed=81, extra_blocks=2)
    bt = torch.full((4, 2048 // BS), -1, dtype=torch.int32)
    bt[:, :bt0.shape[1]] = bt0
    C = lay.compressed_bytes_per_token()
    cache = torch.zeros(nblk, 1, BS, C // 2, dtype=torch.bfloat16, device="cuda")
    im = TTKVAttentionImpl(HQ, D, SCALE, H)
    layer = _Layer(NAME, lay)
    builder = TTKVAttentionMetadataBuilder()
    for r, L in enumerate(lens):                       # first chunks, one request per step
        _step(im, layer, cache, csc, bt[[r]], [(seqs[r], 0, L)])
    b = _DecodeBatch([0, 1, 2, 3], bt, builder, csc_d)
    nxt = list(lens)
    b.fill(seqs, nxt, csc)                             # eager warm-up at the full size
    b.stash()
    im.forward(layer, b.q, b.k, b.v, cache, b.md, output=b.out)
    torch.cuda.synchronize()
    assert int(im.error_word.item()) == 0
    nxt = [p + 1 for p in nxt]
    g = torch.cuda.CUDAGraph()
    b.stash()
    with torch.cuda.graph(g):
        im.forward(layer, b.q, b.k, b.v, cache, b.md, output=b.out)
    for t in range(2):                                 # replays with 2 real requests
        b.fill(seqs, nxt, csc)
        b.md.slot_mapping[2:] = -1
        b.md.seq_lens[2:] = 0
        page_before = cache.view(torch.uint8).reshape(-1, C).clone()
        b.out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert int(im.error_word.item()) == 0, f"replay {t}: error word {int(im.error_word.item())}"
        assert torch.equal(b.out[2:].float().cpu(), torch.zeros(2, HQ, D))
        # the pad tokens wrote nothing: only the two real tokens' slots changed
        after = cache.view(torch.uint8).reshape(-1, C)
        changed = (after != page_before).any(1).nonzero().flatten().cpu().tolist()
        real = [int(bt[r, nxt[r] // BS]) * BS + nxt[r] % BS for r in (0, 1)]
        assert set(changed) <= set(real), changed
        want = _oracle_decode(olay, cache, C, bt, [0, 1], nxt[:2], b.q[:2], csc)
        _check(b.out[:2].float().cpu(), want, f"padded replay {t}")
        nxt = [p + 1 for p in nxt[:2]] + nxt[2:]
    rope_store.clear_stores()
    impl_mod.release_workspaces()
