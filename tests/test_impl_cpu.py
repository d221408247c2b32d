"""The drop-in AttentionImpl / backend surface on the CPU: batch planning, refusals, the raw-key
stash, spec sizing, and that there is no CPU compute path (reference tests: test_impl_decode.py
refusal cases, test_spec_sizing.py)."""
from dataclasses import dataclass

import pytest
import torch

from vllm_ttkv import backend, impl, patch, rope_store
from vllm_ttkv.layout import CONFIGS, layout_for_config
from vllm_ttkv.metadata import TTKVAttentionMetadata, TTKVAttentionMetadataBuilder


def _md(qsl, seq_lens, nblk=64, bs=16):
    B = len(qsl) - 1
    bt = torch.arange(B * 8, dtype=torch.int32).reshape(B, 8)
    N = qsl[-1]
    return TTKVAttentionMetadata(
        seq_lens=torch.tensor(seq_lens, dtype=torch.int32), slot_mapping=torch.arange(N),
        block_table=bt, query_start_loc=torch.tensor(qsl, dtype=torch.int32),
        query_start_loc_cpu=torch.tensor(qsl, dtype=torch.int32), num_actual_tokens=N,
        max_query_len=max(qsl[i + 1] - qsl[i] for i in range(B)), max_seq_len=max(seq_lens))


def test_plan_decodes_first():
    p = impl.BatchPlan.of(_md([0, 1, 2, 10, 30], [5, 9, 8, 40]))
    assert p.n_decodes == 2 and p.prefills == [2, 3] and p.n_reqs == 4


def test_plan_refuses_decode_after_prefill():
    with pytest.raises(RuntimeError, match="not contiguous at the front"):
        impl.BatchPlan.of(_md([0, 5, 6], [5, 9]))


def test_plan_refuses_missing_fields():
    md = _md([0, 1], [3])
    md.block_table = None
    with pytest.raises(RuntimeError, match="missing"):
        impl.BatchPlan.of(md)


@pytest.mark.parametrize("kw,msg", [(dict(alibi_slopes=[1.0]), "ALiBi"),
                                    (dict(logits_soft_cap=30.0), "logits_soft_cap"),
                                    (dict(sliding_window=128), "sliding window"),
                                    (dict(kv_sharing_target_layer_name="x"), "KV sharing")])
def test_constructor_refusals(kw, msg):
    with pytest.raises(NotImplementedError, match=msg):
        impl.TTKVAttentionImpl(24, 128, 128 ** -0.5, 8, **kw)


def test_heads_must_divide():
    with pytest.raises(ValueError, match="multiple"):
        impl.TTKVAttentionImpl(24, 128, 0.1, 7)


def test_output_quant_refused():
    im = impl.TTKVAttentionImpl(24, 128, 0.1, 8)
    with pytest.raises(NotImplementedError, match="quantization"):
        im.forward(None, None, None, None, None, None, output_scale=torch.ones(1))


def test_missing_stash_is_an_error():
    with pytest.raises(RuntimeError, match="no raw"):
        patch.take_raw_k("model.layers.99.self_attn.attn")
    patch.stash_raw_k("L", torch.zeros(1))
    patch.take_raw_k("L")
    with pytest.raises(RuntimeError):  # consumed exactly once
        patch.take_raw_k("L")


@dataclass
class _Layer:
    layer_name: str
    ttkv_layout: object = None


def test_forward_has_no_cpu_path():
    """With every host check passing, CPU tensors reach the kernel wrapper and are refused there:
    the product has no CPU implementation to fall back on."""
    lay = layout_for_config(CONFIGS["safe"], 110)
    name = "model.layers.3.self_attn.attn"
    rope_store.clear_stores()
    im = impl.TTKVAttentionImpl(24, 128, 128 ** -0.5, 8)
    md = _md([0, 1, 2], [5, 9])
    cache = torch.zeros(64, 1, 16, lay.compressed_bytes_per_token() // 2, dtype=torch.bfloat16)
    from vllm_ttkv.rope import cos_sin_cache
    patch.stash_raw_k(name, torch.randn(2, 8 * 128), cos_sin_cache=cos_sin_cache(64))
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        im.forward(_Layer(name, lay), torch.randn(2, 24, 128), torch.randn(2, 8 * 128),
                   torch.randn(2, 8 * 128), cache, md, output=torch.zeros(2, 24, 128))
    rope_store.clear_stores()


def test_layout_mismatch_refused():
    from vllm_ttkv.layout import TTKLayout
    lay = TTKLayout(H=8, d=64, r1=32, qbits=8, res_k=40, res_bits=3, v_lanes=40, v_bits=3)
    im = impl.TTKVAttentionImpl(24, 128, 0.1, 8)
    with pytest.raises(RuntimeError, match="head_dim=64"):
        im._layout(_Layer("model.layers.0.attn", lay))


def test_kv_cache_must_be_one_tensor():
    with pytest.raises(RuntimeError, match="ONE cache tensor"):
        impl.TTKVAttentionImpl._cache_tensor((torch.zeros(1), torch.zeros(1)))


@dataclass(frozen=True)
class _Spec:
    block_size: int = 16
    num_kv_heads: int = 8
    head_size: int = 128
    num_head_slots: int = 8
    state_content_bytes: int | None = None


def test_spec_sizing_from_calibration(tmp_path, monkeypatch):
    """pack_spec_for_layer sizes the page row from the layer's calibrated rank
    (backend.py:165-245): one head slot, row = the blob."""
    art = tmp_path / "cal.json"
    art.write_text('{"layers": 2, "heads": 8, "head_dim": 128, "r1": [40, 110]}')
    rope_store.clear_stores()
    rope_store.load_calibration(art, "safe")
    s1 = backend.pack_spec_for_layer(_Spec(), "model.layers.1.self_attn.attn")
    assert s1.num_head_slots == 1 and s1.state_content_bytes == 912
    s0 = backend.pack_spec_for_layer(_Spec(), "model.layers.0.self_attn.attn")
    assert s0.state_content_bytes < 912
    assert backend.TTKVAttentionBackend.customize_spec(s1) is s1
    with pytest.raises(RuntimeError, match="unpacked"):
        backend.TTKVAttentionBackend.customize_spec(_Spec())
    with pytest.raises(RuntimeError, match="head_dim=128"):
        backend.pack_spec_for_layer(_Spec(head_size=64), "model.layers.1.self_attn.attn")
    rope_store.load_calibration(art, "safe")


def test_backend_flags():
    B = backend.TTKVAttentionBackend
    assert B.forward_includes_kv_cache_update is True
    assert B.get_name() == "CUSTOM" and B.get_impl_cls() is impl.TTKVAttentionImpl
    assert B.get_builder_cls() is TTKVAttentionMetadataBuilder
    assert B.supports_head_size(128) and not B.supports_head_size(64)
    assert "bfloat16" in B.supported_kv_cache_dtypes


def _codec_dec(r1=16, hd=8 * 128, seed=0):
    """A decoder in the codec's form (int8 rows times an fp16 ruler per rank), as every fit
    produces (encode.py:257-298)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-128, 128, (r1, hd), generator=g).float()
    ruler = (torch.rand(r1, generator=g) * 1e-2 + 1e-4).half().float()
    return q * ruler[:, None]


def test_decoder_registry_round_trip():
    """Fixed-capacity pool: registration, release, slot reuse, eviction of the oldest
    registration that is not live, and refusal when every slot is live. The pools are never
    reallocated (a captured graph keeps valid pointers)."""
    lay = layout_for_config(CONFIGS["safe"], 16)
    from vllm_ttkv.encode import KDecoder
    rope_store.clear_stores()
    st = rope_store.TTKVRopeStore(24, 8, 128, torch.zeros(8, 128), "L0", lay, num_blocks=10,
                                  capacity=2)
    from vllm_ttkv.decoder_pool import unpack_decoders
    pools = (st.dec_pool.q.data_ptr(), st.dec_pool.scale.data_ptr(), st.pinv_pool.data_ptr(),
             st.dec_map.data_ptr())
    d1, d2, d3 = (KDecoder(_codec_dec(seed=i)) for i in range(3))
    s1 = st.register(3, d1)
    s2 = st.register(7, d2)
    assert st.dec_map[3] == s1 and st.dec_map[7] == s2 and s1 != s2
    assert torch.equal(unpack_decoders(st.dec_pool.slot(s2), 16), d2.decoder_f)
    assert torch.allclose(st.pinv_pool[s2], d2.pinv.t())
    st.release(3)
    assert st.dec_map[3] == -1 and 3 not in st.decoders
    assert st.register(5, d1) == s1               # freed slot reused
    assert st.register(5, d3) == s1               # re-registering a key keeps its slot
    assert torch.equal(unpack_decoders(st.dec_pool.slot(s1), 16), d3.decoder_f)
    # full: the oldest registration not named live is evicted (7, registered before 5)
    s9 = st.register(9, d1, live=[5, 9])
    assert s9 == s2 and st.dec_map[7] == -1 and 7 not in st.decoders and st.dec_map[9] == s9
    with pytest.raises(RuntimeError, match="live requests"):
        st.register(2, d2, live=[5, 9, 2])
    with pytest.raises(IndexError):
        st.register(10, d1)
    assert (st.dec_pool.q.data_ptr(), st.dec_pool.scale.data_ptr(), st.pinv_pool.data_ptr(),
            st.dec_map.data_ptr()) == pools
    rope_store.clear_stores()


def test_registry_refuses_a_decoder_the_pool_cannot_hold():
    """The pool stores the codec's int8 decoder (int8 rows times one ruler per rank, as every
    fit produces): a decoder of another form is refused with an error, and the pool and map are
    left as they were."""
    lay = layout_for_config(CONFIGS["safe"], 16)
    from vllm_ttkv.encode import KDecoder
    rope_store.clear_stores()
    st = rope_store.TTKVRopeStore(24, 8, 128, torch.zeros(8, 128), "L0", lay, num_blocks=10,
                                  capacity=2)
    ok = st.register(1, KDecoder(_codec_dec(seed=4)))
    before = (st.dec_pool.q.clone(), st.dec_pool.scale.clone(), st.dec_map.clone())
    with pytest.raises(ValueError, match="int8"):
        st.register(2, KDecoder(torch.randn(16, 8 * 128)))
    assert torch.equal(st.dec_pool.q, before[0]) and torch.equal(st.dec_pool.scale, before[1])
    assert torch.equal(st.dec_map, before[2]) and int(st.dec_map[1]) == ok
    assert 2 not in st.decoders and st.register(3, KDecoder(_codec_dec(seed=5))) != ok
    with pytest.raises(RuntimeError, match="live requests"):       # both slots now in use
        st.register(4, KDecoder(_codec_dec(seed=6)), live=[1, 3, 4])
    rope_store.clear_stores()


def test_decoder_eviction_follows_last_use():
    """A full pool evicts the least recently USED key that is not live. Use comes from the write
    kernel's flags (`dec_used`, one per slot, set here by hand as the kernel would): a running
    request that decodes every other step keeps its slot while short requests that registered
    after it, ran their first chunk and finished are evicted, oldest use first. (Registration
    order alone evicted the running request first.)"""
    lay = layout_for_config(CONFIGS["safe"], 16)
    from vllm_ttkv.encode import KDecoder
    rope_store.clear_stores()
    st = rope_store.TTKVRopeStore(24, 8, 128, torch.zeros(8, 128), "L0", lay, num_blocks=40,
                                  capacity=3)
    dec = KDecoder(_codec_dec())
    a = st.register(1, dec, live=[1])                  # the running request
    for step, key in enumerate(range(10, 20)):         # 10 short requests, one per even step
        st.dec_used[a] = 1                             # odd step: request 1 decodes
        st.register(key, dec, live=[key])              # even step: key's first chunk only
        assert st.dec_map[1] == a and 1 in st.decoders, f"running request evicted at {key}"
        assert len(st.decoders) == min(3, 2 + step)
    assert list(st.decoders) == [1, 18, 19]
    # every key used at the same tick: the older registration goes first
    st.dec_used.fill_(1)
    st.observe_use()
    assert st.eviction_order() == [1, 18, 19]
    st.register(30, dec)
    assert 1 not in st.decoders and list(st.decoders) == [18, 19, 30]
    # a released key frees its slot without an eviction
    st.release(18)
    st.register(31, dec)
    assert list(st.decoders) == [19, 30, 31]
    rope_store.clear_stores()


def test_reference_calling_sequence_binds():
    """The reference's own adapter-test sequence (tests/test_impl_decode.py:218-225): build the
    store with its constructor, then `register_decoder(name, request_key(row), KDecoder(dec))`
    through the module functions. Registrations made before a store exists are adopted by it;
    the device map is bound when the cache's block count is known."""
    from vllm_ttkv.encode import KDecoder
    lay = layout_for_config(CONFIGS["safe"], 16)
    rope_store.clear_stores()
    name = "model.layers.4.self_attn"
    from vllm_ttkv.decoder_pool import unpack_decoders
    dec_a, dec_b = _codec_dec(seed=1), _codec_dec(seed=2)
    bt = torch.tensor([[6, 2, 9], [4, 0, -1]], dtype=torch.int32)
    rope_store.register_decoder(name, rope_store.request_key(bt[0]), KDecoder(dec_a))  # pending
    assert rope_store.decoder_for_request(name, 6).decoder_f is not None
    store = rope_store.TTKVRopeStore(24, 8, 128, torch.zeros(64, 128), name, lay)
    assert rope_store.store_for_layer(name) is store and rope_store.layout_for_layer(name) is lay
    rope_store.register_decoder(name, rope_store.request_key_host(bt[1].tolist()),
                                KDecoder(dec_b))
    assert store.dec_map is None                                   # not bound yet
    again = rope_store.ensure_store(name, torch.zeros(64, 128), 24, 8, 128, lay, num_blocks=12)
    assert again is store and store.dec_map.numel() == 12
    for key, dec in ((6, dec_a), (4, dec_b)):
        slot = int(store.dec_map[key])
        assert slot >= 0 and torch.equal(unpack_decoders(store.dec_pool.slot(slot), 16), dec)
        assert rope_store.decoder_for_request(name, key).decoder_f is not None
    assert rope_store.decoder_for_layer(name) is None              # no layer-level decoder
    rope_store.release_decoder(name, 6)
    assert int(store.dec_map[6]) == -1 and rope_store.decoder_for_request(name, 6) is None
    with pytest.raises(ValueError):
        rope_store.request_key(torch.zeros(0, dtype=torch.int32))
    with pytest.raises(RuntimeError):
        rope_store.ensure_store("model.layers.99.x", torch.zeros(4, 128), 24, 8, 128, None)
    rope_store.clear_stores()


def test_layer_index_of_vllm_names():
    li = rope_store._layer_index
    assert li("model.layers.7.self_attn.attn") == 7
    assert li("model.decoder_layers.3.attn.5") == 3
    assert li("layers.12") == 12 and li("attn_9") == 9 and li("attn") is None


class _NoRead:
    """A device tensor stand-in that fails if the host reads it."""

    def __getitem__(self, item):
        raise AssertionError("seq_lens was read back")


def test_prefill_plan_from_host_metadata():
    """With `num_computed_tokens_cpu`, first chunks and exact lengths come from the host: the
    device `seq_lens` is never read. Without it, one read of `seq_lens` decides."""
    md = _md([0, 1, 41, 141], [9, 40, 300])
    plan = impl.BatchPlan.of(md)
    im = impl.TTKVAttentionImpl(24, 128, 128 ** -0.5, 8)
    assert im._first_chunks(md, plan) == [False, True, False]
    assert im._seq_lens_host(md, plan) == [9, 40, 300]
    md.num_computed_tokens_cpu = torch.tensor([8, 0, 200], dtype=torch.int32)
    md.seq_lens = _NoRead()
    assert im._first_chunks(md, plan) == [False, True, False]
    assert im._seq_lens_host(md, plan) == [9, 40, 300]


def test_builder_declares_uniform_decode_graphs(monkeypatch):
    from types import SimpleNamespace
    from vllm_ttkv.metadata import AttentionCGSupport
    assert (TTKVAttentionMetadataBuilder.cudagraph_support
            == AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE)
    monkeypatch.setenv("VLLM_TTKV_MAX_MODEL_LEN", "4096")
    b = TTKVAttentionMetadataBuilder()
    qsl = torch.arange(4, dtype=torch.int32)
    cam = SimpleNamespace(seq_lens=torch.ones(3, dtype=torch.int32),
                          slot_mapping=torch.zeros(3, dtype=torch.int64),
                          block_table_tensor=torch.zeros(3, 4, dtype=torch.int32),
                          query_start_loc=qsl, query_start_loc_cpu=qsl, num_actual_tokens=3,
                          max_query_len=1, max_seq_len=17,
                          _num_computed_tokens_cpu=torch.tensor([16, 3, 0]))
    md = b.build_for_cudagraph_capture(cam)
    assert md.max_seq_len == 4096 and md.ttkv_serial > 0
    assert md.num_computed_tokens_cpu.tolist() == [16, 3, 0]
    assert b.can_run_in_cudagraph(cam)
    cam.max_query_len = 5
    assert not b.can_run_in_cudagraph(cam)
    with pytest.raises(RuntimeError, match="uniform single-token decode"):
        b.build_for_cudagraph_capture(cam)
    monkeypatch.delenv("VLLM_TTKV_MAX_MODEL_LEN")
    cam.max_query_len = 1
    with pytest.raises(RuntimeError, match="maximum length"):
        TTKVAttentionMetadataBuilder().build_for_cudagraph_capture(cam)


def test_fixed_workspaces_are_never_replaced_once_frozen():
    ws = impl.DeviceWorkspaces("cpu")
    a = ws.get("decode", 1000, capacity=4096, fixed=True)
    assert a.numel() == 4096 and ws.get("decode", 4000, fixed=True) is a
    b = ws.get("decode", 5000, fixed=True)           # before any capture: may grow
    assert b.numel() == 5000
    p = ws.get("prefill", 100)
    ws.frozen = True                                 # a graph now holds the decode buffers
    assert ws.get("decode", 5000, fixed=True) is b
    with pytest.raises(RuntimeError, match="captured graph"):
        ws.get("decode", 5001, fixed=True)
    assert ws.get("prefill", 10 ** 4).numel() == 10 ** 4 and ws.get("prefill", 1) is not p


def test_serving_limits_from_environment(monkeypatch):
    monkeypatch.delenv("VLLM_TTKV_MAX_NUM_SEQS", raising=False)
    monkeypatch.delenv("VLLM_TTKV_MAX_MODEL_LEN", raising=False)
    assert impl.serving_limits(1234) == (256, 1234)
    monkeypatch.setenv("VLLM_TTKV_MAX_NUM_SEQS", "12")
    monkeypatch.setenv("VLLM_TTKV_MAX_MODEL_LEN", "777")
    assert impl.serving_limits(1234) == (12, 777)
