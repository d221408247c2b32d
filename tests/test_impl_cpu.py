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


def test_decoder_registry_round_trip():
    lay = layout_for_config(CONFIGS["safe"], 16)
    from vllm_ttkv.encode import KDecoder
    st = rope_store.TTKVRopeStore("L0", torch.zeros(8, 128), lay, num_blocks=10, capacity=1)
    d1 = KDecoder(torch.randn(16, 8 * 128))
    d2 = KDecoder(torch.randn(16, 8 * 128))
    s1 = st.register(3, d1)
    s2 = st.register(7, d2)                       # grows the pool
    assert st.dec_map[3] == s1 and st.dec_map[7] == s2 and s1 != s2
    assert torch.equal(st.dec_pool[s2], d2.decoder_f)
    st.release(3)
    assert st.dec_map[3] == -1 and 3 not in st.decoders
    assert st.register(5, d1) == s1               # slot reused
    with pytest.raises(IndexError):
        st.register(10, d1)
    rope_store.clear_stores()
