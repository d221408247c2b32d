"""The vLLM `AttentionBackend` for the compressed-KV cache (reference: vllm_ttkv/backend.py).

Same flags and hooks: the backend owns its cache write, accepts `auto`/`bfloat16` cache dtypes,
registers as the CUSTOM backend, supports head size 128, uses the LBNHC layout, and sizes each
layer's page from its calibrated layout (`pack_spec_for_layer`). vLLM is imported lazily so the
module imports (and its sizing logic is testable) without vLLM installed.
"""
from __future__ import annotations

import os
from dataclasses import replace

from .impl import TTKVAttentionImpl
from .metadata import TTKVAttentionMetadataBuilder
from .rope_store import calibration_info, layout_for_layer, load_calibration

try:  # pragma: no cover
    from vllm.v1.attention.backend import AttentionBackend as _Base
except Exception:  # noqa: BLE001
    _Base = object

CALIBRATION_ENV = "VLLM_TTKV_CALIBRATION"
_SUPPORTED_HEAD_DIMS = frozenset({128})


def _ensure_calibration() -> None:
    if calibration_info():
        return
    path = os.environ.get(CALIBRATION_ENV)
    if path:
        load_calibration(path, cfg_name=os.environ.get("VLLM_TTKV_CONFIG", "safe"))


class TTKVAttentionBackend(_Base):
    forward_includes_kv_cache_update = True
    supported_kv_cache_dtypes = ["auto", "bfloat16"]

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls():
        return TTKVAttentionImpl

    @staticmethod
    def get_builder_cls():
        return TTKVAttentionMetadataBuilder

    @classmethod
    def supported_kv_cache_layouts(cls):  # pragma: no cover - needs vLLM
        from vllm.v1.kv_cache_layout import KVCacheLayout
        return (KVCacheLayout.LBNHC,)

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        return head_size in _SUPPORTED_HEAD_DIMS

    @classmethod
    def customize_spec(cls, spec):
        """A spec must arrive already packed per layer (backend.py:130-162)."""
        if getattr(spec, "state_content_bytes", None) is not None and spec.num_head_slots == 1:
            return spec
        raise RuntimeError(
            "a TT-KV spec reached `customize_spec` unpacked, so the per-layer sizing hook did not "
            "run; an unpacked spec is sized for dense K||V and the packed writes would read back "
            "as noise.")


def pack_spec_for_layer(spec, layer_name: str):
    """Size one layer's page from its calibrated layout (backend.py:165-245)."""
    _ensure_calibration()
    lay = layout_for_layer(layer_name)
    if lay is None:
        raise RuntimeError(f"no calibrated TT-KV layout for layer {layer_name!r}; set "
                           f"{CALIBRATION_ENV} to a calibration artifact")
    table_d = calibration_info().get("head_dim")
    spec_d = int(getattr(spec, "head_size", 0) or 0)
    if table_d and spec_d and int(table_d) != spec_d:
        raise RuntimeError(f"calibration was measured at head_dim={table_d} but this spec has "
                           f"head_size={spec_d}")
    blob = lay.compressed_bytes_per_token()
    return replace(spec, num_head_slots=1, state_content_bytes=blob, head_size=blob)
