"""Per-step attention metadata: the fields the compressed-KV read and write need.

Field names and meaning follow the reference's `vllm_ttkv/metadata.py:48-147`. vLLM is imported
lazily: without it the dataclass and the builder still work (tests build metadata directly).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

try:  # pragma: no cover - vLLM is not installed in the build container
    from vllm.v1.attention.backend import AttentionMetadata as _MDBase
    from vllm.v1.attention.backend import AttentionMetadataBuilder as _BuilderBase
except Exception:  # noqa: BLE001
    _MDBase = object
    _BuilderBase = object

_SERIAL = [0]


@dataclass
class TTKVAttentionMetadata(_MDBase):
    seq_lens: torch.Tensor | None = None           # [num_reqs] int32, includes this step's token
    slot_mapping: torch.Tensor | None = None       # [num_tokens] int64, block*bs + offset
    block_table: torch.Tensor | None = None        # [num_reqs, max_blocks] int32
    query_start_loc: torch.Tensor | None = None    # [num_reqs + 1] int32
    query_start_loc_cpu: torch.Tensor | None = None
    seq_lens_cpu_upper_bound: torch.Tensor | None = None
    positions: torch.Tensor | None = None
    num_actual_tokens: int = 0
    max_query_len: int = 0
    max_seq_len: int = 0
    ttkv_serial: int = 0


class TTKVAttentionMetadataBuilder(_BuilderBase):
    """Copies the fields off vLLM's CommonAttentionMetadata and stamps a serial
    (metadata.py:93-147). Decodes are reordered to the front (`reorder_batch_threshold = 1`)."""

    reorder_batch_threshold: int = 1

    def __init__(self, kv_cache_spec=None, layer_names=None, vllm_config=None, device=None):
        if _BuilderBase is not object:  # pragma: no cover
            super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        if vllm_config is not None and getattr(vllm_config, "speculative_config", None) is not None:
            raise NotImplementedError("TT-KV does not support speculative decoding")
        if _BuilderBase is not object and hasattr(self, "_init_reorder_batch_threshold"):
            self._init_reorder_batch_threshold(reorder_batch_threshold=1,
                                               supports_spec_as_decode=False)

    def build(self, common_prefix_len=None, common_attn_metadata=None, fast_build=False):
        cam = common_attn_metadata
        if cam is None:
            raise RuntimeError("build() was called without `common_attn_metadata`")
        _SERIAL[0] += 1
        return TTKVAttentionMetadata(
            seq_lens=cam.seq_lens, slot_mapping=cam.slot_mapping,
            block_table=cam.block_table_tensor, query_start_loc=cam.query_start_loc,
            query_start_loc_cpu=getattr(cam, "query_start_loc_cpu", None),
            seq_lens_cpu_upper_bound=getattr(cam, "seq_lens_cpu_upper_bound", None),
            positions=getattr(cam, "positions", None), num_actual_tokens=cam.num_actual_tokens,
            max_query_len=cam.max_query_len, max_seq_len=cam.max_seq_len,
            ttkv_serial=_SERIAL[0])
