"""Per-step attention metadata: the fields the compressed-KV read and write need.

Field names and meaning follow the reference's `vllm_ttkv/metadata.py:48-147`. vLLM is imported
lazily: without it the dataclass and the builder still work (tests build metadata directly).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

import enum
import os

try:  # pragma: no cover - vLLM is not installed in the build container
    from vllm.v1.attention.backend import AttentionMetadata as _MDBase
    from vllm.v1.attention.backend import AttentionMetadataBuilder as _BuilderBase
except Exception:  # noqa: BLE001
    _MDBase = object
    _BuilderBase = object

try:  # pragma: no cover
    from vllm.v1.attention.backends.utils import AttentionCGSupport
except Exception:  # noqa: BLE001
    try:  # pragma: no cover
        from vllm.v1.attention.backend import AttentionCGSupport
    except Exception:  # noqa: BLE001
        class AttentionCGSupport(enum.Enum):
            """vLLM's graph-support levels, for use without vLLM."""
            ALWAYS = 3
            UNIFORM_BATCH = 2
            UNIFORM_SINGLE_TOKEN_DECODE = 1
            NEVER = 0

_SERIAL = [0]


def _host_field(cam, name):
    """A CPU tensor vLLM keeps on the common metadata under `name` or `_name`, read only when it
    is a stored attribute (a property of that name may synchronise to build it)."""
    attrs = getattr(cam, "__dict__", {})
    for key in (name, "_" + name):
        if attrs.get(key) is not None:
            return attrs[key]
    return None


@dataclass
class TTKVAttentionMetadata(_MDBase):
    seq_lens: torch.Tensor | None = None           # [num_reqs] int32, includes this step's token
    slot_mapping: torch.Tensor | None = None       # [num_tokens] int64, block*bs + offset
    block_table: torch.Tensor | None = None        # [num_reqs, max_blocks] int32
    query_start_loc: torch.Tensor | None = None    # [num_reqs + 1] int32
    query_start_loc_cpu: torch.Tensor | None = None
    seq_lens_cpu_upper_bound: torch.Tensor | None = None
    positions: torch.Tensor | None = None
    # [num_reqs] CPU: tokens already in the cache before this step (exact; 0 = a first chunk).
    # Lets a prefill step plan its fits without reading `seq_lens` back.
    num_computed_tokens_cpu: torch.Tensor | None = None
    num_actual_tokens: int = 0
    max_query_len: int = 0
    max_seq_len: int = 0
    ttkv_serial: int = 0


class TTKVAttentionMetadataBuilder(_BuilderBase):
    """Copies the fields off vLLM's CommonAttentionMetadata and stamps a serial
    (metadata.py:93-147). Decodes are reordered to the front (`reorder_batch_threshold = 1`).

    Unlike the reference's builder (which keeps vLLM's default, NEVER), this one declares
    UNIFORM_SINGLE_TOKEN_DECODE: a decode-only step issues device-only work on buffers that are
    never replaced (`impl`), so vLLM may capture it. The capture metadata sets `max_seq_len` to
    the model's maximum length: K1's grid is sized from it, and its work plan follows the real
    lengths on the device at every replay."""

    reorder_batch_threshold: int = 1
    cudagraph_support = AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE

    def __init__(self, kv_cache_spec=None, layer_names=None, vllm_config=None, device=None):
        if _BuilderBase is not object:  # pragma: no cover
            super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        if vllm_config is not None and getattr(vllm_config, "speculative_config", None) is not None:
            raise NotImplementedError("TT-KV does not support speculative decoding")
        if _BuilderBase is not object and hasattr(self, "_init_reorder_batch_threshold"):
            self._init_reorder_batch_threshold(reorder_batch_threshold=1,
                                               supports_spec_as_decode=False)
        mc = getattr(vllm_config, "model_config", None)
        env = os.environ.get("VLLM_TTKV_MAX_MODEL_LEN")
        self.max_model_len = int(env) if env else getattr(mc, "max_model_len", None)

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
            positions=getattr(cam, "positions", None),
            num_computed_tokens_cpu=_host_field(cam, "num_computed_tokens_cpu"),
            num_actual_tokens=cam.num_actual_tokens,
            max_query_len=cam.max_query_len, max_seq_len=cam.max_seq_len,
            ttkv_serial=_SERIAL[0])

    def build_for_cudagraph_capture(self, common_attn_metadata):
        """Metadata for capturing a uniform decode step: as `build`, with `max_seq_len` raised to
        the model's maximum length so the captured grid covers every later length."""
        cam = common_attn_metadata
        if int(cam.max_query_len) != 1:
            raise RuntimeError(f"TT-KV captures uniform single-token decode steps only; the "
                               f"capture batch has max_query_len={cam.max_query_len}")
        if self.max_model_len is None:
            raise RuntimeError("capturing a decode step needs the model's maximum length (the "
                               "vLLM config's max_model_len or VLLM_TTKV_MAX_MODEL_LEN)")
        md = self.build(0, cam)
        md.max_seq_len = max(int(self.max_model_len), int(cam.max_seq_len))
        return md

    def can_run_in_cudagraph(self, common_attn_metadata) -> bool:
        return int(common_attn_metadata.max_query_len) == 1
