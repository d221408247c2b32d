"""Per-layer state the attention layer needs: calibrated layouts, the RoPE table, and each
request's fitted decoder in a device-addressable pool.

Same surface as the reference's `vllm_ttkv/rope_store.py:70-300` (`load_calibration`,
`layout_for_layer`, `register_decoder`, `decoder_for_request`, `release_decoder`,
`clear_decoders`, `ensure_store`, `store_for_layer`), with one structural change: a decoder is
registered into a per-layer DEVICE pool (`dec_pool [slots, r1, H*d]`, `pinv_pool [slots, H*d,
r1]`) and the request key -> slot map (`dec_map [num_blocks]`, keyed by `block_table[r, 0]` as in
the reference, rope_store.py:148-163) lives on the device too. The decode and write kernels
resolve a request's decoder themselves, so a step needs no host read of the block table.
"""
from __future__ import annotations

import json
import pathlib
import re

import torch

from .encode import KDecoder
from .layout import CONFIGS, TTKLayout, layout_for_config

CONFIG_ENV = "VLLM_TTKV_CONFIG"

_CALIBRATED: dict[int, TTKLayout] = {}
_CALIBRATION: dict = {}
_STORES: dict[str, "TTKVRopeStore"] = {}


def _layer_index(layer_name: str):
    m = re.search(r"layers\.(\d+)", layer_name)
    if m:
        return int(m.group(1))
    nums = re.findall(r"(\d+)", layer_name)
    return int(nums[-1]) if nums else None


def load_calibration(path, cfg_name: str = "safe", cfg: dict | None = None) -> dict:
    """Per-layer layouts from a calibration artifact (`{"layers", "heads", "head_dim", "r1":[..]}`),
    rope_store.py:70-98."""
    global _CALIBRATION
    cfg = CONFIGS[cfg_name] if cfg is None else cfg
    data = json.loads(pathlib.Path(path).read_text())
    r1 = data["r1"]
    if len(r1) != data["layers"]:
        raise ValueError(f"{path}: r1 has {len(r1)} entries but layers={data['layers']}")
    _CALIBRATED.clear()
    for idx, rank in enumerate(r1):
        _CALIBRATED[idx] = layout_for_config(cfg, int(rank), H=data["heads"], d=data["head_dim"])
    _CALIBRATION = dict(data)
    return _CALIBRATION


def set_layout(layer_index: int, lay: TTKLayout) -> None:
    """Install one layer's layout directly (tests, tools)."""
    _CALIBRATED[layer_index] = lay


def calibration_info() -> dict:
    return dict(_CALIBRATION)


def layout_for_layer(layer_name: str | None) -> TTKLayout | None:
    if layer_name is None:
        return None
    st = _STORES.get(layer_name)
    if st is not None:
        return st.layout
    idx = _layer_index(layer_name)
    return _CALIBRATED.get(idx) if idx is not None else None


class TTKVRopeStore:
    """One layer's RoPE table (fp32, vLLM layout) and its decoder pool."""

    def __init__(self, layer_name: str, cos_sin_cache: torch.Tensor, layout: TTKLayout,
                 num_blocks: int, capacity: int = 64):
        dev = cos_sin_cache.device
        self.layer_name = layer_name
        self.layout = layout
        # bf16/fp16 model tables convert to fp32 exactly; the values are the model's own.
        self.cos_sin_cache = cos_sin_cache.to(torch.float32).contiguous()
        H, d, r1 = layout.H, layout.d, layout.r1
        self.dec_pool = torch.zeros(capacity, r1, H * d, dtype=torch.float32, device=dev)
        self.pinv_pool = torch.zeros(capacity, H * d, r1, dtype=torch.float32, device=dev)
        self.dec_map = torch.full((num_blocks,), -1, dtype=torch.int32, device=dev)
        self._slot_of: dict[int, int] = {}
        self._free = list(range(capacity - 1, -1, -1))
        self.decoders: dict[int, KDecoder] = {}
        _STORES[layer_name] = self

    def _grow(self):
        cap = self.dec_pool.shape[0]
        self.dec_pool = torch.cat([self.dec_pool, torch.zeros_like(self.dec_pool)])
        self.pinv_pool = torch.cat([self.pinv_pool, torch.zeros_like(self.pinv_pool)])
        self._free.extend(range(2 * cap - 1, cap - 1, -1))

    def register(self, key: int, dec: KDecoder) -> int:
        if dec.decoder_f.shape != (self.layout.r1, self.layout.H * self.layout.d):
            raise ValueError(f"decoder is {tuple(dec.decoder_f.shape)}; the layout budgets "
                             f"[{self.layout.r1}, {self.layout.H * self.layout.d}]")
        if not (0 <= key < self.dec_map.numel()):
            raise IndexError(f"request key (first block) {key} outside the cache's "
                             f"{self.dec_map.numel()} blocks")
        slot = self._slot_of.get(key)
        if slot is None:
            if not self._free:
                self._grow()
            slot = self._free.pop()
            self._slot_of[key] = slot
        self.dec_pool[slot].copy_(dec.decoder_f)
        self.pinv_pool[slot].copy_(dec.pinv)
        self.dec_map[key] = slot
        self.decoders[key] = dec
        return slot

    def release(self, key: int) -> None:
        slot = self._slot_of.pop(key, None)
        self.decoders.pop(key, None)
        if slot is not None:
            self.dec_map[key] = -1
            self._free.append(slot)


def ensure_store(layer_name: str, cos_sin_cache: torch.Tensor, layout: TTKLayout | None,
                 num_blocks: int) -> TTKVRopeStore:
    st = _STORES.get(layer_name)
    if st is not None:
        return st
    if layout is None:
        raise RuntimeError(f"cannot create a TT-KV store for layer {layer_name!r}: no calibrated "
                           f"layout (point VLLM_TTKV_CALIBRATION at a calibration artifact)")
    return TTKVRopeStore(layer_name, cos_sin_cache, layout, num_blocks)


def store_for_layer(layer_name: str | None) -> TTKVRopeStore | None:
    return _STORES.get(layer_name) if layer_name else None


def register_decoder(layer_name: str, key: int, decoder: KDecoder) -> None:
    st = _STORES.get(layer_name)
    if st is None:
        raise RuntimeError(f"no TT-KV store for layer {layer_name!r}")
    st.register(key, decoder)


def decoder_for_request(layer_name: str | None, key: int) -> KDecoder | None:
    st = _STORES.get(layer_name) if layer_name else None
    return None if st is None else st.decoders.get(key)


def release_decoder(layer_name: str, key: int) -> None:
    st = _STORES.get(layer_name)
    if st is not None:
        st.release(key)


def clear_decoders() -> None:
    for st in _STORES.values():
        for k in list(st.decoders):
            st.release(k)


def clear_stores() -> None:
    _STORES.clear()
