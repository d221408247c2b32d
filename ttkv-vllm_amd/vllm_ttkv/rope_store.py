"""Per-layer state the attention layer needs: calibrated layouts, the RoPE table, and each
request's fitted decoder in a device-addressable pool.

Same surface as the reference's `vllm_ttkv/rope_store.py:70-300`: `load_calibration`,
`calibration_info`, `layout_for_layer`, `store_for_layer`, `decoder_for_layer`,
`request_key` / `request_key_host`, `register_decoder`, `decoder_for_request`, `release_decoder`,
`clear_decoders`, `TTKVRopeStore(num_heads, num_kv_heads, head_dim, cos_sin_cache, layer_name,
layout)` and `ensure_store(layer_name, cos_sin_cache, num_heads, num_kv_heads, head_dim, layout)`.

What is different underneath: a registered decoder is copied into its layer's DEVICE pool
(`dec_pool`: the codec's int8 decoder with its per-rank rulers, `q [capacity, H*d, R]` int8 +
`scale [capacity, R]` fp32, see `decoder_pool`; `pinv_pool [capacity, r1, H*d]` fp32: each decoder's pseudo-inverse by rank, the layout the
write's projection reads in whole rows) and the
request key -> pool slot map is a device array (`dec_map [num_blocks]`, -1 = none), keyed by
`block_table[r, 0]`
as in the reference (rope_store.py:148-163). The decode, continuation and write kernels resolve a
request's decoder through that map themselves, so a step needs no host read of the block table.

The pools are allocated ONCE, at a fixed capacity (argument, or `VLLM_TTKV_MAX_DECODERS`, default
64 requests per layer), and the map once the cache's block count is known. Nothing is ever
reallocated, so a HIP graph captured over the kernels keeps valid pointers for the store's
lifetime. A full pool evicts the least recently USED registration that the caller does not name
as live (the impl names the current step's requests): the write kernel flags every slot a written
token uses (`dec_used`, read back only when a registration happens), so a running request that
sits out a few steps outlives requests that finished earlier. `release_decoder` frees a finished
request's slot at once. If every slot is live, registration raises.
"""
from __future__ import annotations

import json
import os
import pathlib
import re
from collections import OrderedDict

import torch

from .decoder_pool import empty_pool
from .encode import KDecoder
from .layout import TTKLayout, config_named, layout_for_config

CONFIG_ENV = "VLLM_TTKV_CONFIG"
CAPACITY_ENV = "VLLM_TTKV_MAX_DECODERS"
DEFAULT_CAPACITY = 64

_CALIBRATED: dict[int, TTKLayout] = {}
_CALIBRATION: dict = {}
_STORES: dict[str, "TTKVRopeStore"] = {}
# registrations made before their layer's store exists; the store adopts them when it is created
_PENDING: dict[tuple[str, int], KDecoder] = {}


def _layer_index(layer_name: str):
    """Transformer block index of a vLLM layer name: the integer after a `...layers` component
    (`model.layers.7.self_attn.attn` -> 7); failing that, the last integer in the name; else
    None. (reference rope_store.py:63-67 resolves names the same way.)"""
    parts = layer_name.split(".")
    for tag, nxt in zip(parts, parts[1:]):
        if tag.endswith("layers") and nxt.isdigit():
            return int(nxt)
    found = re.findall(r"\d+", layer_name)
    return int(found[-1]) if found else None


def load_calibration(path, cfg_name: str = "safe", cfg: dict | None = None,
                     layer_prefix: str = "model.layers") -> dict:
    """Install per-layer layouts from a calibration artifact, a JSON object with `layers`,
    `heads`, `head_dim` and one rank per layer in `r1` (reference rope_store.py:70-98). Returns
    the artifact's metadata. `layer_prefix` is accepted for signature compatibility; layers are
    matched by index (`_layer_index`)."""
    global _CALIBRATION
    alloc = dict(cfg) if cfg is not None else dict(config_named(cfg_name))
    meta = json.loads(pathlib.Path(path).read_text())
    missing = [k for k in ("layers", "heads", "head_dim", "r1") if k not in meta]
    if missing:
        raise ValueError(f"calibration artifact {path} lacks {missing}")
    ranks = [int(x) for x in meta["r1"]]
    if len(ranks) != int(meta["layers"]):
        raise ValueError(f"calibration artifact {path} lists {len(ranks)} ranks for "
                         f"{meta['layers']} layers; every layer needs exactly one r1")
    table = {i: layout_for_config(alloc, rk, H=int(meta["heads"]), d=int(meta["head_dim"]))
             for i, rk in enumerate(ranks)}
    _CALIBRATED.clear()
    _CALIBRATED.update(table)
    _CALIBRATION = dict(meta)
    return _CALIBRATION


def set_layout(layer_index: int, lay: TTKLayout) -> None:
    """Install one layer's layout directly (tests, tools)."""
    _CALIBRATED[layer_index] = lay


def calibration_info() -> dict:
    return dict(_CALIBRATION)


def layout_for_layer(layer_name: str | None) -> TTKLayout | None:
    """A live store's layout when the layer has one (its decoders were fitted at that rank),
    otherwise the calibrated table's entry for the layer's index; None when neither exists (the
    caller refuses: the slot width cannot be guessed)."""
    if layer_name is None:
        return None
    if layer_name in _STORES:
        return _STORES[layer_name].layout
    idx = _layer_index(layer_name)
    return None if idx is None else _CALIBRATED.get(idx)


def store_for_layer(layer_name: str | None) -> "TTKVRopeStore | None":
    return _STORES.get(layer_name) if layer_name else None


def decoder_for_layer(layer_name: str | None):
    """The layer-level `[r1, H*d]` fp32 decoder (`store.decoder_f`), or None (reference
    rope_store.py:131-146). Used only where one decode request makes it unambiguous."""
    st = store_for_layer(layer_name)
    return None if st is None else st.decoder_f


def request_key_host(row) -> int:
    """A request's key from its block-table row already on the host: its first block id
    (reference rope_store.py:180-193)."""
    if not len(row):
        raise ValueError("empty block table row: a request with no blocks has no key")
    return int(row[0])


def request_key(block_row) -> int:
    """A request's key from its block-table row (a tensor): `block_row[0]`, the request's first
    physical block, fixed for its lifetime and computable by a kernel from the batch metadata
    (reference rope_store.py:196-207)."""
    if block_row.numel() == 0:
        raise ValueError("empty block table row: a request with no blocks has no key")
    return int(block_row.reshape(-1)[0])


class TTKVRopeStore:
    """One layer's RoPE table (fp32, vLLM layout), its layout, and its decoder pool."""

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int,
                 cos_sin_cache: torch.Tensor, layer_name: str, layout: TTKLayout, *,
                 num_blocks: int | None = None, capacity: int | None = None):
        if num_kv_heads != layout.H or head_dim != layout.d:
            raise ValueError(f"the layout is for H={layout.H}, d={layout.d}; this layer has "
                             f"{num_kv_heads} KV heads of width {head_dim}")
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads={num_heads} is not a multiple of {num_kv_heads}")
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.layer_name = layer_name
        self.layout = layout
        dev = cos_sin_cache.device
        # bf16/fp16 model tables convert to fp32 exactly; the values are the model's own
        self.cos_sin_cache = cos_sin_cache.to(torch.float32).contiguous()
        self.decoder_f: torch.Tensor | None = None   # layer-level decoder (single-request use)
        cap = int(capacity if capacity is not None else
                  os.environ.get(CAPACITY_ENV, DEFAULT_CAPACITY))
        if cap <= 0:
            raise ValueError(f"decoder pool capacity must be positive, got {cap}")
        H, d, r1 = layout.H, layout.d, layout.r1
        self.capacity = cap
        self.dec_pool = empty_pool(cap, r1, H, d, dev)
        self.pinv_pool = torch.zeros(cap, r1, H * d, dtype=torch.float32, device=dev)
        self.dec_map: torch.Tensor | None = None
        self.decoders: "OrderedDict[int, KDecoder]" = OrderedDict()  # key -> decoder, oldest first
        self._slot_of: dict[int, int] = {}
        self._free = list(range(cap - 1, -1, -1))
        # Last use: the write kernel sets dec_used[slot] = 1 for every slot a written token used
        # (every scheduled request writes every step, decode-only steps included, with no host
        # read). A registration reads the flags back (it runs in a fitting step, which
        # synchronises anyway), stamps the flagged slots with the current tick and clears them;
        # eviction then takes the least recently used slot not in the step.
        self.dec_used = torch.zeros(cap, dtype=torch.int32, device=dev)
        self._last_use: dict[int, int] = {}   # slot -> tick of its last observed use
        self._tick = 0
        if num_blocks is not None:
            self.bind_blocks(num_blocks)
        _STORES[layer_name] = self
        for (ln, key) in [k for k in _PENDING if k[0] == layer_name]:
            self.register(key, _PENDING.pop((ln, key)))

    def bind_blocks(self, num_blocks: int) -> torch.Tensor:
        """Allocate the device key -> slot map for a cache of `num_blocks` blocks (once)."""
        if self.dec_map is not None:
            if self.dec_map.numel() != num_blocks:
                raise RuntimeError(f"layer {self.layer_name!r}: the decoder map was sized for "
                                   f"{self.dec_map.numel()} blocks, the cache now has "
                                   f"{num_blocks}")
            return self.dec_map
        m = torch.full((num_blocks,), -1, dtype=torch.int32)
        for key, slot in self._slot_of.items():
            if not 0 <= key < num_blocks:
                raise IndexError(f"request key (first block) {key} outside the cache's "
                                 f"{num_blocks} blocks")
            m[key] = slot
        self.dec_map = m.to(self.pinv_pool.device)
        return self.dec_map

    def observe_use(self) -> None:
        """Fold the write kernel's use flags into the last-use record (one small read back)."""
        self._tick += 1
        used = self.dec_used.tolist()
        for slot, u in enumerate(used):
            if u:
                self._last_use[slot] = self._tick
        if any(used):
            self.dec_used.zero_()

    def eviction_order(self, live=()) -> list:
        """Registered keys that may be evicted, least recently used first as last observed
        (`observe_use`; ties: the older registration first); keys in `live` (this step's
        requests) never appear."""
        live = {int(k) for k in live}
        keys = [k for k in self.decoders if k not in live]     # registration order
        return sorted(keys, key=lambda k: self._last_use.get(self._slot_of[k], 0))

    def register(self, key: int, dec: KDecoder, live=()) -> int:
        """Copy `dec` into the pool under request key `key` and map the key to it. A key that is
        already registered keeps its slot (a recycled first block, re-fitted). When the pool is
        full, the least recently used registration whose key is not in `live` is evicted: use is
        what the write kernel flags (every scheduled request writes every step), so a running
        request that sits out a few steps outlives requests that finished before its last step."""
        key = int(key)
        lay = self.layout
        if tuple(dec.decoder_f.shape) != (lay.r1, lay.H * lay.d):
            raise ValueError(f"decoder is {tuple(dec.decoder_f.shape)}; the layout budgets "
                             f"[{lay.r1}, {lay.H * lay.d}]")
        if self.dec_map is not None and not 0 <= key < self.dec_map.numel():
            raise IndexError(f"request key (first block) {key} outside the cache's "
                             f"{self.dec_map.numel()} blocks")
        # the pool form and the pseudo-inverse first: a decoder the pool cannot hold is refused
        # before any slot is taken or evicted
        packed, pinv = dec.packed, dec.pinv
        self.observe_use()
        slot = self._slot_of.get(key)
        if slot is None:
            if not self._free:
                order = self.eviction_order(live)
                if not order:
                    raise RuntimeError(
                        f"layer {self.layer_name!r}: all {self.capacity} decoder slots belong "
                        f"to live requests; raise {CAPACITY_ENV} or release finished requests")
                self.release(order[0])
            slot = self._free.pop()
            self._slot_of[key] = slot
        self.dec_pool.q[slot].copy_(packed.q)
        self.dec_pool.scale[slot].copy_(packed.scale)
        self.pinv_pool[slot].copy_(pinv.t())
        if self.dec_map is not None:
            self.dec_map[key] = slot
        self.decoders.pop(key, None)
        self.decoders[key] = dec
        self._last_use[slot] = self._tick
        return slot

    def release(self, key: int) -> None:
        key = int(key)
        slot = self._slot_of.pop(key, None)
        self.decoders.pop(key, None)
        if slot is not None:
            if self.dec_map is not None:
                self.dec_map[key] = -1
            self._last_use.pop(slot, None)
            self._free.append(slot)


def ensure_store(layer_name: str, cos_sin_cache: torch.Tensor, num_heads: int,
                 num_kv_heads: int, head_dim: int, layout: TTKLayout | None, *,
                 num_blocks: int | None = None, capacity: int | None = None) -> TTKVRopeStore:
    """The layer's store, created on first use by the writer (reference rope_store.py:280-300).
    `num_blocks` binds the device key map if it is not bound yet. A new store's pool holds
    `VLLM_TTKV_MAX_DECODERS` decoders when that is set, else max(64, `capacity`) -- the writer
    passes the engine's `max_num_seqs`, so every running request keeps its slot."""
    st = _STORES.get(layer_name)
    if st is None:
        if layout is None:
            raise RuntimeError(f"cannot create a TT-KV store for layer {layer_name!r}: no "
                               f"calibrated layout (point VLLM_TTKV_CALIBRATION at a calibration "
                               f"artifact)")
        cap = None
        if not os.environ.get(CAPACITY_ENV) and capacity is not None:
            cap = max(DEFAULT_CAPACITY, int(capacity))
        st = TTKVRopeStore(num_heads, num_kv_heads, head_dim, cos_sin_cache, layer_name, layout,
                           capacity=cap)
    if num_blocks is not None:
        st.bind_blocks(num_blocks)
    return st


def register_decoder(layer_name: str, key: int, decoder: KDecoder, live=()) -> None:
    """Publish a request's fitted decoder for this layer (reference rope_store.py:210-219). With
    no store yet for the layer, the registration waits and the store adopts it on creation."""
    st = _STORES.get(layer_name)
    if st is None:
        _PENDING[(layer_name, int(key))] = decoder
    else:
        st.register(key, decoder, live)


def decoder_for_request(layer_name: str | None, key: int) -> KDecoder | None:
    if layer_name is None:
        return None
    st = _STORES.get(layer_name)
    if st is None:
        return _PENDING.get((layer_name, int(key)))
    return st.decoders.get(int(key))


def release_decoder(layer_name: str, key: int) -> None:
    """Drop a finished request's decoder (frees its pool slot)."""
    _PENDING.pop((layer_name, int(key)), None)
    st = _STORES.get(layer_name)
    if st is not None:
        st.release(key)


def clear_decoders() -> None:
    _PENDING.clear()
    for st in _STORES.values():
        for k in list(st.decoders):
            st.release(k)


def clear_stores() -> None:
    _PENDING.clear()
    _STORES.clear()
