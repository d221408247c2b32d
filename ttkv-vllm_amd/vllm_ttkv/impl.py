"""`AttentionImpl` for the compressed-KV cache: write this step's raw K/V into slots, then read.

Drop-in for the reference's `TTKVAttentionImpl` (vllm_ttkv/impl.py:326-901): same constructor,
same refusals, same `forward` contract (writes into `output`; the store write happens first and
unconditionally; decodes must sit at the front of the batch). What changes is how the work is
issued:

  * the write is the HIP kernel K3 (`kernels.write_paged`) for all tokens of a step -- one launch
    for every request that already has a decoder (the kernel resolves each token's decoder from
    its request's first block through the device registry), plus a fit on the device for a
    request's first chunk;
  * the decode read is ONE K1 launch (`kernels.decode_paged`) over all decode requests of the
    layer, instead of the reference's per-request loop of ~7 launches (impl.py:468-493, 511-540);
  * a decode-only step reads nothing back to the host: the batch split comes from
    `query_start_loc_cpu`, the grid from `max_seq_len`, and the kernels read block tables,
    sequence lengths and decoder slots on the device. Device-side refusals (a block outside the
    cache, a padded slot id, a request without a decoder) set bits in `self.error_word`;
    `VLLM_TTKV_CHECK=1` makes every forward synchronise and raise on them.
  * a continuation chunk (seq_len > q_len) uses the multi-query kernel K2 over the whole store;
    a first chunk attends over its own post-RoPE q/k/v with SDPA, as in the reference
    (impl.py:684-723, decode.py:363-389).

Graph capture (uniform single-token decode steps only; the reference captures nothing,
metadata.py:96-102): a decode step's launches read only device tensors, and the buffers they hold
are never replaced. The decoder pools have a fixed capacity (`rope_store`), and the decode-step
workspaces are shared by all layers of a device and allocated at the serving limits
(`max_num_seqs` x `max_model_len`, `serving_limits`). Once a step has been captured on the
device, a step that would need more raises instead of reallocating. K1's grid is sized by the
metadata's `max_seq_len`, and its work plan follows the actual lengths on the device, so a
graph captured with `max_seq_len = max_model_len`
(`TTKVAttentionMetadataBuilder.build_for_cudagraph_capture`) is valid for every later batch of
its size. A step with prefill chunks refuses to run under capture.
"""
from __future__ import annotations

import logging
import os
from dataclasses import dataclass

import torch

from . import _hip, kernels
from . import encode as enc
from .layout import TTKLayout, config_named
from .patch import take_raw_k
from .rope_store import decoder_for_layer, ensure_store, layout_for_layer

logger = logging.getLogger("vllm.ttkv")

try:  # pragma: no cover
    from vllm.v1.attention.backend import AttentionImpl as _ImplBase
    from vllm.v1.attention.backend import AttentionType
except Exception:  # noqa: BLE001
    _ImplBase = object
    AttentionType = None

CHECK_ENV = "VLLM_TTKV_CHECK"
MAX_SEQS_ENV = "VLLM_TTKV_MAX_NUM_SEQS"
MAX_LEN_ENV = "VLLM_TTKV_MAX_MODEL_LEN"
DEFAULT_MAX_SEQS = 256


def serving_limits(fallback_len: int | None = None) -> tuple[int, int | None]:
    """(max_num_seqs, max_model_len) the fixed buffers are sized for: the environment
    (`VLLM_TTKV_MAX_NUM_SEQS`, `VLLM_TTKV_MAX_MODEL_LEN`) over the running vLLM config, else 256
    sequences and `fallback_len` (the RoPE table's length: no position beyond it has an angle)."""
    seqs = lens = None
    try:  # pragma: no cover - vLLM is not installed in the build container
        from vllm.config import get_current_vllm_config
        vc = get_current_vllm_config()
        seqs = getattr(getattr(vc, "scheduler_config", None), "max_num_seqs", None)
        lens = getattr(getattr(vc, "model_config", None), "max_model_len", None)
    except Exception:  # noqa: BLE001
        pass
    seqs = int(os.environ.get(MAX_SEQS_ENV) or seqs or DEFAULT_MAX_SEQS)
    lens = os.environ.get(MAX_LEN_ENV) or lens or fallback_len
    return seqs, (None if lens is None else int(lens))


class DeviceWorkspaces:
    """Kernel scratch for one device, shared by every layer (the layers of a step run one after
    another on one stream; each kernel leaves its counters at zero). The decode step's buffers
    (`fixed=True`) are allocated at the capacity the caller states for the serving limits. Once
    any step has been captured on this device (`frozen`), they are never replaced: a graph holds
    their addresses, and a step that needs more raises. Before that, an eager step may still
    replace them with larger ones. The prefill buffers may be replaced at any time outside
    capture (prefill steps are never captured). Nothing is allocated under capture."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.bufs: dict[str, torch.Tensor] = {}
        self.frozen = False

    def get(self, kind: str, need: int, capacity: int = 0, fixed: bool = False) -> torch.Tensor:
        buf = self.bufs.get(kind)
        if buf is not None and buf.numel() >= need:
            return buf
        if buf is not None and fixed and self.frozen:
            raise RuntimeError(
                f"the {kind} workspace ({buf.numel()} bytes, sized for the serving limits) is "
                f"held by a captured graph and cannot be replaced, but this step needs {need}; "
                f"raise {MAX_SEQS_ENV} / {MAX_LEN_ENV}")
        if _capturing():
            raise RuntimeError(f"the {kind} workspace would be allocated during graph capture; "
                               f"run one eager step of the captured shape first")
        buf = torch.zeros(max(int(need), int(capacity), 256), dtype=torch.uint8,
                          device=self.device)
        self.bufs[kind] = buf
        return buf


_WORKSPACES: dict = {}


def _capturing() -> bool:
    """Is the current stream recording a graph? (False where there is no device.)"""
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def workspaces(device) -> DeviceWorkspaces:
    """The workspaces of `device` ("cuda" means the current device)."""
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    if dev not in _WORKSPACES:
        _WORKSPACES[dev] = DeviceWorkspaces(dev)
    return _WORKSPACES[dev]


def release_workspaces() -> None:
    """Drop every device's workspaces and their frozen state. Only for when no captured graph
    that used them will be replayed again (tests, a model reload)."""
    _WORKSPACES.clear()


@dataclass
class BatchPlan:
    """Which requests decode (a leading run of q_len == 1) and where each request's tokens sit."""

    qsl: list
    n_decodes: int
    prefills: list

    @property
    def n_reqs(self) -> int:
        return len(self.qsl) - 1

    @classmethod
    def of(cls, md) -> "BatchPlan":
        if md.query_start_loc is None or md.seq_lens is None or md.block_table is None:
            raise RuntimeError("the attention metadata is missing one of `query_start_loc` / "
                               "`seq_lens` / `block_table`, so the batch cannot be split or "
                               "addressed")
        src = md.query_start_loc_cpu if md.query_start_loc_cpu is not None else md.query_start_loc
        qsl = [int(x) for x in src.tolist()]
        q_len = [qsl[i + 1] - qsl[i] for i in range(len(qsl) - 1)]
        decodes = [r for r, q in enumerate(q_len) if q == 1]
        nd = len(decodes)
        if decodes != list(range(nd)):
            raise RuntimeError(f"decode requests are not contiguous at the front of the batch "
                               f"(decode rows {decodes}, query lengths {q_len}); vLLM's reorder "
                               f"puts them there and the split relies on it")
        return cls(qsl=qsl, n_decodes=nd, prefills=[r for r, q in enumerate(q_len) if q > 1])


def as_kv_heads(x: torch.Tensor, H: int, d: int, what: str) -> torch.Tensor:
    """`[T, H*d]` or `[T, H, d]` -> `[T, H, d]` (encode.py:131-148)."""
    if x.dim() == 2:
        if x.shape[-1] != H * d:
            raise ValueError(f"{what} is [T, {x.shape[-1]}] but {H} kv heads of width {d} need "
                             f"{H * d}")
        return x.reshape(x.shape[0], H, d)
    if x.dim() == 3 and tuple(x.shape[1:]) == (H, d):
        return x
    raise ValueError(f"{what} has shape {tuple(x.shape)}; expected [T, {H}, {d}] or [T, {H * d}]")


class TTKVAttentionImpl(_ImplBase):
    def __init__(self, num_heads: int, head_size: int, scale: float,
                 num_kv_heads: int | None = None, alibi_slopes=None, sliding_window=None,
                 kv_cache_dtype: str = "auto", logits_soft_cap=None, attn_type=None,
                 kv_sharing_target_layer_name=None, **kwargs):
        if alibi_slopes is not None:
            raise NotImplementedError("TT-KV does not support ALiBi: the score kernel has no "
                                      "bias term")
        if logits_soft_cap is not None:
            raise NotImplementedError("TT-KV does not support logits_soft_cap")
        if sliding_window is not None:
            raise NotImplementedError("TT-KV does not support a sliding window: the read attends "
                                      "over the whole store")
        if kv_sharing_target_layer_name is not None:
            raise NotImplementedError("TT-KV does not support KV sharing: a shared layer would "
                                      "read another layer's store and decoder")
        if (AttentionType is not None and attn_type is not None
                and attn_type != AttentionType.DECODER):  # pragma: no cover
            raise NotImplementedError(f"TT-KV only supports decoder attention, got {attn_type!r}")
        self.num_heads = num_heads
        self.head_size = head_size
        self.num_kv_heads = num_kv_heads or num_heads
        self.scale = float(scale)
        self.kv_cache_dtype = kv_cache_dtype
        if num_heads % self.num_kv_heads:
            raise ValueError(f"num_heads={num_heads} is not a multiple of "
                             f"num_kv_heads={self.num_kv_heads}")
        self.error_word = None

    # ------------------------------------------------------------------ entry point
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        """`query`/`key` are post-RoPE (used by the first-chunk SDPA); the store is written from
        the raw key stashed by the rotary call. Writes into `output` and returns it."""
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("TT-KV does not support fused output quantization")
        if attn_metadata is None:
            if output is None:
                raise ValueError("attn_metadata and output are both None; nothing to write")
            return output.fill_(0)
        lay = self._layout(layer)
        cache = self._cache_tensor(kv_cache)
        md = attn_metadata
        plan = BatchPlan.of(md)
        N = plan.qsl[-1]
        n_tokens = query.shape[0]
        if output is None:
            output = torch.empty(n_tokens, self.num_heads, self.head_size, dtype=query.dtype,
                                 device=query.device)
        actual = getattr(md, "num_actual_tokens", None)
        if actual and int(actual) != N:
            raise RuntimeError(f"query_start_loc says {N} query tokens but num_actual_tokens "
                               f"says {actual}")
        if N > n_tokens:
            raise RuntimeError(f"metadata describes {N} query tokens but the query tensor holds "
                               f"{n_tokens}")
        if N == 0:
            return output
        if self.error_word is None or self.error_word.device != query.device:
            self.error_word = torch.zeros(1, dtype=torch.int32, device=query.device)

        if _capturing():
            if plan.prefills:
                raise RuntimeError("only uniform single-token decode steps can be captured in a "
                                   "graph; this step has prefill chunks")
            workspaces(query.device).frozen = True
        name = getattr(layer, "layer_name", None)
        stash = take_raw_k(name)                # pops: the write comes first, unconditionally
        csc = self._cos_sin_cache(layer, stash)
        self._limits = serving_limits(int(csc.shape[0]))
        store = ensure_store(name, csc, self.num_heads, self.num_kv_heads, self.head_size, lay,
                             num_blocks=int(cache.shape[0]), capacity=self._limits[0])
        self._write_store(lay, cache, stash, value, md, plan, store)

        q3 = query.view(n_tokens, self.num_heads, self.head_size)
        self._layer_decoder = getattr(layer, "ttkv_decoder_f", None)
        if plan.n_decodes:
            nd = plan.n_decodes
            self._decode(lay, cache, store, q3, md, nd, output)
        if plan.prefills:
            self._prefill(lay, cache, store, q3, key, value, md, plan, output)
        if os.environ.get(CHECK_ENV):
            torch.cuda.synchronize(query.device)
            err = int(self.error_word.item())
            if err:
                raise RuntimeError(f"vllm_ttkv: device refusal bits {err} (1 no decoder, 2 block "
                                   f"outside the cache, 4 padded/out-of-range slot id, 8 "
                                   f"seq_len beyond max_seq_len) in layer {name!r}")
        return output

    # ------------------------------------------------------------------ write
    def _write_store(self, lay, cache, stash, value, md, plan, store):
        if value is None:
            raise RuntimeError("no value tensor, so V cannot be stored")
        if lay.H != self.num_kv_heads:
            raise RuntimeError(f"the layout holds H={lay.H} head rows but this layer has "
                               f"{self.num_kv_heads} KV heads")
        N = plan.qsl[-1]
        K = as_kv_heads(stash["raw_k"], lay.H, lay.d, "the captured raw key")[:N]
        V = as_kv_heads(value, lay.H, lay.d, "value")[:N]
        if not K.is_contiguous():
            K = K.contiguous()
        if not V.is_contiguous():
            V = V.contiguous()
        slots = md.slot_mapping[:N].to(torch.int64)
        qsl_d = md.query_start_loc[:plan.n_reqs + 1].to(torch.int32)
        bt = md.block_table.to(torch.int32)
        if not plan.prefills:
            # decode-only step: every request has a decoder; one launch, no host reads
            kernels.write_paged(lay, K, V, slots, qsl_d, bt, store.dec_map, store.dec_pool,
                                store.pinv_pool, cache, error_word=self.error_word,
                                workspace=self._write_workspace(lay, N, K.device, fixed=True),
                                dec_used=store.dec_used)
            return
        # A step with prefill chunks. A request whose whole context arrives in this step
        # (seq_len == q_len) is on its first chunk and is fitted (encode.py:257-298) -- ALWAYS,
        # even when its key already has a decoder: keys are first block ids, and a finished
        # request's recycled first block must not hand its basis to the next request. The fit
        # re-registers the key (its slot is reused). Which requests start here comes from the
        # host metadata when the engine provides it (`num_computed_tokens_cpu`). Only a step that
        # fits reads the first block ids back (the fit synchronises anyway): all of them, since
        # every key of the batch is live and must survive an eviction. A continuation whose key
        # has no decoder is refused on the device (error bit 1, NaN output rows).
        first = self._first_chunks(md, plan)
        cfg = config_named(os.environ.get("VLLM_TTKV_CONFIG", "safe"))
        frozen, fitted = [], []
        keys = []
        if any(first):
            keys = [int(x) for x in md.block_table[:plan.n_reqs, 0].tolist()]
        for r in range(plan.n_reqs):
            s, e = plan.qsl[r], plan.qsl[r + 1]
            if e <= s:
                continue
            if first[r]:
                fk = enc.fit_into_budget(K[s:e].permute(1, 0, 2), lay, cfg)
                store.register(keys[r], fk.decoder, live=keys)
                fitted.append((r, fk))
            else:
                frozen.append(r)
        dev = K.device

        def launch(reqs, cq=None, cs=None):
            idx = torch.cat([torch.arange(plan.qsl[r], plan.qsl[r + 1], device=dev) for r in reqs])
            starts = [0]
            for r in reqs:
                starts.append(starts[-1] + plan.qsl[r + 1] - plan.qsl[r])
            sub_qsl = torch.tensor(starts, dtype=torch.int32, device=dev)
            rows = torch.tensor(reqs, device=dev)
            kernels.write_paged(lay, K[idx].contiguous(), V[idx].contiguous(), slots[idx], sub_qsl,
                                bt[rows].contiguous(), store.dec_map, store.dec_pool,
                                store.pinv_pool, cache, coeff_q_in=cq, coeff_scale_in=cs,
                                error_word=self.error_word, dec_used=store.dec_used,
                                workspace=None if cq is not None else
                                self._write_workspace(lay, len(idx), dev))

        if frozen:
            launch(frozen)
        if fitted and lay.qbits == 8:
            launch([r for r, _ in fitted], torch.cat([fk.coeff_q for _, fk in fitted]),
                   torch.cat([fk.coeff_scale for _, fk in fitted]))
        elif fitted:  # fp16 / 4-bit coefficients: the projection onto the new decoder
            launch([r for r, _ in fitted])

    # ------------------------------------------------------------------ read
    def _first_chunks(self, md, plan) -> list:
        """Per request: does its whole context arrive in this step (seq_len == q_len)? From
        `num_computed_tokens_cpu` when present (no device read), else from one read of
        `seq_lens`."""
        q_len = [plan.qsl[r + 1] - plan.qsl[r] for r in range(plan.n_reqs)]
        ncomp = getattr(md, "num_computed_tokens_cpu", None)
        if ncomp is not None:
            return [int(c) == 0 for c in ncomp[:plan.n_reqs].tolist()]
        seq = md.seq_lens[:plan.n_reqs].tolist()
        return [int(sl) == q for sl, q in zip(seq, q_len)]

    def _seq_lens_host(self, md, plan) -> list:
        """Exact per-request context lengths on the host: computed tokens + this step's."""
        ncomp = getattr(md, "num_computed_tokens_cpu", None)
        if ncomp is not None:
            return [int(c) + plan.qsl[r + 1] - plan.qsl[r]
                    for r, c in enumerate(ncomp[:plan.n_reqs].tolist())]
        return [int(x) for x in md.seq_lens[:plan.n_reqs].tolist()]

    def _workspace(self, lay, num_reqs, max_seq_len, block_size, device):
        L = _hip.lib()
        g = _hip.Layout.of(lay)
        need = L.ttkv_decode_workspace_bytes(g, self.num_heads, num_reqs, max_seq_len, block_size)
        seqs, lens = self._limits
        cap = L.ttkv_decode_workspace_bytes(g, self.num_heads, max(seqs, num_reqs),
                                            max(lens or 0, max_seq_len), block_size)
        return workspaces(device).get("decode", need, cap, fixed=True)

    def _write_workspace(self, lay, num_tokens, device, fixed=False):
        L = _hip.lib()
        g = _hip.Layout.of(lay)
        need = L.ttkv_write_workspace_bytes(g, num_tokens)
        if fixed:   # a decode step's tokens: one per sequence
            cap = L.ttkv_write_workspace_bytes(g, max(self._limits[0], num_tokens))
            return workspaces(device).get("decode_write", need, cap, fixed=True)
        return workspaces(device).get("prefill_write", need)

    def _prefill_workspace(self, lay, num_reqs, max_q, max_seq, device, block_size):
        need = _hip.lib().ttkv_prefill_workspace_bytes(_hip.Layout.of(lay), self.num_heads,
                                                       num_reqs, max_q, max_seq, block_size)
        return workspaces(device).get("prefill", need)

    def _decode(self, lay, cache, store, q3, md, nd, output):
        bs = self._block_size(cache)
        if nd == 1 and not _capturing():
            self._single_request_fallback(store, md)
        max_len = int(md.max_seq_len) if md.max_seq_len else int(md.seq_lens[:nd].max())
        kernels.decode_paged(lay, q3, cache, bs, md.block_table[:nd].to(torch.int32),
                             md.seq_lens[:nd].to(torch.int32),
                             md.query_start_loc[:nd + 1].to(torch.int32), max_len, store.dec_map,
                             store.dec_pool, store.cos_sin_cache, self.scale, out=output,
                             workspace=self._workspace(lay, nd, max_len, bs, q3.device),
                             error_word=self.error_word)

    def _single_request_fallback(self, store, md):
        """With ONE decode request, a layer-level decoder (`layer.ttkv_decoder_f` or
        `store.decoder_f`) is that request's decoder when none is registered under its key
        (reference impl.py:463-477, 891-901). Only when such a decoder exists is the key read
        back to the host; the ordinary path reads nothing."""
        dec = getattr(self, "_layer_decoder", None)
        if dec is None:
            dec = decoder_for_layer(store.layer_name)
        if dec is None:
            return
        key = int(md.block_table[0, 0])
        if store.decoders.get(key) is None:
            store.register(key, enc.KDecoder(dec), live=(key,))

    def _prefill(self, lay, cache, store, q3, key, value, md, plan, output):
        seq_lens = self._seq_lens_host(md, plan)
        cont = []
        for r in plan.prefills:
            s, e = plan.qsl[r], plan.qsl[r + 1]
            q_len, seq = e - s, seq_lens[r]
            if seq < q_len:
                raise RuntimeError(f"request {r} has seq_len={seq} but {q_len} query tokens")
            if seq == q_len:
                output[s:e] = self._sdpa(q3[s:e], key[s:e], value[s:e]).to(output.dtype)
            else:
                cont.append(r)
        if cont:
            # every continuation chunk of the step in one K2 launch
            max_q = max(plan.qsl[r + 1] - plan.qsl[r] for r in cont)
            max_seq = max(seq_lens[r] for r in cont)
            dev = q3.device
            kernels.prefill_paged(
                lay, q3, cache, self._block_size(cache), md.block_table.to(torch.int32),
                md.seq_lens.to(torch.int32), md.query_start_loc.to(torch.int32), max_q, max_seq,
                store.dec_map, store.dec_pool, store.cos_sin_cache, self.scale,
                req_index=torch.tensor(cont, dtype=torch.int32, device=dev), out=output,
                workspace=self._prefill_workspace(lay, len(cont), max_q, max_seq, dev,
                                                  self._block_size(cache)),
                error_word=self.error_word)

    def _sdpa(self, q, k, v):
        """First chunk: causal SDPA over the chunk's own post-RoPE q/k/v, in fp32
        (decode.py:363-389)."""
        G = self.num_heads // self.num_kv_heads
        k = as_kv_heads(k, self.num_kv_heads, self.head_size, "key").float()
        v = as_kv_heads(v, self.num_kv_heads, self.head_size, "value").float()
        T = q.shape[0]
        kk = k[:, :, None, :].expand(T, self.num_kv_heads, G, self.head_size).reshape(
            T, self.num_heads, self.head_size)
        vv = v[:, :, None, :].expand(T, self.num_kv_heads, G, self.head_size).reshape(
            T, self.num_heads, self.head_size)
        o = torch.nn.functional.scaled_dot_product_attention(
            q.float().transpose(0, 1).unsqueeze(0), kk.transpose(0, 1).unsqueeze(0),
            vv.transpose(0, 1).unsqueeze(0), is_causal=True, scale=self.scale)
        return o.squeeze(0).transpose(0, 1)

    # ------------------------------------------------------------------ resolution / guards
    def _layout(self, layer) -> TTKLayout:
        lay = getattr(layer, "ttkv_layout", None)
        if lay is None:
            lay = layout_for_layer(getattr(layer, "layer_name", None))
        if lay is None:
            raise RuntimeError(f"no TT-KV layout for layer {getattr(layer, 'layer_name', None)!r}"
                               f"; load a calibration table (VLLM_TTKV_CALIBRATION)")
        if lay.d != self.head_size:
            raise RuntimeError(f"the layout was built for head_dim={lay.d} but this layer has "
                               f"head_size={self.head_size}")
        return lay

    @staticmethod
    def _cache_tensor(kv_cache):
        if isinstance(kv_cache, (tuple, list)):
            raise RuntimeError(f"expected ONE cache tensor but got {len(kv_cache)}: K and V "
                               f"share one region per token")
        return kv_cache

    @staticmethod
    def _block_size(cache) -> int:
        if cache.dim() == 4:
            return int(cache.shape[2])
        if cache.dim() == 3:
            return int(cache.shape[1])
        raise ValueError(f"expected an LBNHC page [num_blocks, head_slots, block_size, C], got "
                         f"{tuple(cache.shape)}")

    @staticmethod
    def _cos_sin_cache(layer, stash):
        csc = stash.get("cos_sin_cache")
        if csc is None:
            csc = getattr(getattr(layer, "rotary_emb", None), "cos_sin_cache", None)
        if csc is None:
            raise RuntimeError(f"layer {getattr(layer, 'layer_name', None)!r} has no RoPE table "
                               f"(the rotary stash and layer.rotary_emb both lack one)")
        return csc
