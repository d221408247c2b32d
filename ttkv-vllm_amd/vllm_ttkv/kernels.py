"""torch-facing wrappers over the libttkv_hip C ABI.

Each wrapper validates what the host can see, allocates nothing on its own except when the
caller did not pass an output or workspace, and launches on torch's current stream. The tensors
must live on a HIP device; there is no CPU path.
"""
from __future__ import annotations

import torch

from . import _hip
from .decoder_pool import DecoderPool, decoder_ranks
from .layout import TTKLayout


def _need_device(*ts):
    ts = [u for t in ts for u in (t if isinstance(t, DecoderPool) else (t,))]
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("libttkv_hip kernels take device tensors; got a "
                               f"{t.device.type} tensor (there is no CPU implementation)")


def _i32(t, name):
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor, got {t.dtype}")
    return t


def pool_args(lay: TTKLayout, dec_pool: DecoderPool) -> tuple[int, int, int]:
    """(dec_q pointer, dec_scale pointer, slots) of a decoder pool, after checking it has the
    layout's shape: `q [slots, H*d, R]` int8 and `scale [slots, R]` fp32, both contiguous, R =
    decoder_ranks(r1) (see `decoder_pool`)."""
    if not isinstance(dec_pool, DecoderPool):
        raise TypeError("dec_pool must be a DecoderPool (a store's `dec_pool`, or "
                        "decoder_pool.pack_decoders of fp32 decoders)")
    q, sc = dec_pool
    R = decoder_ranks(lay.r1)
    if (q.dtype != torch.int8 or q.dim() != 3 or tuple(q.shape[1:]) != (lay.H * lay.d, R)
            or not q.is_contiguous()):
        raise ValueError(f"dec_pool.q must be contiguous int8 [slots, {lay.H * lay.d}, {R}], got "
                         f"{q.dtype} {tuple(q.shape)} (a decoder written at one rank cannot be "
                         f"read at another)")
    if sc.dtype != torch.float32 or tuple(sc.shape) != (q.shape[0], R) or not sc.is_contiguous():
        raise ValueError(f"dec_pool.scale must be contiguous fp32 [{q.shape[0]}, {R}], got "
                         f"{sc.dtype} {tuple(sc.shape)}")
    return q.data_ptr(), sc.data_ptr(), int(q.shape[0])


def page_bytes(page: torch.Tensor, blob: int) -> torch.Tensor:
    """`[n_slots, W]` uint8 view of a paged cache `[num_blocks, (1,) block_size, C]` in any dtype.

    The last dim of a vLLM page counts MODEL-dtype elements (decode.py:125-157), so the row is
    reinterpreted as bytes. W >= blob is accepted (vLLM rounds the row up to whole elements)."""
    u8 = page if page.dtype == torch.uint8 else page.view(torch.uint8)
    if u8.shape[-1] < blob:
        raise ValueError(f"the cache row is {u8.shape[-1]} bytes but the layout needs {blob}")
    if not u8.is_contiguous():
        raise ValueError("the cache page must be contiguous")
    return u8.reshape(-1, u8.shape[-1])


def decode_workspace(lay: TTKLayout, num_heads: int, num_reqs: int, max_seq_len: int,
                     device, block_size: int = 16) -> torch.Tensor:
    """A zero-filled workspace sized for this batch shape. Its counter region (the first 64 KiB)
    is left zero by every call, so a buffer this large serves later calls of any shape."""
    n = _hip.lib().ttkv_decode_workspace_bytes(_hip.Layout.of(lay), num_heads, num_reqs,
                                               max_seq_len, block_size)
    if n < 0:
        raise ValueError("invalid layout / head count for the decode workspace")
    return torch.zeros(max(int(n), 256), dtype=torch.uint8, device=device)


def decode_paged(lay: TTKLayout, query: torch.Tensor, page: torch.Tensor, block_size: int,
                 block_table: torch.Tensor, seq_lens: torch.Tensor,
                 query_start_loc: torch.Tensor, max_seq_len: int,
                 dec_slot_of_block: torch.Tensor, dec_pool: DecoderPool,
                 cos_sin_cache: torch.Tensor, scale: float, out: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None,
                 error_word: torch.Tensor | None = None) -> torch.Tensor:
    """K1: one launch over all decode requests. See `ttkv_decode_paged` in include/ttkv_hip.h.

    query [N, HQ, d]; page: the layer's cache (bytes reinterpreted); block_table [B, max_blocks]
    int32; seq_lens [B] int32; query_start_loc [>=B] int32 (row of request r's query);
    dec_slot_of_block [num_blocks] int32; dec_pool: the decoder pool (`DecoderPool`);
    cos_sin_cache [max_pos, d] fp32 (vLLM layout). Returns `out` [N, HQ, d] with the decode rows
    written."""
    _need_device(query, page, block_table, seq_lens, query_start_loc, dec_slot_of_block,
                 dec_pool, cos_sin_cache)
    L = _hip.lib()
    num_reqs = int(seq_lens.numel())
    N, HQ, d = query.shape
    if d != lay.d:
        raise ValueError(f"query head dim {d} != layout d {lay.d}")
    if query.stride(2) != 1 or query.stride(1) != d:
        raise ValueError("query must be contiguous within a token ([HQ, d] rows)")
    blob = lay.compressed_bytes_per_token()
    flat = page_bytes(page, blob)
    _i32(block_table, "block_table")
    _i32(seq_lens, "seq_lens")
    _i32(query_start_loc, "query_start_loc")
    _i32(dec_slot_of_block, "dec_slot_of_block")
    dq, ds, n_dec = pool_args(lay, dec_pool)
    if cos_sin_cache.dtype != torch.float32 or not cos_sin_cache.is_contiguous():
        raise ValueError("cos_sin_cache must be contiguous fp32 [max_pos, d]")
    if cos_sin_cache.shape[-1] != lay.d:
        raise NotImplementedError(
            f"rotary_dim={cos_sin_cache.shape[-1]} != head_dim={lay.d} (partial rotary) is not "
            f"supported: the kernel pairs (j, j+d/2) across the whole row")
    if out is None:
        out = torch.empty_like(query)
    if out.shape != query.shape or out.stride(2) != 1 or out.stride(1) != d:
        raise ValueError("out must match query's shape with contiguous [HQ, d] rows")
    if out.dtype not in _hip.DTYPE_CODE or query.dtype not in _hip.DTYPE_CODE:
        raise ValueError("query/out dtype must be fp32, fp16 or bf16")
    if workspace is None:
        workspace = decode_workspace(lay, HQ, num_reqs, max_seq_len, query.device, block_size)
    if error_word is None:
        error_word = torch.zeros(1, dtype=torch.int32, device=query.device)
    rc = L.ttkv_decode_paged(
        _hip.Layout.of(lay), HQ, float(scale),
        query.data_ptr(), _hip.DTYPE_CODE[query.dtype], query.stride(0),
        flat.data_ptr(), flat.shape[0], flat.stride(0),
        int(block_size), block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        seq_lens.data_ptr(), query_start_loc.data_ptr(), num_reqs, int(max_seq_len),
        dec_slot_of_block.data_ptr(), dec_slot_of_block.numel(), dq, ds, n_dec,
        cos_sin_cache.data_ptr(), cos_sin_cache.shape[0],
        out.data_ptr(), _hip.DTYPE_CODE[out.dtype], out.stride(0),
        workspace.data_ptr(), workspace.numel(), error_word.data_ptr(),
        _hip.stream_ptr(query.device))
    _hip.check(rc, "ttkv_decode_paged")
    return out


def write_paged(lay: TTKLayout, key: torch.Tensor, value: torch.Tensor,
                slot_mapping: torch.Tensor, query_start_loc: torch.Tensor,
                block_table: torch.Tensor, dec_slot_of_block: torch.Tensor,
                dec_pool: DecoderPool, pinv_pool: torch.Tensor | None, page: torch.Tensor,
                coeff_q_in: torch.Tensor | None = None,
                coeff_scale_in: torch.Tensor | None = None,
                coeff_out: torch.Tensor | None = None, resid_out: torch.Tensor | None = None,
                error_word: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None,
                dec_used: torch.Tensor | None = None) -> None:
    """K3: encode + pack `key`/`value` ([N, H, d], raw pre-RoPE keys) into their slots.

    See `ttkv_write_paged` in include/ttkv_hip.h. `pinv_pool` [slots, r1, H*d] fp32 (each decoder's pinv transposed: row a
    is rank a's projection vector) drives the
    frozen projection; `coeff_q_in`/`coeff_scale_in` replace it with a fit's coefficients.
    `dec_used` ([slots] int32, optional) receives 1 for every decoder slot a token used."""
    _need_device(key, value, slot_mapping, query_start_loc, block_table, dec_slot_of_block,
                 dec_pool, pinv_pool, page)
    N = key.shape[0]
    if key.dim() != 3 or key.shape[1:] != (lay.H, lay.d) or value.shape != key.shape:
        raise ValueError(f"key/value must be [N, {lay.H}, {lay.d}], got {tuple(key.shape)} and "
                         f"{tuple(value.shape)}")
    for t, nm in ((key, "key"), (value, "value")):
        if t.stride(2) != 1 or t.stride(1) != lay.d:
            raise ValueError(f"{nm} must be contiguous within a token")
        if t.dtype not in _hip.DTYPE_CODE:
            raise ValueError(f"{nm} dtype must be fp32, fp16 or bf16")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() < N:
        raise ValueError("slot_mapping must be int64 with one id per token")
    _i32(query_start_loc, "query_start_loc")
    _i32(block_table, "block_table")
    _i32(dec_slot_of_block, "dec_slot_of_block")
    dq, ds, n_dec = pool_args(lay, dec_pool)
    if pinv_pool is not None and (pinv_pool.dtype != torch.float32 or
                                  tuple(pinv_pool.shape[1:]) != (lay.r1, lay.H * lay.d)):
        raise ValueError("pinv_pool must be fp32 [slots, r1, H*d] (each pinv transposed)")
    flat = page_bytes(page, lay.compressed_bytes_per_token())
    if error_word is None:
        error_word = torch.zeros(1, dtype=torch.int32, device=key.device)
    if dec_used is not None:
        _i32(dec_used, "dec_used")
        if dec_used.numel() < n_dec:
            raise ValueError("dec_used needs one flag per decoder pool slot")
    cq = None
    if coeff_q_in is not None:
        if lay.qbits != 8:
            raise ValueError("coeff_q_in is the int8 mode's; the fp16 and 4-bit coefficient "
                             "modes quantise the projection themselves (pass pinv_pool)")
        cq = coeff_q_in.to(torch.int8).contiguous()
        if coeff_scale_in is None:
            raise ValueError("coeff_q_in needs coeff_scale_in (fp32)")
        coeff_scale_in = coeff_scale_in.to(torch.float32).contiguous()
    if workspace is None and cq is None:
        workspace = write_workspace(lay, N, key.device)
    rc = _hip.lib().ttkv_write_paged(
        _hip.Layout.of(lay), key.data_ptr(), _hip.DTYPE_CODE[key.dtype], key.stride(0),
        value.data_ptr(), _hip.DTYPE_CODE[value.dtype], value.stride(0),
        slot_mapping.data_ptr(), N, query_start_loc.data_ptr(), query_start_loc.numel() - 1,
        block_table.data_ptr(), block_table.stride(0), dec_slot_of_block.data_ptr(),
        dec_slot_of_block.numel(), dq, ds, _hip.ptr(pinv_pool), n_dec,
        _hip.ptr(dec_used), _hip.ptr(cq), _hip.ptr(coeff_scale_in), flat.data_ptr(),
        flat.shape[0], flat.stride(0),
        _hip.ptr(coeff_out), _hip.ptr(resid_out), _hip.ptr(workspace),
        0 if workspace is None else workspace.numel(), error_word.data_ptr(),
        _hip.stream_ptr(key.device))
    _hip.check(rc, "ttkv_write_paged")


def write_workspace(lay: TTKLayout, num_tokens: int, device) -> torch.Tensor:
    """A zero-filled workspace for `write_paged` over `num_tokens` projected tokens."""
    n = _hip.lib().ttkv_write_workspace_bytes(_hip.Layout.of(lay), int(num_tokens))
    if n < 0:
        raise ValueError("invalid layout for the write workspace")
    return torch.zeros(max(int(n), 256), dtype=torch.uint8, device=device)


def _read_checks(lay: TTKLayout, query, page, block_table, seq_lens, query_start_loc,
                 dec_slot_of_block, dec_pool, cos_sin_cache):
    """Host-visible checks shared by the read kernels (K1, K2)."""
    _need_device(query, page, block_table, seq_lens, query_start_loc, dec_slot_of_block,
                 dec_pool, cos_sin_cache)
    if query.dim() != 3 or query.shape[2] != lay.d:
        raise ValueError(f"query must be [N, num_heads, {lay.d}], got {tuple(query.shape)}")
    if query.stride(2) != 1 or query.stride(1) != lay.d:
        raise ValueError("query must be contiguous within a token ([HQ, d] rows)")
    if query.dtype not in _hip.DTYPE_CODE:
        raise ValueError("query dtype must be fp32, fp16 or bf16")
    flat = page_bytes(page, lay.compressed_bytes_per_token())
    _i32(block_table, "block_table")
    _i32(seq_lens, "seq_lens")
    _i32(query_start_loc, "query_start_loc")
    _i32(dec_slot_of_block, "dec_slot_of_block")
    pool_args(lay, dec_pool)
    if cos_sin_cache.dtype != torch.float32 or not cos_sin_cache.is_contiguous():
        raise ValueError("cos_sin_cache must be contiguous fp32 [max_pos, d]")
    if cos_sin_cache.shape[-1] != lay.d:
        raise NotImplementedError(
            f"rotary_dim={cos_sin_cache.shape[-1]} != head_dim={lay.d} (partial rotary) is not "
            f"supported: the kernels pair (j, j+d/2) across the whole row")
    return flat


def prefill_workspace(lay: TTKLayout, num_heads: int, num_reqs: int, max_q_len: int,
                      max_seq_len: int, device, block_size: int = 16) -> torch.Tensor:
    n = _hip.lib().ttkv_prefill_workspace_bytes(_hip.Layout.of(lay), num_heads, num_reqs,
                                                max_q_len, max_seq_len, block_size)
    if n < 0:
        raise ValueError("invalid layout / head count for the prefill workspace")
    return torch.zeros(max(int(n), 256), dtype=torch.uint8, device=device)


def prefill_paged(lay: TTKLayout, query: torch.Tensor, page: torch.Tensor, block_size: int,
                  block_table: torch.Tensor, seq_lens: torch.Tensor,
                  query_start_loc: torch.Tensor, max_q_len: int, max_seq_len: int,
                  dec_slot_of_block: torch.Tensor, dec_pool: DecoderPool,
                  cos_sin_cache: torch.Tensor, scale: float,
                  req_index: torch.Tensor | None = None, out: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None,
                  error_word: torch.Tensor | None = None) -> torch.Tensor:
    """K2: continuation attention for a batch of chunked-prefill requests, one launch.

    Rows `query_start_loc[r] .. [r+1]` of `query` [N, HQ, d] (post-RoPE) attend causally over the
    `seq_lens[r]` stored keys of request r (p0 = seq_len - q_len). `req_index` picks the batch
    rows to process (default: all `seq_lens.numel()`). See `ttkv_prefill_paged`."""
    flat = _read_checks(lay, query, page, block_table, seq_lens, query_start_loc,
                        dec_slot_of_block, dec_pool, cos_sin_cache)
    if req_index is not None:
        _i32(req_index, "req_index")
        num_reqs = int(req_index.numel())
    else:
        num_reqs = int(seq_lens.numel())
    N, HQ, d = query.shape
    if out is None:
        out = torch.empty_like(query)
    if out.shape != query.shape or out.stride(2) != 1 or out.stride(1) != d:
        raise ValueError("out must match query's shape with contiguous [HQ, d] rows")
    if out.dtype not in _hip.DTYPE_CODE:
        raise ValueError("out dtype must be fp32, fp16 or bf16")
    if workspace is None:
        workspace = prefill_workspace(lay, HQ, num_reqs, max_q_len, max_seq_len, query.device,
                                      block_size)
    if error_word is None:
        error_word = torch.zeros(1, dtype=torch.int32, device=query.device)
    rc = _hip.lib().ttkv_prefill_paged(
        _hip.Layout.of(lay), HQ, float(scale),
        query.data_ptr(), _hip.DTYPE_CODE[query.dtype], query.stride(0),
        flat.data_ptr(), flat.shape[0], flat.stride(0),
        int(block_size), block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        seq_lens.data_ptr(), query_start_loc.data_ptr(), _hip.ptr(req_index), num_reqs,
        int(max_q_len), int(max_seq_len),
        dec_slot_of_block.data_ptr(), dec_slot_of_block.numel(), *pool_args(lay, dec_pool),
        cos_sin_cache.data_ptr(), cos_sin_cache.shape[0],
        out.data_ptr(), _hip.DTYPE_CODE[out.dtype], out.stride(0),
        workspace.data_ptr(), workspace.numel(), error_word.data_ptr(),
        _hip.stream_ptr(query.device))
    _hip.check(rc, "ttkv_prefill_paged")
    return out


def multi_scores_paged(lay: TTKLayout, query: torch.Tensor, page: torch.Tensor,
                       block_size: int, block_table: torch.Tensor, seq_lens: torch.Tensor,
                       query_start_loc: torch.Tensor, max_q_len: int, max_seq_len: int,
                       dec_slot_of_block: torch.Tensor, dec_pool: DecoderPool,
                       cos_sin_cache: torch.Tensor, scale: float,
                       scores: torch.Tensor | None = None,
                       error_word: torch.Tensor | None = None,
                       workspace: torch.Tensor | None | bool = None) -> torch.Tensor:
    """K2 scores mode for ONE request (row 0 of block_table / seq_lens / query_start_loc):
    returns `scores` [HQ, Q, n] fp32 with -inf where key t > p0 + j (`krt_multi_from_slots`).
    Q and n are `max_q_len` / `max_seq_len`, which must equal the request's own lengths.
    `workspace`: None allocates `ttkv_multi_scores_workspace_bytes` (a chunk of two or more
    queries then reads every stored key expanded once), False runs the fused kernel."""
    flat = _read_checks(lay, query, page, block_table, seq_lens, query_start_loc,
                        dec_slot_of_block, dec_pool, cos_sin_cache)
    HQ = query.shape[1]
    if scores is None:
        scores = torch.empty(HQ, max_q_len, max_seq_len, dtype=torch.float32,
                             device=query.device)
    if (scores.dtype != torch.float32 or scores.dim() != 3 or scores.shape[0] != HQ
            or scores.shape[1] < max_q_len or scores.shape[2] < max_seq_len
            or scores.stride(2) != 1):
        raise ValueError(f"scores must be fp32 [{HQ}, >= {max_q_len}, >= {max_seq_len}] with "
                         f"contiguous key rows")
    if error_word is None:
        error_word = torch.zeros(1, dtype=torch.int32, device=query.device)
    if workspace is None:
        n = _hip.lib().ttkv_multi_scores_workspace_bytes(_hip.Layout.of(lay), HQ, int(max_q_len),
                                                         int(max_seq_len))
        if n < 0:
            raise ValueError("invalid layout / head count for the scores workspace")
        workspace = torch.empty(int(n), dtype=torch.uint8, device=query.device) if n else False
    ws_ptr, ws_bytes = (0, 0) if workspace is False else (workspace.data_ptr(), workspace.numel())
    rc = _hip.lib().ttkv_multi_scores_paged(
        _hip.Layout.of(lay), HQ, float(scale),
        query.data_ptr(), _hip.DTYPE_CODE[query.dtype], query.stride(0),
        flat.data_ptr(), flat.shape[0], flat.stride(0),
        int(block_size), block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        seq_lens.data_ptr(), query_start_loc.data_ptr(), int(max_q_len), int(max_seq_len),
        dec_slot_of_block.data_ptr(), dec_slot_of_block.numel(), *pool_args(lay, dec_pool),
        cos_sin_cache.data_ptr(), cos_sin_cache.shape[0],
        scores.data_ptr(), scores.stride(0), scores.stride(1), ws_ptr, ws_bytes,
        error_word.data_ptr(), _hip.stream_ptr(query.device))
    _hip.check(rc, "ttkv_multi_scores_paged")
    return scores


def dense_decode_paged(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       block_size: int, block_table: torch.Tensor, seq_lens: torch.Tensor,
                       query_start_loc: torch.Tensor, max_seq_len: int, scale: float,
                       out: torch.Tensor | None = None,
                       workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Benchmark comparator: dense paged decode attention over uncompressed caches
    k_cache / v_cache [n_slots, H, d] (fp16 or bf16, same dtype as query). One launch."""
    _need_device(query, k_cache, v_cache, block_table, seq_lens, query_start_loc)
    N, HQ, d = query.shape
    n_slots, H, d2 = k_cache.shape
    if d2 != d or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache / v_cache must be [n_slots, H, d] with the query's d")
    if query.dtype not in (torch.float16, torch.bfloat16) or k_cache.dtype != query.dtype \
            or v_cache.dtype != query.dtype:
        raise ValueError("dense comparator: query and caches must share fp16 or bf16")
    for t in (query, k_cache, v_cache):
        if not t.is_contiguous():
            raise ValueError("dense comparator tensors must be contiguous")
    _i32(block_table, "block_table")
    _i32(seq_lens, "seq_lens")
    _i32(query_start_loc, "query_start_loc")
    B = int(seq_lens.numel())
    if out is None:
        out = torch.empty_like(query)
    if workspace is None:
        n = _hip.lib().ttkv_dense_workspace_bytes(H, HQ, B, int(max_seq_len), int(block_size))
        workspace = torch.zeros(max(int(n), 256), dtype=torch.uint8, device=query.device)
    rc = _hip.lib().ttkv_dense_decode_paged(
        H, HQ, d, float(scale), query.data_ptr(), query.stride(0), k_cache.data_ptr(),
        v_cache.data_ptr(), _hip.DTYPE_CODE[query.dtype], n_slots, int(block_size),
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1], seq_lens.data_ptr(),
        query_start_loc.data_ptr(), B, int(max_seq_len), out.data_ptr(), out.stride(0),
        workspace.data_ptr(), workspace.numel(), _hip.stream_ptr(query.device))
    _hip.check(rc, "ttkv_dense_decode_paged")
    return out
