"""ctypes binding of libttkv_hip.so (the C ABI declared in include/ttkv_hip.h).

This is the only way the package reaches the GPU kernels. There is no fallback: if the library is
missing or a call fails, a RuntimeError names the reason. Tensors cross the boundary as raw
`data_ptr()`s plus sizes, launched on torch's current HIP stream -- the same pattern the reference
uses for its CUDA path (codec/cuda_driver.py:164-175), with the delivery swapped for an AOT gfx950
shared object.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import torch

LIB_NAME = "libttkv_hip.so"
_LIB = None

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

ERR_NO_DECODER = 1
ERR_BAD_BLOCK = 2
ERR_BAD_SLOT = 4
ERR_SEQ_LEN = 8


class Layout(ctypes.Structure):
    """`ttkv_layout` -- TTKLayout's eight defining integers."""
    _fields_ = [(n, ctypes.c_int32) for n in
                ("H", "d", "r1", "qbits", "res_k", "res_bits", "v_lanes", "v_bits")]

    @classmethod
    def of(cls, lay) -> "Layout":
        return cls(lay.H, lay.d, lay.r1, lay.qbits, lay.res_k, lay.res_bits, lay.v_lanes,
                   lay.v_bits)


def lib_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get("TTKV_HIP_LIB",
                                       pathlib.Path(__file__).with_name(LIB_NAME)))


def lib():
    """The loaded library, loading it on first use. Raises if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    p = lib_path()
    if not p.exists():
        raise RuntimeError(
            f"{p} is not built. The compressed-KV attention path has no non-HIP implementation; "
            f"build it with `python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950).")
    L = ctypes.CDLL(str(p))
    P, I32, I64, F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    LP = ctypes.POINTER(Layout)
    L.ttkv_last_error.restype = ctypes.c_char_p
    L.ttkv_last_error.argtypes = []
    L.ttkv_decoder_ranks.restype = I32
    L.ttkv_decoder_ranks.argtypes = [I32]
    L.ttkv_blob_bytes.restype = I64
    L.ttkv_blob_bytes.argtypes = [LP]
    L.ttkv_decode_workspace_bytes.restype = I64
    L.ttkv_decode_workspace_bytes.argtypes = [LP, I32, I32, I32, I32]
    L.ttkv_decode_paged.restype = ctypes.c_int
    L.ttkv_decode_paged.argtypes = [
        LP, I32, F32,                 # layout, num_heads, scale
        P, I32, I64,                  # query, q_dtype, q_row_stride
        P, I64, I64,                  # page, n_slots, slot_stride
        I32, P, I64, I32,             # block_size, block_table, bt_row_stride, max_blocks
        P, P, I32, I32,               # seq_lens, query_start_loc, num_reqs, max_seq_len
        P, I64,                       # dec_slot_of_block, num_blocks
        P, P, I64,                    # dec_q, dec_scale, n_dec_slots
        P, I64,                       # cos_sin_cache, max_position
        P, I32, I64,                  # out, out_dtype, out_row_stride
        P, I64, P,                    # workspace, workspace_bytes, error_word
        P,                            # stream
    ]
    L.ttkv_decode_paged_noalloc.restype = ctypes.c_int
    L.ttkv_decode_paged_noalloc.argtypes = [
        LP, I32, F32,                 # layout, num_heads, scale
        P, I32, I64,                  # query, q_dtype, q_row_stride
        P, I64, I64,                  # page, n_slots, slot_stride
        I32, P, I64, I32,             # block_size, block_table, bt_row_stride, max_blocks
        P, P, I32, I32,               # seq_lens, query_start_loc, num_reqs, max_seq_len
        P, I64,                       # dec_slot_of_block, num_blocks
        P, P, I64,                    # dec_q, dec_scale, n_dec_slots
        P, I64,                       # cos_sin_cache, max_position
        P, I32, I64,                  # out, out_dtype, out_row_stride
        P,                            # error_word
        P,                            # stream
    ]
    L.ttkv_write_paged.restype = ctypes.c_int
    L.ttkv_write_paged.argtypes = [
        LP, P, I32, I64,              # layout, key, k_dtype, k_row_stride
        P, I32, I64,                  # value, v_dtype, v_row_stride
        P, I32, P, I32,               # slot_mapping, num_tokens, query_start_loc, num_reqs
        P, I64, P, I64,               # block_table, bt_row_stride, dec_slot_of_block, num_blocks
        P, P, P, I64, P,              # dec_q, dec_scale, pinv_pool, n_dec_slots, dec_slot_used
        P, P,                         # coeff_q_in, coeff_scale_in
        P, I64, I64,                  # page, n_slots, slot_stride
        P, P,                         # coeff_out, resid_out
        P, I64, P, P,                 # workspace, workspace_bytes, error_word, stream
    ]
    L.ttkv_write_workspace_bytes.restype = I64
    L.ttkv_write_workspace_bytes.argtypes = [LP, I32]
    L.ttkv_prefill_workspace_bytes.restype = I64
    L.ttkv_prefill_workspace_bytes.argtypes = [LP, I32, I32, I32, I32, I32]
    L.ttkv_prefill_paged.restype = ctypes.c_int
    L.ttkv_prefill_paged.argtypes = [
        LP, I32, F32,                 # layout, num_heads, scale
        P, I32, I64,                  # query, q_dtype, q_row_stride
        P, I64, I64,                  # page, n_slots, slot_stride
        I32, P, I64, I32,             # block_size, block_table, bt_row_stride, max_blocks
        P, P, P,                      # seq_lens, query_start_loc, req_index
        I32, I32, I32,                # num_reqs, max_q_len, max_seq_len
        P, I64,                       # dec_slot_of_block, num_blocks
        P, P, I64,                    # dec_q, dec_scale, n_dec_slots
        P, I64,                       # cos_sin_cache, max_position
        P, I32, I64,                  # out, out_dtype, out_row_stride
        P, I64, P,                    # workspace, workspace_bytes, error_word
        P,                            # stream
    ]
    L.ttkv_multi_scores_paged.restype = ctypes.c_int
    L.ttkv_multi_scores_paged.argtypes = [
        LP, I32, F32,                 # layout, num_heads, scale
        P, I32, I64,                  # query, q_dtype, q_row_stride
        P, I64, I64,                  # page, n_slots, slot_stride
        I32, P, I64, I32,             # block_size, block_table, bt_row_stride, max_blocks
        P, P, I32, I32,               # seq_lens, query_start_loc, max_q_len, max_seq_len
        P, I64,                       # dec_slot_of_block, num_blocks
        P, P, I64,                    # dec_q, dec_scale, n_dec_slots
        P, I64,                       # cos_sin_cache, max_position
        P, I64, I64,                  # scores, s_head_stride, s_q_stride
        P, I64, P, P,                 # workspace, workspace_bytes, error_word, stream
    ]
    L.ttkv_multi_scores_workspace_bytes.restype = I64
    L.ttkv_multi_scores_workspace_bytes.argtypes = [LP, I32, I32, I32]
    L.ttkv_dense_workspace_bytes.restype = I64
    L.ttkv_dense_workspace_bytes.argtypes = [I32, I32, I32, I32, I32]
    L.ttkv_dense_decode_paged.restype = ctypes.c_int
    L.ttkv_dense_decode_paged.argtypes = [
        I32, I32, I32, F32,           # H, num_heads, d, scale
        P, I64, P, P, I32, I64,       # query, q_row_stride, k_cache, v_cache, dtype, n_slots
        I32, P, I64, I32,             # block_size, block_table, bt_row_stride, max_blocks
        P, P, I32, I32,               # seq_lens, query_start_loc, num_reqs, max_seq_len
        P, I64, P, I64, P,            # out, out_row_stride, workspace, workspace_bytes, stream
    ]
    L.ttkv_container_krt.restype = ctypes.c_int
    L.ttkv_container_krt.argtypes = [
        I32, I32, I32, I32, I32, I32,  # H, num_heads, d, B, n, r1
        P, P, P, I32,                 # coeff_q, coeff_scale, decoder_f, decoder_per_seq
        P, P, P, I32, I32,            # res_bitmap, res_packed, res_scale, res_pb, res_bits
        P, P, P, P, P,                # cos, sin, query, scores, stream
    ]
    L.ttkv_container_v_out.restype = ctypes.c_int
    L.ttkv_container_v_out.argtypes = [
        I32, I32, I32, I32, I32,      # H, num_heads, d, B, n
        P, I64, I64,                  # p, p_head_stride, p_batch_stride
        P, P, P, I32, I32,            # v_bitmap, v_packed, v_scale, v_pb, v_bits
        P, P,                         # out, stream
    ]
    for name in EXPORTS:
        getattr(L, name)  # every declared symbol must resolve
    _LIB = L
    return L


# Every symbol include/ttkv_hip.h declares (checked by tests/test_abi.py).
EXPORTS = ("ttkv_last_error", "ttkv_decoder_ranks", "ttkv_blob_bytes",
           "ttkv_decode_workspace_bytes", "ttkv_decode_paged", "ttkv_decode_paged_noalloc",
           "ttkv_write_paged", "ttkv_prefill_workspace_bytes", "ttkv_prefill_paged", "ttkv_multi_scores_paged", "ttkv_multi_scores_workspace_bytes",
           "ttkv_dense_workspace_bytes",
           "ttkv_dense_decode_paged", "ttkv_write_workspace_bytes", "ttkv_container_krt",
           "ttkv_container_v_out")


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().ttkv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def stream_ptr(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
