"""The C ABI library (libttkv_hip.so): every symbol include/ttkv_hip.h declares is exported, the
host-side geometry helper agrees with the layout, and host-checkable refusals return an error
code before any launch. No GPU compute is issued here."""
import ctypes
import pathlib
import re

import pytest

from vllm_ttkv import _hip
from vllm_ttkv.layout import CONFIGS, TTKLayout, layout_for_config

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "ttkv_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(ttkv_[a-z_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert sorted(_hip.EXPORTS) == _declared()


def test_library_exports_every_declared_symbol():
    if not _hip.lib_path().exists():
        pytest.fail(f"{_hip.lib_path()} is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(str(_hip.lib_path()))
    for name in _declared():
        assert hasattr(L, name), name


def test_blob_bytes_matches_layout():
    L = _hip.lib()
    for name, cfg in CONFIGS.items():
        for r1 in (14, 64, 110, 143):
            lay = layout_for_config(cfg, r1)
            assert L.ttkv_blob_bytes(_hip.Layout.of(lay)) == lay.compressed_bytes_per_token()
    bad = _hip.Layout(8, 100, 110, 8, 81, 3, 81, 3)
    assert L.ttkv_blob_bytes(bad) == -1


def _decode_call(lay, **kw):
    L = _hip.lib()
    args = dict(num_heads=24, scale=0.088, query=1, q_dtype=1, q_row_stride=3072, page=4096,
                n_slots=16, slot_stride=912, block_size=16, block_table=1, bt_row_stride=1,
                max_blocks=1, seq_lens=1, qsl=1, num_reqs=1, max_seq_len=16, dec_map=1,
                num_blocks=1, dec_pool=1, n_dec=1, cs=16, max_pos=64, out=1, out_dtype=1,
                out_row_stride=3072, ws=256, ws_bytes=1 << 20, err=1)
    args.update(kw)
    a = args
    return L.ttkv_decode_paged(_hip.Layout.of(lay), a["num_heads"], a["scale"], a["query"],
                               a["q_dtype"], a["q_row_stride"], a["page"], a["n_slots"],
                               a["slot_stride"], a["block_size"], a["block_table"],
                               a["bt_row_stride"], a["max_blocks"], a["seq_lens"], a["qsl"],
                               a["num_reqs"], a["max_seq_len"], a["dec_map"], a["num_blocks"],
                               a["dec_pool"], a["n_dec"], a["cs"], a["max_pos"], a["out"],
                               a["out_dtype"], a["out_row_stride"], a["ws"], a["ws_bytes"],
                               a["err"], None)


def test_host_refusals_before_launch():
    """Refused on the host, mirroring the reference's refusals (decode.py:93-118 partial rotary
    and positions past the table, decode.py:200-234 rows too short, backend.py:115-127 head
    dims). Every pointer here is a dummy: a refused call must not touch any of them."""
    L = _hip.lib()
    safe = layout_for_config(CONFIGS["safe"], 110)
    d64 = TTKLayout(H=8, d=64, r1=110, qbits=8, res_k=40, res_bits=3, v_lanes=40, v_bits=3)
    assert _decode_call(d64) == 2 and b"head dim" in L.ttkv_last_error()
    assert _decode_call(safe, num_heads=20) == 1                        # not a multiple of H
    assert _decode_call(safe, max_pos=10) == 1 and b"cos_sin_cache" in L.ttkv_last_error()
    assert _decode_call(safe, max_seq_len=17) == 1 and b"blocks" in L.ttkv_last_error()
    assert _decode_call(safe, slot_stride=900) == 1                     # narrower than the blob
    assert _decode_call(safe, page=4097) == 1                           # misaligned page
    assert _decode_call(safe, err=0) == 1                               # no error word
    big = layout_for_config(CONFIGS["safe"], 200)
    assert _decode_call(big) == 2 and b"r1" in L.ttkv_last_error()
    mixed = TTKLayout(H=8, d=128, r1=110, qbits=8, res_k=81, res_bits=3, v_lanes=64, v_bits=4)
    assert _decode_call(mixed) == 2
