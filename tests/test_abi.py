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
                num_blocks=1, dec_q=16, dec_scale=16, n_dec=1, cs=16, max_pos=64, out=1, out_dtype=1,
                out_row_stride=3072, ws=256, ws_bytes=1 << 20, err=1)
    args.update(kw)
    a = args
    return L.ttkv_decode_paged(_hip.Layout.of(lay), a["num_heads"], a["scale"], a["query"],
                               a["q_dtype"], a["q_row_stride"], a["page"], a["n_slots"],
                               a["slot_stride"], a["block_size"], a["block_table"],
                               a["bt_row_stride"], a["max_blocks"], a["seq_lens"], a["qsl"],
                               a["num_reqs"], a["max_seq_len"], a["dec_map"], a["num_blocks"],
                               a["dec_q"], a["dec_scale"], a["n_dec"], a["cs"], a["max_pos"],
                               a["out"],
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
    assert _decode_call(safe, dec_scale=20) == 1 and b"16-byte" in L.ttkv_last_error()
    assert _decode_call(safe, dec_q=0) == 1 and b"decoder pool" in L.ttkv_last_error()
    big = layout_for_config(CONFIGS["safe"], 200)
    assert _decode_call(big) == 2 and b"r1" in L.ttkv_last_error()
    mixed = TTKLayout(H=8, d=128, r1=110, qbits=8, res_k=81, res_bits=3, v_lanes=64, v_bits=4)
    assert _decode_call(mixed) == 2


def _prefill_call(lay, **kw):
    L = _hip.lib()
    a = dict(num_heads=24, scale=0.088, query=1, q_dtype=1, q_row_stride=3072, page=4096,
             n_slots=64, slot_stride=912, block_size=16, block_table=1, bt_row_stride=4,
             max_blocks=4, seq_lens=1, qsl=1, req_index=0, num_reqs=1, max_q_len=8,
             max_seq_len=64, dec_map=1, num_blocks=4, dec_q=16, dec_scale=16, n_dec=1, cs=16,
             max_pos=64,
             out=1, out_dtype=1, out_row_stride=3072, ws=256, ws_bytes=1 << 24, err=1)
    a.update(kw)
    return L.ttkv_prefill_paged(_hip.Layout.of(lay), a["num_heads"], a["scale"], a["query"],
                                a["q_dtype"], a["q_row_stride"], a["page"], a["n_slots"],
                                a["slot_stride"], a["block_size"], a["block_table"],
                                a["bt_row_stride"], a["max_blocks"], a["seq_lens"], a["qsl"],
                                a["req_index"], a["num_reqs"], a["max_q_len"], a["max_seq_len"],
                                a["dec_map"], a["num_blocks"], a["dec_q"], a["dec_scale"],
                                a["n_dec"], a["cs"],
                                a["max_pos"], a["out"], a["out_dtype"], a["out_row_stride"],
                                a["ws"], a["ws_bytes"], a["err"], None)


def _write_call(lay, **kw):
    L = _hip.lib()
    a = dict(key=1, k_dtype=1, k_row_stride=1024, value=1, v_dtype=1, v_row_stride=1024,
             slot_mapping=1, num_tokens=4, qsl=1, num_reqs=1, block_table=1, bt_row_stride=1,
             dec_map=1, num_blocks=1, dec_q=16, dec_scale=16, pinv_pool=1, n_dec=1, dec_used=0,
             cq_in=0,
             cs_in=0,
             page=4096, n_slots=16, slot_stride=912, c_out=0, r_out=0, ws=256, ws_bytes=1 << 20,
             err=1)
    a.update(kw)
    return L.ttkv_write_paged(_hip.Layout.of(lay), a["key"], a["k_dtype"], a["k_row_stride"],
                              a["value"], a["v_dtype"], a["v_row_stride"], a["slot_mapping"],
                              a["num_tokens"], a["qsl"], a["num_reqs"], a["block_table"],
                              a["bt_row_stride"], a["dec_map"], a["num_blocks"], a["dec_q"],
                              a["dec_scale"], a["pinv_pool"], a["n_dec"], a["dec_used"], a["cq_in"],
                              a["cs_in"], a["page"],
                              a["n_slots"], a["slot_stride"], a["c_out"], a["r_out"], a["ws"],
                              a["ws_bytes"], a["err"], None)


def test_prefill_host_refusals_before_launch():
    """K2's host refusals (the continuation read, impl.py:725-778): geometry it is not built for,
    a causal chunk longer than the store, positions past the angle table, a block table too
    short for the context, and missing outputs. Dummy pointers only: nothing is launched."""
    L = _hip.lib()
    safe = layout_for_config(CONFIGS["safe"], 110)
    d64 = TTKLayout(H=8, d=64, r1=110, qbits=8, res_k=40, res_bits=3, v_lanes=40, v_bits=3)
    assert _prefill_call(d64) == 2 and b"head dim" in L.ttkv_last_error()
    assert _prefill_call(safe, num_heads=20) == 1
    assert _prefill_call(safe, max_q_len=65) == 1 and b"max_q_len" in L.ttkv_last_error()
    assert _prefill_call(safe, max_pos=10) == 1 and b"cos_sin_cache" in L.ttkv_last_error()
    assert _prefill_call(safe, max_blocks=2) == 1 and b"blocks" in L.ttkv_last_error()
    assert _prefill_call(safe, out=0) == 1 and b"out" in L.ttkv_last_error()
    assert _prefill_call(safe, cs=17) == 1 and b"16-aligned" in L.ttkv_last_error()
    assert _prefill_call(layout_for_config(CONFIGS["safe"], 200)) == 2
    assert _prefill_call(safe, q_dtype=7) == 1 and b"dtype" in L.ttkv_last_error()
    assert _prefill_call(safe, dec_q=24) == 1 and b"16-byte" in L.ttkv_last_error()


def test_write_host_refusals_before_launch():
    """K3's host refusals (encode.py:446-468 slot checks stay on the device; these are the
    geometry and argument checks): nothing is launched."""
    L = _hip.lib()
    safe = layout_for_config(CONFIGS["safe"], 110)
    d64 = TTKLayout(H=8, d=64, r1=110, qbits=8, res_k=40, res_bits=3, v_lanes=40, v_bits=3)
    assert _write_call(d64) == 2 and b"head dim" in L.ttkv_last_error()
    h16 = TTKLayout(H=16, d=128, r1=110, qbits=8, res_k=81, res_bits=3, v_lanes=81, v_bits=3)
    assert _write_call(h16) == 2 and b"H > 8" in L.ttkv_last_error()
    assert _write_call(layout_for_config(CONFIGS["safe"], 300)) == 2
    assert _write_call(safe, pinv_pool=0) == 1 and b"pinv_pool" in L.ttkv_last_error()
    assert _write_call(safe, pinv_pool=0, cq_in=1) == 1 and b"coeff_scale_in" in L.ttkv_last_error()
    assert _write_call(safe, slot_stride=800) == 1 and b"slot stride" in L.ttkv_last_error()
    assert _write_call(safe, key=0) == 1 and b"null" in L.ttkv_last_error()
    assert _write_call(safe, v_dtype=5) == 1 and b"dtype" in L.ttkv_last_error()
    assert _write_call(safe, ws=0) == 4 and b"workspace" in L.ttkv_last_error()
    assert _write_call(safe, dec_q=8) == 1 and b"16-byte aligned" in L.ttkv_last_error()
    assert _write_call(safe, dec_scale=0) == 1 and b"decoder pool" in L.ttkv_last_error()
    assert _write_call(safe, num_tokens=0) == 0                          # nothing to do


def test_container_host_refusals_before_launch():
    """The container reads' host refusals: geometry they are not built for, missing arrays and
    weight strides smaller than [B, HQ, n]. Dummy pointers only: nothing is launched."""
    L = _hip.lib()

    def krt(**kw):
        a = dict(H=8, HQ=24, d=128, B=1, n=64, r1=110, cq=16, cs=16, dec=16, per=0, bm=16,
                 pk=16, rs=16, pb=31, bits=3, cos=16, sin=16, q=16, s=16)
        a.update(kw)
        return L.ttkv_container_krt(a["H"], a["HQ"], a["d"], a["B"], a["n"], a["r1"], a["cq"],
                                    a["cs"], a["dec"], a["per"], a["bm"], a["pk"], a["rs"],
                                    a["pb"], a["bits"], a["cos"], a["sin"], a["q"], a["s"], None)

    def vout(**kw):
        a = dict(H=8, HQ=24, d=128, B=1, n=64, p=16, ph=64, pbs=24 * 64, bm=16, pk=16, rs=16,
                 pb=31, bits=3, o=16)
        a.update(kw)
        return L.ttkv_container_v_out(a["H"], a["HQ"], a["d"], a["B"], a["n"], a["p"], a["ph"],
                                      a["pbs"], a["bm"], a["pk"], a["rs"], a["pb"], a["bits"],
                                      a["o"], None)

    assert krt(d=64) == 2 and b"head dim" in L.ttkv_last_error()
    assert krt(HQ=20) == 1
    assert krt(r1=161) == 2 and b"r1" in L.ttkv_last_error()
    assert krt(pb=49) == 2 and b"packed row" in L.ttkv_last_error()
    assert krt(bits=5) == 2
    assert krt(q=0) == 1 and b"null" in L.ttkv_last_error()
    assert krt(pk=0) == 1 and b"residual" in L.ttkv_last_error()
    assert krt(cos=8) == 1 and b"aligned" in L.ttkv_last_error()
    assert krt(q=24) == 1 and b"aligned" in L.ttkv_last_error()
    assert krt(HQ=40, H=8) == 2                                    # 5 heads per KV head
    assert krt(n=0) == 0                                           # nothing to do
    assert vout(ph=63) == 1 and b"strides" in L.ttkv_last_error()
    assert vout(o=0) == 1
    assert vout(bits=2) == 2


def test_header_compiles_as_plain_c(tmp_path):
    """include/ttkv_hip.h is a C header (no C++ or HIP types): a C99 translation unit that
    includes it and takes every entry point's address compiles with gcc."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not installed")
    src = tmp_path / "use_header.c"
    refs = "\n".join(f"  (entry_fn){name}," for name in _declared())
    src.write_text('#include "ttkv_hip.h"\n'
                   "typedef void (*entry_fn)(void);\n"
                   "entry_fn entry_points[] = {\n" + refs + "\n};\n")
    r = subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-pedantic", "-fsyntax-only",
                        "-I", str(HEADER.parent), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
