"""`ttkv_decode_paged_noalloc` (K1 with its split-K scratch in a file-scope device array) through
the C ABI, against `ttkv_decode_paged` with a caller workspace on the same inputs: identical
outputs (same kernels, same work plan), on two calls in a row, the second with a smaller batch,
plus the host-side refusal of a batch whose split-K state exceeds the array. This entry point has
no counterpart in the reference; it exists for callers that cannot allocate."""
import ctypes

import pytest
import torch

from helpers import HQ, device_store, llama3_cache
from vllm_ttkv import _hip, kernels, synth

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _noalloc(st, q, cos_sin, out, err, max_len=None):
    B = st["seq_lens"].numel()
    qsl = torch.arange(B + 1, dtype=torch.int32, device="cuda")
    flat = kernels.page_bytes(st["page"], st["play"].compressed_bytes_per_token())
    max_len = int(st["seq_lens"].max()) if max_len is None else max_len
    rc = _hip.lib().ttkv_decode_paged_noalloc(
        _hip.Layout.of(st["play"]), HQ, ctypes.c_float(SCALE),
        q.data_ptr(), _hip.DTYPE_CODE[q.dtype], q.stride(0),
        flat.data_ptr(), flat.shape[0], flat.stride(0),
        st["block_size"], st["block_table"].data_ptr(), st["block_table"].stride(0),
        st["block_table"].shape[1], st["seq_lens"].data_ptr(), qsl.data_ptr(), B, max_len,
        st["dec_map"].data_ptr(), st["dec_map"].numel(), st["dec_pool"].q.data_ptr(),
        st["dec_pool"].scale.data_ptr(), st["dec_pool"].slots, cos_sin.data_ptr(),
        cos_sin.shape[0],
        out.data_ptr(), _hip.DTYPE_CODE[out.dtype], out.stride(0), err.data_ptr(),
        _hip.stream_ptr(q.device))
    return rc


def _with_workspace(st, q, cos_sin):
    B = st["seq_lens"].numel()
    out = torch.zeros(B, HQ, 128, dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    kernels.decode_paged(st["play"], q, st["page"], st["block_size"], st["block_table"],
                         st["seq_lens"], torch.arange(B + 1, dtype=torch.int32, device="cuda"),
                         int(st["seq_lens"].max()), st["dec_map"], st["dec_pool"], cos_sin,
                         SCALE, out=out, error_word=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    return out


def test_noalloc_matches_workspace_path_on_two_calls():
    cos_sin = llama3_cache(8192).cuda()
    big = device_store("safe", [3000, 1200, 5000, 700, 64, 2500, 1, 4100], seed=61)
    small = device_store("safe", [900, 40, 2000], seed=62)
    for what, st, seed in (("first call, 8 requests", big, 1), ("second call, 3 requests",
                                                                small, 2)):
        print(f"no-alloc: {what}", flush=True)
        B = st["seq_lens"].numel()
        q = synth.queries(B, seed=seed).cuda()
        out = torch.full((B, HQ, 128), float("nan"), dtype=torch.float16, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        rc = _noalloc(st, q, cos_sin, out, err)
        assert rc == 0, _hip.lib().ttkv_last_error().decode()
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        want = _with_workspace(st, q, cos_sin)
        assert torch.equal(out, want), f"{what}: outputs differ from the workspace path"


def test_noalloc_refuses_a_batch_beyond_its_scratch():
    st = device_store("safe", [64, 64], seed=63)
    q = synth.queries(2, seed=3).cuda()
    out = torch.zeros(2, HQ, 128, dtype=torch.float16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    # sized for 2 requests of 4M tokens: far more split-K state than 8 MiB; refused before launch
    rc = _noalloc(st, q, llama3_cache(128).cuda(), out, err, max_len=1 << 22)
    assert rc == 4, rc                                               # TTKV_E_WORKSPACE
    assert "no-allocation" in _hip.lib().ttkv_last_error().decode()
