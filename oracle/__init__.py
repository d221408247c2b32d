"""CPU oracle for the compressed-KV attention hot path.

TEST INFRASTRUCTURE ONLY. This package is a torch-CPU restatement of the reference's algorithm
(Yaweni/ttkv-vllm: `vllm_ttkv/layout.py`, `vllm_ttkv/reference.py`, `vllm_ttkv/encode.py`,
`codec/ttkv_packed_cache.py`, `codec/ttkv_codec.py`). It is imported by `tests/`, by
`__graft_entry__.smoke()` and by the `cpu_baseline` leg of `bench.py`, and by nothing else: the
product path (`ttkv-vllm_amd/vllm_ttkv`) never imports it and fails loudly when its HIP library is
missing.

Modules
  layout   -- slot geometry and pack/unpack of the per-token blob   (layout.py)
  codec    -- bit packing, bitmaps, PackedRows build/materialise,
              TT-SVD fit, the three allocations                      (ttkv_packed_cache.py, ttkv_codec.py)
  encode   -- fit_into_budget / encode_frozen / encode_v / slot write (encode.py)
  attend   -- dense reconstruction, per-row RoPE, scores, softmax,
              V readout, paged batch decode, continuation scores     (reference.py, decode.py, impl.py)
  rope     -- llama3 frequency table and vLLM's cos_sin_cache layout  (decode.py; public Llama 3 config)
  coef_modes -- fp16 and 4-bit (group-32) coefficient fields: this build's own storage modes,
              not the reference's (parity unpinned against it; pinned by closed forms, brute
              force and round trips in tests/test_coef_modes.py)

Pinning (what each part is checked against; see `tests/test_oracle_*.py`):
  * layout geometry: closed-form table of byte offsets (safe/tight/campaign4x) and the
    reference's own slot-arithmetic assertions (test_layout.py, test_decode_conventions.py).
  * bit packing / bitmaps: brute-force bit-by-bit packer on small inputs, numpy packbits, and
    round trips.
  * PackedRows.build: per-field closed forms (ruler, code range, exactly-k bitmap, zero rows)
    and a planted-mistake control.
  * scores / attention: two index orders (`attend_raw_store` vs `oracle_attend`), negative
    controls on rotation, one-hot readout, causal pattern, brute-force float64 loops.
  * TT-SVD fit and pinv projection: invariants (rank rule, exact zero padding, least squares),
    and vectors written by the reference implementation itself on the CPU
    (`tests/golden/ref_encode_*.npz`, `tests/test_golden.py`): the fit, the frozen encode and the
    V encode reproduce the reference's bytes exactly, on a capped and on a padded rank. A
    different LAPACK may still change the fit's bits; the invariants hold there.
"""
