"""Writes small input/output vectors from the reference implementation, for the functions whose
bits the oracle's closed-form checks cannot pin:

  * the first-chunk fit, `vllm_ttkv/encode.py:257-298` (`fit_into_budget` -> `build_k_layer` ->
    `tt_svd`, codec/ttkv_codec.py:78-163), whose bits depend on the SVD;
  * the frozen encode, `vllm_ttkv/encode.py:301-351` (projection through `pinv`, coefficient
    quantisation, residual) and its torch packing (`PackedRows.build`), on the CPU;
  * the V encode, `vllm_ttkv/encode.py:431-443`, with its slot bytes (`layout.py:161-239`);
  * `PackedRows.build` on fixed (X, mask) pairs (codec/ttkv_packed_cache.py:203-231) for the three
    allocations' residual and V shapes, from fp32 and from bf16-valued inputs;
  * the attention oracle on a fitted store (`vllm_ttkv/reference.py:94-176`): `raw_scores`,
    `raw_scores_multi` with and without the causal offset, `attend_raw_store`, `oracle_attend`.

Run in the build container only, where the reference tree is mounted (it is never shipped):

    python tests/golden/make_fixtures.py /root/reference

Inputs are drawn here from a seeded generator and rounded to fp16 values (exactly representable,
so the fixture can store them as fp16); everything the reference computes from them is stored
bit-exactly. Two cases: "safe" at r1 = 16, where the fit is capped by the budget, and
"campaign4x" at r1 = 64, where the natural rank falls below the budget and the store is padded.
Outputs: tests/golden/ref_encode_<config>_r<r1>.npz, ref_packed_rows.npz, ref_attend_safe.npz.
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np
import torch


def main(ref_root: str) -> None:
    ref = pathlib.Path(ref_root)
    sys.path[:0] = [str(ref), str(ref / "codec")]
    from ttkv_codec import CONFIGS                        # noqa: E402  (reference)
    from vllm_ttkv import encode as renc                  # noqa: E402  (reference)
    from vllm_ttkv import layout as rlay                  # noqa: E402  (reference)

    for name, r1, seed in (("safe", 16, 20261201), ("campaign4x", 64, 20261202)):
        write_case(CONFIGS, renc, rlay, name, r1, seed)
    import ttkv_packed_cache as pc                         # noqa: E402  (reference)
    from vllm_ttkv import reference as rref                # noqa: E402  (reference)
    write_packed_rows(pc)
    write_attend(CONFIGS, renc, rlay, rref)


def write_packed_rows(pc) -> None:
    """PackedRows.build on fixed inputs: (rows, k, bits) of the K residual and V rows of safe
    (81 @ 3), tight (32 @ 3, 45 @ 3) and campaign4x (64 @ 4); fp32 and bf16-valued X."""
    g = torch.Generator().manual_seed(20261203)
    out = {}
    for tag, k, bits in (("k81b3", 81, 3), ("k32b3", 32, 3), ("k45b3", 45, 3), ("k64b4", 64, 4)):
        for src in ("f32", "bf16"):
            X = torch.randn(24, 128, generator=g) * 2.0
            X[3] = 0.0                                     # an all-zero row
            if src == "bf16":
                X = X.to(torch.bfloat16).float()
            idx = torch.topk(X.abs() + 1e-3 * torch.rand(24, 128, generator=g), k, dim=1).indices
            mask = torch.zeros_like(X, dtype=torch.bool).scatter_(1, idx, True)
            pr = pc.PackedRows.build(X, mask, bits, k=k, check=True)
            key = f"{tag}_{src}"
            out[f"{key}_X"] = X.numpy()
            out[f"{key}_mask"] = mask.numpy()
            out[f"{key}_bitmap"] = pr.bitmap.numpy()
            out[f"{key}_packed"] = pr.packed.numpy()
            out[f"{key}_scale"] = pr.scale.numpy()
            out[f"{key}_bits"] = np.array(bits)
            out[f"{key}_k"] = np.array(k)
    path = pathlib.Path(__file__).with_name("ref_packed_rows.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


def write_attend(CONFIGS, renc, rlay, rref) -> None:
    """The attention oracle on a fitted safe store: n = 96 rows, HQ = 24, d = 128, Q = 5."""
    torch.manual_seed(0)
    g = torch.Generator().manual_seed(20261204)
    H, d, n, HQ, Q, r1 = 8, 128, 96, 24, 5, 32
    cfg = CONFIGS["safe"]
    lay = rlay.layout_for_config(cfg, r1, H=H, d=d)
    K = torch.empty(H, n, d)
    for h in range(H):
        K[h] = torch.randn(n, 12, generator=g) @ (torch.randn(12, d, generator=g) / 12 ** 0.5)
    K = (K + 0.05 * torch.randn(H, n, d, generator=g)).half().float()
    V = torch.randn(H, n, d, generator=g).half().float()
    fk = renc.fit_into_budget(K, lay, cfg)
    k_slots = rlay.pack_k_slots(lay, fk.coeff_q, fk.coeff_scale, fk.resid)
    v_slots = rlay.pack_v_slots(lay, renc.encode_v(V, lay))
    dec = fk.decoder.decoder_f
    cos, sin = rref.rope_tables(torch.arange(n), d, theta=500000.0)
    q = torch.randn(HQ, d, generator=g).half().float()
    qm = torch.randn(HQ, Q, d, generator=g).half().float()
    p0 = n - Q
    path = pathlib.Path(__file__).with_name("ref_attend_safe.npz")
    np.savez_compressed(
        path, H=H, d=d, r1=r1, config=np.array("safe"), p0=p0,
        k_slots=k_slots.numpy(), v_slots=v_slots.numpy(), decoder_f=dec.numpy(),
        cos=cos.numpy(), sin=sin.numpy(), q=q.numpy(), qm=qm.numpy(),
        raw_scores=rref.raw_scores(lay, k_slots, dec, q, cos, sin).numpy(),
        raw_scores_multi=rref.raw_scores_multi(lay, k_slots, dec, qm, cos, sin).numpy(),
        raw_scores_multi_causal=rref.raw_scores_multi(lay, k_slots, dec, qm, cos, sin,
                                                      p0=p0).numpy(),
        attend_raw_store=rref.attend_raw_store(lay, k_slots, v_slots, dec, q, cos, sin).numpy(),
        oracle_attend=rref.oracle_attend(lay, k_slots, v_slots, dec, q, cos, sin).numpy(),
    )
    print(f"wrote {path} ({path.stat().st_size} bytes)")


def write_case(CONFIGS, renc, rlay, name: str, r1: int, seed: int) -> None:
    torch.manual_seed(0)
    g = torch.Generator().manual_seed(seed)
    H, d, n, m = 8, 128, 32, 6
    cfg = CONFIGS[name]
    lay = rlay.layout_for_config(cfg, r1, H=H, d=d)

    def keys(T):
        K = torch.empty(H, T, d)
        for h in range(H):
            Z = torch.randn(T, 12, generator=g)
            B = torch.randn(12, d, generator=g) / 12 ** 0.5
            K[h] = Z @ B + 0.05 * torch.randn(T, d, generator=g)
        K[:, :, :8] *= 8.0
        return K.half().float()

    K0 = keys(n)                                           # first chunk [H, n, d]
    K1 = keys(m)                                           # later tokens [H, m, d]
    V0 = torch.randn(H, n, d, generator=g).half().float()

    fk = renc.fit_into_budget(K0, lay, cfg)
    k_slots0 = rlay.pack_k_slots(lay, fk.coeff_q, fk.coeff_scale, fk.resid)
    ff = renc.encode_frozen(K1, fk.decoder, lay)
    k_slots1 = rlay.pack_k_slots(lay, ff.coeff_q, ff.coeff_scale, ff.resid)
    vrows = renc.encode_v(V0, lay)
    v_slots0 = rlay.pack_v_slots(lay, vrows)

    out = pathlib.Path(__file__).with_name(f"ref_encode_{name}_r{r1}.npz")
    np.savez_compressed(
        out,
        H=H, d=d, r1=r1, config=np.array(name),
        K0=K0.half().numpy(), K1=K1.half().numpy(), V0=V0.half().numpy(),
        fit_coeff_q=fk.coeff_q.numpy(), fit_coeff_scale=fk.coeff_scale.numpy(),
        fit_decoder_f=fk.decoder.decoder_f.numpy(), fit_rank=fk.fitted_rank,
        fit_k_slots=k_slots0.numpy(),
        pinv=fk.decoder.pinv.numpy(),
        frozen_coeff_q=ff.coeff_q.numpy(), frozen_coeff_scale=ff.coeff_scale.numpy(),
        frozen_resid_src=ff.resid_src.numpy(), frozen_k_slots=k_slots1.numpy(),
        v_slots=v_slots0.numpy(),
    )
    print(f"wrote {out} ({out.stat().st_size} bytes); fitted rank {fk.fitted_rank}/{r1}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
