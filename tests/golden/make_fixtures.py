"""Writes small input/output vectors from the reference implementation, for the functions whose
bits the oracle's closed-form checks cannot pin:

  * the first-chunk fit, `vllm_ttkv/encode.py:257-298` (`fit_into_budget` -> `build_k_layer` ->
    `tt_svd`, codec/ttkv_codec.py:78-163), whose bits depend on the SVD;
  * the frozen encode, `vllm_ttkv/encode.py:301-351` (projection through `pinv`, coefficient
    quantisation, residual) and its torch packing (`PackedRows.build`), on the CPU;
  * the V encode, `vllm_ttkv/encode.py:431-443`, with its slot bytes (`layout.py:161-239`).

Run in the build container only, where the reference tree is mounted (it is never shipped):

    python tests/golden/make_fixtures.py /root/reference

Inputs are drawn here from a seeded generator and rounded to fp16 values (exactly representable,
so the fixture can store them as fp16); everything the reference computes from them is stored
bit-exactly. Two cases: "safe" at r1 = 16, where the fit is capped by the budget, and
"campaign4x" at r1 = 64, where the natural rank falls below the budget and the store is padded.
Output: tests/golden/ref_encode_<config>_r<r1>.npz.
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
