"""The container-layout oracle (oracle/container.py) pinned on the CPU.

The container readers compute the slot readers' formulas over separate arrays, so the pins pack
the same container into slots and read it through the slot oracle (itself pinned by the golden
vectors in test_golden.py): scores and V readout must agree to float64 rounding. The pooled
(B > 1) row order is pinned against per-sequence calls, and a rotation that ignored the row's own
position fails the negative control (the reference's test_kernel_krt.py:97-119)."""
import pytest
import torch

from oracle import attend, codec, container
from oracle.layout import layout_for_config, pack_k_slots, pack_v_slots
from oracle.rope import cos_sin_from_cache, inv_freq_theta, vllm_cos_sin_cache

H, D, HQ = 8, 128, 32
G = HQ // H


def _store(cfg_name, n, seed, max_rank=None):
    g = torch.Generator().manual_seed(seed)
    cfg = codec.CONFIGS[cfg_name]
    K = ((torch.randn(n, 16, generator=g) * 0.2) @ (torch.randn(16, D * H, generator=g) * 0.2)
         ).reshape(n, H, D).permute(1, 0, 2).contiguous()
    K = K + 0.02 * torch.randn(H, n, D, generator=g)
    kl = codec.build_k_layer(K, cfg["tols"], cfg["qbits"], cfg["res_frac"], cfg["res_bits"],
                             max_rank=max_rank)
    V = torch.randn(H, n, D, generator=g)
    vr = codec.build_v_layer(V, cfg["k_lanes"], cfg["vbits"])
    return cfg, kl, vr


def _angles(n):
    cache = vllm_cos_sin_cache(inv_freq_theta(D, 500000.0), n + 8)
    return cos_sin_from_cache(cache, torch.arange(n), D)


@pytest.mark.parametrize("cfg_name", ["safe", "campaign4x", "tight"])
def test_container_scores_and_readout_equal_the_slot_oracle(cfg_name):
    n = 70
    cfg, kl, vr = _store(cfg_name, n, seed=3)
    cos, sin = _angles(n)
    q = torch.randn(HQ, D, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    s = container.krt(kl["coeff_q"], kl["coeff_scale"], kl["decoder_f"], kl["resid"], cos, sin,
                      q, n, H, D, kl["res_k"], cfg["res_bits"])
    lay = layout_for_config(cfg, r1=kl["r1"])
    ks = pack_k_slots(lay, kl["coeff_q"], kl["coeff_scale"], *kl["resid"])
    want = attend.raw_scores(lay, ks, kl["decoder_f"], q, cos, sin, scale=1.0,
                             dtype=torch.float64).T
    assert torch.allclose(s, want, rtol=1e-12, atol=1e-12 * want.abs().max())

    p = torch.softmax(torch.randn(HQ, n, generator=torch.Generator().manual_seed(5),
                                  dtype=torch.float64), -1)
    o = container.v_out(p, vr, n, H, D, cfg["k_lanes"], cfg["vbits"])
    vs = pack_v_slots(lay, *vr)
    Vd = attend.dense_v_from_slots(lay, vs, torch.float64)                 # [H, n, d]
    want_o = torch.einsum("pn,pnd->pd", p, Vd[torch.arange(HQ) // G])
    assert torch.allclose(o, want_o, rtol=1e-12, atol=1e-12)


def test_pooled_rows_follow_b_h_i_order():
    """B = 2 pooled: coefficients at row b*n + i, rows at b*H*n + h*n + i, one decoder each."""
    n = 40
    cfg, kl0, vr0 = _store("safe", n, seed=11)
    _, kl1, vr1 = _store("safe", n, seed=12)
    r1 = max(kl0["r1"], kl1["r1"])

    def pad(kl):
        cq = torch.zeros(n, r1, dtype=torch.int8)
        cq[:, :kl["r1"]] = kl["coeff_q"]
        dec = torch.zeros(r1, H * D)
        dec[:kl["r1"]] = kl["decoder_f"]
        return cq, dec

    cq0, d0 = pad(kl0)
    cq1, d1 = pad(kl1)
    cos, sin = _angles(n)
    q = torch.randn(2, HQ, D, generator=torch.Generator().manual_seed(13), dtype=torch.float64)
    resid = tuple(torch.cat([a, b]) for a, b in zip(kl0["resid"], kl1["resid"]))
    s = container.krt(torch.cat([cq0, cq1]), torch.cat([kl0["coeff_scale"], kl1["coeff_scale"]]),
                      torch.stack([d0, d1]), resid, cos, sin, q, n, H, D, kl0["res_k"], 3)
    for b, (cq, dec, kl) in enumerate(((cq0, d0, kl0), (cq1, d1, kl1))):
        one = container.krt(cq, kl["coeff_scale"], dec, kl["resid"], cos, sin, q[b], n, H, D,
                            kl["res_k"], 3)
        assert torch.allclose(s[b], one, rtol=1e-12, atol=1e-12 * one.abs().max())
    p = torch.rand(2, HQ, n, generator=torch.Generator().manual_seed(14), dtype=torch.float64)
    vr = tuple(torch.cat([a, b]) for a, b in zip(vr0, vr1))
    o = container.v_out(p, vr, n, H, D, 81, 3)
    for b, v in enumerate((vr0, vr1)):
        assert torch.allclose(o[b], container.v_out(p[b], v, n, H, D, 81, 3), rtol=1e-12, atol=0)


def test_rotation_uses_each_rows_own_position():
    n = 60
    cfg, kl, _ = _store("campaign4x", n, seed=21)
    cos, sin = _angles(n)
    q = torch.randn(HQ, D, generator=torch.Generator().manual_seed(22), dtype=torch.float64)
    args = (kl["coeff_q"], kl["coeff_scale"], kl["decoder_f"], kl["resid"])
    good = container.krt(*args, cos, sin, q, n, H, D, kl["res_k"], 4)
    rolled = container.krt(*args, cos.roll(1, 0), sin.roll(1, 0), q, n, H, D, kl["res_k"], 4)
    assert ((good - rolled).abs().max() / good.abs().max()) > 1e-2
