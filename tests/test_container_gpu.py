"""Container-layout reads (`ttkv_container_krt` / `ttkv_container_v_out`) on the GPU against the
CPU oracle (oracle/container.py), mirroring the reference's kernel tests over the same container
(test_kernel_krt.py:60-119: relative error < 1e-4 of the largest score, and a rolled-angle
negative control). Containers are built by the oracle's `build_k_layer` / `build_v_layer`
(ttkv_packed_cache.py:337-385), single and pooled (B = 2, one decoder per sequence), at 3- and
4-bit rows and ranks that take 1 to 5 MFMA k-steps."""
import pytest
import torch

from oracle import codec, container as ocont
from oracle.rope import cos_sin_from_cache, inv_freq_theta, vllm_cos_sin_cache
from vllm_ttkv import container

pytestmark = pytest.mark.gpu
H, D = 8, 128
DEV = "cuda"


def _store(cfg_name, n, seed, rank=16, noise=0.02, max_rank=None, tol=None):
    g = torch.Generator().manual_seed(seed)
    cfg = codec.CONFIGS[cfg_name]
    K = ((torch.randn(n, rank, generator=g) * 0.2) @ (torch.randn(rank, D * H, generator=g) * 0.2)
         ).reshape(n, H, D).permute(1, 0, 2).contiguous()
    K = K + noise * torch.randn(H, n, D, generator=g)
    K[:, :, :8] *= 8.0                                   # outlier channels, as the bench keys
    kl = codec.build_k_layer(K, cfg["tols"] if tol is None else tol, cfg["qbits"], cfg["res_frac"],
                             cfg["res_bits"], max_rank=max_rank)
    vr = codec.build_v_layer(torch.randn(H, n, D, generator=g), cfg["k_lanes"], cfg["vbits"])
    return cfg, kl, vr


def _angles(n):
    cache = vllm_cos_sin_cache(inv_freq_theta(D, 500000.0), n + 8)
    return cos_sin_from_cache(cache, torch.arange(n), D)


def _rows(t, bits):
    return container.PackedRows(*(x.to(DEV) for x in t), bits)


def _rel(got, want):
    return float((got.double().cpu() - want).abs().max() / want.abs().max())


@pytest.mark.parametrize("cfg_name,n,rank,max_rank,HQ", [
    ("safe", 96, 16, None, 32), ("campaign4x", 200, 16, None, 24), ("tight", 77, 16, None, 8),
    ("safe", 300, 200, 110, 24), ("campaign4x", 260, 200, 150, 32), ("safe", 130, 200, 60, 16),
    ("safe", 250, 300, 90, 24), ("campaign4x", 400, 300, 160, 24), ("tight", 300, 300, 145, 64)])
def test_krt_matches_the_oracle(cfg_name, n, rank, max_rank, HQ):
    cfg, kl, _ = _store(cfg_name, n, seed=n + HQ, rank=rank, noise=0.05, max_rank=max_rank,
                        tol=0.02 if rank >= 300 else None)
    cos, sin = _angles(n)
    q = torch.randn(HQ, D, generator=torch.Generator().manual_seed(1)) * 0.1
    dec_q, dec_scale = kl["dec_q"], kl["dec_scale"]
    s = container.krt(kl["coeff_q"].to(DEV), kl["coeff_scale"].to(DEV), dec_q.to(DEV),
                      dec_scale.to(DEV), _rows(kl["resid"], cfg["res_bits"]), cos.to(DEV),
                      sin.to(DEV), q.to(DEV), n, HQ, HQ // H, D)
    torch.cuda.synchronize()
    want = ocont.krt(kl["coeff_q"], kl["coeff_scale"], kl["decoder_f"], kl["resid"], cos, sin, q,
                     n, H, D, kl["res_k"], cfg["res_bits"])
    rel = _rel(s, want)
    print(f"{cfg_name} r1={kl['r1']} n={n} HQ={HQ}: rel {rel:.2e}")
    assert torch.isfinite(s).all()
    assert rel < 1e-4


def test_krt_pooled_batch_with_per_sequence_decoders_and_no_residual():
    n = 150
    cfg, kl0, _ = _store("safe", n, seed=31, rank=200, noise=0.05, max_rank=64)
    _, kl1, _ = _store("safe", n, seed=32, rank=200, noise=0.05, max_rank=64)
    assert kl0["r1"] == kl1["r1"] == 64
    cos, sin = _angles(n)
    HQ = 24
    q = torch.randn(2, HQ, D, generator=torch.Generator().manual_seed(2)) * 0.1
    cq = torch.cat([kl0["coeff_q"], kl1["coeff_q"]])
    cs = torch.cat([kl0["coeff_scale"], kl1["coeff_scale"]])
    dq = torch.stack([kl0["dec_q"], kl1["dec_q"]])
    ds = torch.stack([kl0["dec_scale"], kl1["dec_scale"]])
    resid = tuple(torch.cat([a, b]) for a, b in zip(kl0["resid"], kl1["resid"]))
    dec_f = torch.stack([kl0["decoder_f"], kl1["decoder_f"]])
    args = (cq.to(DEV), cs.to(DEV), dq.to(DEV), ds.to(DEV))
    s = container.krt(*args, _rows(resid, 3), cos.to(DEV), sin.to(DEV), q.to(DEV), n, HQ, 3, D)
    s0 = container.krt(*args, None, cos.to(DEV), sin.to(DEV), q.to(DEV), n, HQ, 3, D)
    torch.cuda.synchronize()
    want = ocont.krt(cq, cs, dec_f, resid, cos, sin, q, n, H, D, kl0["res_k"], 3)
    want0 = ocont.krt(cq, cs, dec_f, None, cos, sin, q, n, H, D)
    assert _rel(s, want) < 1e-4
    assert _rel(s0, want0) < 1e-4
    assert _rel(s, want0) > 1e-3                          # the residual does enter


def test_krt_rotation_is_per_row():
    """Negative control on the device (test_kernel_krt.py:97-119): rolling the angle table by one
    position must move the scores materially."""
    n = 96
    cfg, kl, _ = _store("campaign4x", n, seed=41)
    cos, sin = _angles(n)
    q = (torch.randn(32, D, generator=torch.Generator().manual_seed(3)) * 0.1).to(DEV)
    base = (kl["coeff_q"].to(DEV), kl["coeff_scale"].to(DEV), kl["dec_q"].to(DEV),
            kl["dec_scale"].to(DEV), _rows(kl["resid"], 4))
    good = container.krt(*base, cos.to(DEV), sin.to(DEV), q, n, 32, 4, D)
    rolled = container.krt(*base, cos.roll(1, 0).to(DEV), sin.roll(1, 0).to(DEV), q, n, 32, 4, D)
    torch.cuda.synchronize()
    assert float((good - rolled).abs().max() / good.abs().max()) > 1e-2


def test_krt_reads_the_first_half_of_the_angle_rows():
    """Rotate-half tables duplicate their d/2 ramp (column j == column j + d/2). Like the codec
    kernel (ttkv_kernels.cu:472-491) the launch reads columns [0, d/2) only: poisoning the second
    half leaves the scores bit-identical."""
    n = 80
    cfg, kl, _ = _store("safe", n, seed=61)
    cos, sin = _angles(n)
    assert torch.equal(cos[:, :D // 2], cos[:, D // 2:]) and torch.equal(sin[:, :D // 2], sin[:, D // 2:])
    q = (torch.randn(32, D, generator=torch.Generator().manual_seed(7)) * 0.1).to(DEV)
    base = (kl["coeff_q"].to(DEV), kl["coeff_scale"].to(DEV), kl["dec_q"].to(DEV),
            kl["dec_scale"].to(DEV), _rows(kl["resid"], 3))
    good = container.krt(*base, cos.to(DEV), sin.to(DEV), q, n, 32, 4, D)
    cp, sp = cos.clone(), sin.clone()
    cp[:, D // 2:] = float("nan")
    sp[:, D // 2:] = float("nan")
    poisoned = container.krt(*base, cp.to(DEV), sp.to(DEV), q, n, 32, 4, D)
    torch.cuda.synchronize()
    assert torch.isfinite(good).all()
    assert torch.equal(good, poisoned)


@pytest.mark.parametrize("cfg_name,B,n,HQ", [("safe", 1, 300, 24), ("campaign4x", 2, 129, 32),
                                             ("tight", 2, 64, 8), ("safe", 1, 1, 24),
                                             ("campaign4x", 3, 517, 64), ("safe", 2, 255, 16)])
def test_v_out_matches_the_oracle(cfg_name, B, n, HQ):
    cfg = codec.CONFIGS[cfg_name]
    stores = [_store(cfg_name, n, seed=50 + b)[2] for b in range(B)]
    vr = tuple(torch.cat(parts) for parts in zip(*stores))
    # weights as a slice of a wider buffer (the codec passes p_attn[:, :, :n])
    wide = torch.softmax(torch.randn(B, HQ, n + 5, generator=torch.Generator().manual_seed(6)), -1)
    p = wide.to(DEV)[:, :, :n]
    o = container.v_out(p if B > 1 else p[0], _rows(vr, cfg["vbits"]), n, HQ, HQ // H, D)
    torch.cuda.synchronize()
    want = ocont.v_out(wide[:, :, :n] if B > 1 else wide[0, :, :n], vr, n, H, D, cfg["k_lanes"],
                       cfg["vbits"])
    rel = _rel(o, want)
    print(f"v_out {cfg_name} B={B} n={n}: rel {rel:.2e}")
    assert rel < 1e-5


def test_long_sequence_walks_several_tiles_per_workgroup():
    """At 8,300 tokens each workgroup walks several tiles (krt 3 of 64 tokens, v_out 2 of 128 on
    a 256-CU part), so the next-tile prefetch and the double-buffered weights are exercised."""
    n, HQ = 8300, 24
    cfg, kl, vr = _store("safe", n, seed=71, rank=200, noise=0.05, max_rank=110)
    cos, sin = _angles(n)
    q = torch.randn(HQ, D, generator=torch.Generator().manual_seed(8)) * 0.1
    s = container.krt(kl["coeff_q"].to(DEV), kl["coeff_scale"].to(DEV), kl["dec_q"].to(DEV),
                      kl["dec_scale"].to(DEV), _rows(kl["resid"], 3), cos.to(DEV), sin.to(DEV),
                      q.to(DEV), n, HQ, HQ // H, D)
    p = torch.softmax(torch.randn(HQ, n, generator=torch.Generator().manual_seed(9)), -1)
    o = container.v_out(p.to(DEV), _rows(vr, 3), n, HQ, HQ // H, D)
    torch.cuda.synchronize()
    want = ocont.krt(kl["coeff_q"], kl["coeff_scale"], kl["decoder_f"], kl["resid"], cos, sin, q,
                     n, H, D, kl["res_k"], 3)
    want_o = ocont.v_out(p, vr, n, H, D, cfg["k_lanes"], 3)
    assert _rel(s, want) < 1e-4
    assert _rel(o, want_o) < 1e-5
