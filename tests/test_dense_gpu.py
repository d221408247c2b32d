"""The dense fp16/bf16 paged-attention comparator kernel (benchmark only) against torch fp32."""
import pytest
import torch

from vllm_ttkv import kernels, synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dense_comparator_matches_fp32_attention(dtype):
    lens = [1, 37, 700, 3000]
    H, HQ, D, BS = 8, 24, 128, 16
    bt, nblk = synth.shuffled_block_table(lens, BS, seed=4, extra_blocks=2)
    g = torch.Generator().manual_seed(0)
    kc = torch.randn(nblk * BS, H, D, generator=g).to(dtype)
    vc = torch.randn(nblk * BS, H, D, generator=g).to(dtype)
    q = torch.randn(len(lens), HQ, D, generator=g).to(dtype)
    scale = D ** -0.5
    out = kernels.dense_decode_paged(q.cuda(), kc.cuda(), vc.cuda(), BS, bt.cuda(),
                                     torch.tensor(lens, dtype=torch.int32).cuda(),
                                     torch.arange(len(lens) + 1, dtype=torch.int32).cuda(),
                                     max(lens), scale)
    torch.cuda.synchronize()
    for r, n in enumerate(lens):
        pos = torch.arange(n)
        slots = bt[r, pos // BS].long() * BS + pos % BS
        k = kc[slots].float().repeat_interleave(3, dim=1)      # [n, HQ, D]
        v = vc[slots].float().repeat_interleave(3, dim=1)
        p = torch.softmax(torch.einsum("hd,nhd->hn", q[r].float(), k) * scale, dim=-1)
        want = torch.einsum("hn,nhd->hd", p, v)
        e = (out[r].float().cpu() - want).abs().max().item()
        tol = 2e-3 if dtype == torch.float16 else 1.6e-2
        assert e <= tol, (r, n, e)


@pytest.mark.parametrize("lens", [[14402] * 3, [8258, 1581, 8579, 5467, 11927, 5395, 3922, 1263],
                                  [0, 5, 20000]])
def test_dense_comparator_ragged_and_long(lens):
    """The device work plan: long contexts split into many chunks (combined in the launch), a
    ragged batch, and an empty request (zero output)."""
    H, HQ, D, BS = 8, 24, 128, 16
    bt, nblk = synth.shuffled_block_table(lens, BS, seed=5, extra_blocks=2)
    g = torch.Generator().manual_seed(1)
    kc = torch.randn(nblk * BS, H, D, generator=g).half()
    vc = torch.randn(nblk * BS, H, D, generator=g).half()
    q = torch.randn(len(lens), HQ, D, generator=g).half()
    scale = D ** -0.5
    out = kernels.dense_decode_paged(q.cuda(), kc.cuda(), vc.cuda(), BS, bt.cuda(),
                                     torch.tensor(lens, dtype=torch.int32).cuda(),
                                     torch.arange(len(lens) + 1, dtype=torch.int32).cuda(),
                                     max(lens), scale)
    torch.cuda.synchronize()
    for r, n in enumerate(lens):
        if n == 0:
            assert torch.equal(out[r].float().cpu(), torch.zeros(HQ, D))
            continue
        pos = torch.arange(n)
        slots = bt[r, pos // BS].long() * BS + pos % BS
        k = kc[slots].float().repeat_interleave(3, dim=1)
        v = vc[slots].float().repeat_interleave(3, dim=1)
        p = torch.softmax(torch.einsum("hd,nhd->hn", q[r].float(), k) * scale, dim=-1)
        want = torch.einsum("hn,nhd->hd", p, v)
        e = (out[r].float().cpu() - want).abs().max().item()
        assert e <= 2e-3, (r, n, e)
