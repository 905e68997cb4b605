"""GQA head packing in the forward and dQ kernels: a workgroup holds gp query
heads of one kv-head group (gp the largest power of two dividing the group, up
to its 32-row tiles: 4 in the 128-row forward and dQ kernels, 8 in the 256-row
ping-pong forward) at fewer positions each.  Each output row is computed
exactly as without packing, so GQA results (O, LSE, dQ) must equal, bit for
bit, MHA on K / V expanded per query head (the reference's GQA semantics,
flash_fwd_kernel.h:76 and :85: query head h reads kv head h / (h / h_k));
small shapes also go against the fp32 oracle, dK / dV included (their GQA sum
over the group is not the expanded MHA's, so only the oracle checks them)."""

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, assert_lse, check_varlen, cu_from_lengths, randn16
from oracle.attention import attention_bwd, attention_fwd, bwd_fp32_noise
from oracle.twin import bwd_twin, fwd_twin


def _expand(t, group):
    return t.repeat_interleave(group, dim=-2).contiguous()


# batch, sq, sk, h, hk, hd, causal: groups 4, 8, 12 (gp 4), 2 (gp 2), 3 (gp 1) on the
# 128-row kernel, ragged ends, sq = 1, sq != sk both ways.
SMALL = [
    (2, 100, 100, 8, 2, 128, True),
    (2, 33, 257, 16, 2, 64, True),
    (1, 257, 65, 12, 1, 128, True),
    (3, 1, 300, 8, 1, 64, False),
    (2, 190, 190, 10, 5, 128, False),
    (2, 129, 129, 6, 2, 64, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,sk,h,hk,hd,causal", SMALL)
def test_gqa_pack_small(device, b, sq, sk, h, hk, hd, causal):
    g = torch.Generator().manual_seed(9100 + sq + 3 * sk + h + hd)
    q, k, v = randn16((b, sq, h, hd), g), randn16((b, sk, hk, hd), g), randn16((b, sk, hk, hd), g)
    s = hd ** -0.5
    print(f"case gqa small b={b} sq={sq} sk={sk} h={h} hk={hk} hd={hd} causal={causal}", flush=True)
    out, lse = fai._flash_attn_forward(q.to(device), k.to(device), v.to(device), s, causal)
    out_m, lse_m = fai._flash_attn_forward(q.to(device), _expand(k, h // hk).to(device),
                                           _expand(v, h // hk).to(device), s, causal)
    torch.cuda.synchronize()
    assert torch.equal(out, out_m) and torch.equal(lse, lse_m), "packed GQA must equal expanded MHA bitwise"
    o_ref, l_ref = attention_fwd(q, k, v, s, causal)
    assert_2x("out", out.cpu(), o_ref, fwd_twin(q, k, v, s, causal)[0])
    assert_lse(lse.cpu(), l_ref)


# Full-size shapes on both kernels (the ping-pong one at 2048+ rows with a grid
# of at least twice the CU count): bitwise against expanded MHA only.
LARGE = [
    (4, 2100, 2100, 16, 2, 128, True),   # ping-pong, 8 heads x 32 positions
    (4, 2300, 1900, 16, 8, 128, True),   # ping-pong, 2 heads x 128 positions
    (2, 4096, 4096, 32, 8, 128, False),  # ping-pong, 4 heads x 64 positions
    (2, 1500, 1500, 32, 4, 128, True),   # 128-row kernel, 4 heads x 32 positions
    (4, 3000, 3000, 32, 8, 64, True),    # head_dim 64, two query tiles per wave, 4 heads x 64 positions
    (4, 2048, 2048, 16, 2, 64, True),    # head_dim 64, groups of 8: still 4 heads x 64 positions
    (4, 2048, 1900, 16, 1, 64, False),   # head_dim 64, one kv head (group 16), sq != sk
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,sk,h,hk,hd,causal", LARGE)
def test_gqa_pack_large_bitwise(device, b, sq, sk, h, hk, hd, causal):
    g = torch.Generator().manual_seed(9200 + sq + sk + h + hd)
    q = randn16((b, sq, h, hd), g).to(device)
    k, v = randn16((b, sk, hk, hd), g).to(device), randn16((b, sk, hk, hd), g).to(device)
    s = hd ** -0.5
    print(f"case gqa large b={b} sq={sq} sk={sk} h={h} hk={hk} hd={hd} causal={causal}", flush=True)
    out, lse = fai._flash_attn_forward(q, k, v, s, causal)
    out_m, lse_m = fai._flash_attn_forward(q, _expand(k, h // hk), _expand(v, h // hk), s, causal)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out, out_m) and torch.equal(lse, lse_m), "packed GQA must equal expanded MHA bitwise"


@pytest.mark.gpu
@pytest.mark.parametrize("lens_q,lens_k,h,hk,hd,causal", [
    ([300, 0, 1, 77, 31, 33], None, 16, 2, 128, True),
    ([200, 17, 90, 64], [100, 300, 90, 0], 8, 2, 64, False),
    # head_dim 64 with a grid large enough for two query tiles per wave, groups of 8
    ([1900, 1200, 2048, 700, 1500, 1000, 1800, 2000], None, 16, 2, 64, True),
])
def test_gqa_pack_varlen(device, lens_q, lens_k, h, hk, hd, causal):
    """Packed sequences with empty and one-row members: every head of a pack
    writes its own rows and its own LSE padding past the sequence end."""
    lens_k = lens_k or lens_q
    g = torch.Generator().manual_seed(9300 + sum(lens_q) + hd)
    cu_q, cu_k = cu_from_lengths(lens_q), cu_from_lengths(lens_k)
    tq, tk = int(cu_q[-1]), int(cu_k[-1])
    q, k, v = randn16((tq, h, hd), g), randn16((tk, hk, hd), g), randn16((tk, hk, hd), g)
    s = hd ** -0.5
    mq, mk = max(lens_q), max(lens_k)
    print(f"case gqa varlen lens_q={lens_q} h={h} hk={hk} hd={hd} causal={causal}", flush=True)
    out, lse = fai._flash_attn_varlen_forward(q.to(device), k.to(device), v.to(device), cu_q.to(device),
                                              cu_k.to(device), mq, mk, s, causal)
    torch.cuda.synchronize()
    check_varlen("gqa varlen", cu_q, cu_k, q, k, v, None, out.cpu(), lse.cpu(), None, s, causal)


def _fwd_bwd(q, k, v, do, s, causal):
    out, lse = fai._flash_attn_forward(q, k, v, s, causal)
    return (out, lse) + tuple(fai._flash_attn_backward(do, q, k, v, out, lse, s, causal))


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,sk,h,hk,hd,causal", SMALL)
def test_gqa_pack_dq_small(device, b, sq, sk, h, hk, hd, causal):
    g = torch.Generator().manual_seed(9400 + sq + 3 * sk + h + hd)
    q, k, v = randn16((b, sq, h, hd), g), randn16((b, sk, hk, hd), g), randn16((b, sk, hk, hd), g)
    do = randn16((b, sq, h, hd), g)
    s = hd ** -0.5
    print(f"case gqa dq small b={b} sq={sq} sk={sk} h={h} hk={hk} hd={hd} causal={causal}", flush=True)
    got = _fwd_bwd(q.to(device), k.to(device), v.to(device), do.to(device), s, causal)
    mha = _fwd_bwd(q.to(device), _expand(k, h // hk).to(device), _expand(v, h // hk).to(device), do.to(device), s,
                   causal)
    torch.cuda.synchronize()
    assert torch.equal(got[2], mha[2]), "packed GQA dQ must equal expanded MHA bitwise"
    o_ref, l_ref = attention_fwd(q, k, v, s, causal)
    g_ref = attention_bwd(q, k, v, o_ref, l_ref, do, s, causal)
    o_tw, l_tw = fwd_twin(q, k, v, s, causal)
    g_tw = bwd_twin(q, k, v, o_tw, l_tw, do, s, causal)
    noise = bwd_fp32_noise(q, k, v, o_ref, l_ref, do, s, causal)
    for name, x, r, t, n in zip(("dq", "dk", "dv"), got[2:], g_ref, g_tw, noise):
        assert_2x(name, x.cpu(), r, t, n)


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,sk,h,hk,hd,causal", [
    (4, 2100, 2100, 16, 2, 128, True),
    (2, 1500, 1700, 32, 8, 128, True),
    (2, 3000, 3000, 32, 16, 64, False),
])
def test_gqa_pack_dq_large_bitwise(device, b, sq, sk, h, hk, hd, causal):
    g = torch.Generator().manual_seed(9500 + sq + sk + h + hd)
    q, do = randn16((b, sq, h, hd), g).to(device), randn16((b, sq, h, hd), g).to(device)
    k, v = randn16((b, sk, hk, hd), g).to(device), randn16((b, sk, hk, hd), g).to(device)
    s = hd ** -0.5
    print(f"case gqa dq large b={b} sq={sq} sk={sk} h={h} hk={hk} hd={hd} causal={causal}", flush=True)
    got = _fwd_bwd(q, k, v, do, s, causal)
    mha = _fwd_bwd(q, _expand(k, h // hk), _expand(v, h // hk), do, s, causal)
    torch.cuda.synchronize()
    assert torch.isfinite(got[2]).all()
    assert torch.equal(got[2], mha[2]), "packed GQA dQ must equal expanded MHA bitwise"
    # dK / dV of the group = the expanded MHA's summed over the group's heads (fp32 sums in another order).
    for x, m in zip(got[3:], mha[3:]):
        ms = m.float().reshape(b, sk, hk, h // hk, hd).sum(3)
        assert (x.float() - ms).abs().max().item() <= 4e-3 * max(1.0, ms.abs().max().item())
