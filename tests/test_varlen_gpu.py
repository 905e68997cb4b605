"""Varlen (packed) forward + backward parity on the GPU against the per-sequence
fp32 oracle (test_flash_attn.py:467-503 restated), 2x-twin bounds, and the LSE
layout [b, h, max_seqlen_q] with zero padding (flash_api.cpp:388)."""

import pytest
import torch

import flash_attention_interface as fai
from helpers import check_varlen, cu_from_lengths, randn16

CASES = [
    # lengths_q, lengths_k, h, hk, hd, causal
    ([128, 1, 300, 77], None, 4, 2, 64, True),
    ([513, 64, 129], None, 8, 2, 128, True),
    ([200, 17, 90], [100, 300, 90], 6, 3, 128, False),
    ([200, 17, 90], [100, 300, 90], 4, 1, 64, True),
    ([1, 1, 1], [50, 0, 3], 2, 2, 128, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("lens_q,lens_k,h,hk,hd,causal", CASES)
def test_varlen_parity(device, lens_q, lens_k, h, hk, hd, causal):
    lens_k = lens_k or lens_q
    g = torch.Generator().manual_seed(3000 + sum(lens_q) + hd)
    cu_q, cu_k = cu_from_lengths(lens_q), cu_from_lengths(lens_k)
    tq, tk = int(cu_q[-1]), int(cu_k[-1])
    q = randn16((tq, h, hd), g)
    k = randn16((tk, hk, hd), g)
    v = randn16((tk, hk, hd), g)
    do = randn16((tq, h, hd), g)
    s = hd ** -0.5
    mq, mk = max(lens_q), max(lens_k)
    qd, kd, vd = (t.to(device).requires_grad_() for t in (q, k, v))
    out, lse = fai._flash_attn_varlen_forward(qd, kd, vd, cu_q.to(device), cu_k.to(device), mq, mk, s, causal)
    dq, dk, dv = fai._flash_attn_varlen_backward(
        do.to(device), qd, kd, vd, out, lse, cu_q.to(device), cu_k.to(device), mq, mk, s, causal
    )
    torch.cuda.synchronize()
    assert lse.shape == (len(lens_q), h, mq)
    check_varlen("varlen", cu_q, cu_k, q, k, v, do, out.cpu(), lse.cpu(), (dq.cpu(), dk.cpu(), dv.cpu()), s, causal)


@pytest.mark.gpu
def test_varlen_public_packed_variants(device):
    g = torch.Generator().manual_seed(31)
    lens = [100, 37, 260]
    cu = cu_from_lengths(lens).to(device)
    qkv = randn16((sum(lens), 3, 4, 64), g).to(device)
    out_p = fai.flash_attn_varlen_qkvpacked_func(qkv, cu, max(lens), causal=True)
    q, k, v = (qkv[:, i] for i in range(3))
    out = fai.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal=True)
    assert torch.equal(out_p, out)
    out_kv = fai.flash_attn_varlen_kvpacked_func(q, qkv[:, 1:], cu, cu, max(lens), max(lens), causal=True)
    assert torch.equal(out_kv, out)
    # Against the oracle directly (the packed views are read in place).
    qc, kc, vc = (t.cpu() for t in (q, k, v))
    cuc = cu.cpu()
    for tag, o in (("qkvpacked", out_p), ("kvpacked", out_kv)):
        check_varlen(tag, cuc, cuc, qc, kc, vc, None, o.cpu(), None, None, 64 ** -0.5, True)


@pytest.mark.gpu
def test_varlen_packed_bwd_matches_unpacked(device):
    # Packed varlen gradients (one dqkv / dkv written slice by slice; rows past
    # the last sequence read 0) equal the unpacked path's, bit for bit.
    g = torch.Generator().manual_seed(32)
    lens = [100, 37, 260]
    cu = cu_from_lengths(lens).to(device)
    total = sum(lens) + 5  # 5 packed rows no sequence covers
    qkv = randn16((total, 3, 4, 64), g).to(device).requires_grad_()
    do = randn16((total, 4, 64), g).to(device)
    fai.flash_attn_varlen_qkvpacked_func(qkv, cu, max(lens), causal=True).backward(do)
    q, k, v = (qkv.detach()[:, i].clone().requires_grad_() for i in range(3))
    fai.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal=True).backward(do)
    for i, t in enumerate((q, k, v)):
        assert torch.equal(qkv.grad[:, i], t.grad)
    assert not qkv.grad[sum(lens):].any()
    q2 = q.detach().clone().requires_grad_()
    kv = qkv.detach()[:, 1:].clone().requires_grad_()
    fai.flash_attn_varlen_kvpacked_func(q2, kv, cu, cu, max(lens), max(lens), causal=True).backward(do)
    assert torch.equal(q2.grad, q.grad)
    assert torch.equal(kv.grad[:, 0], k.grad) and torch.equal(kv.grad[:, 1], v.grad)
    # The packed gradients against the per-sequence oracle.
    qc, kc, vc = (qkv.detach()[:, i].cpu() for i in range(3))
    grads = tuple(qkv.grad[:, i].cpu() for i in range(3))
    out = fai.flash_attn_varlen_qkvpacked_func(qkv.detach(), cu, max(lens), causal=True)
    check_varlen("qkvpacked bwd", cu.cpu(), cu.cpu(), qc, kc, vc, do.cpu(), out.cpu(), None, grads, 64 ** -0.5, True)
    kv_grads = (q2.grad.cpu(), kv.grad[:, 0].cpu(), kv.grad[:, 1].cpu())
    check_varlen("kvpacked bwd", cu.cpu(), cu.cpu(), qc, kc, vc, do.cpu(), out.cpu(), None, kv_grads, 64 ** -0.5, True)
