"""Backward parity on the GPU: dQ, dK, dV from the HIP kernels (through
torch.autograd and the drop-in interface) vs the fp32 closed-form oracle,
bounded by 2x the reference kernel's own error (rounding-point twin of
flash_bwd_kernel.h / flash_api.cpp:338-348 including its GQA fp16 sum)."""

import itertools

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, randn16
from oracle.attention import attention_bwd, attention_fwd, bwd_fp32_noise
from oracle.twin import bwd_twin, fwd_twin

SEQLENS = [(1, 1), (37, 1), (63, 65), (128, 128), (127, 129), (257, 190), (190, 257), (512, 512), (700, 1025)]
HEADS = [(2, 1), (6, 3), (4, 4), (6, 1)]
SCALES = [None, 0.3]

CASES = [
    (hd, causal, sq, sk, HEADS[i % len(HEADS)], 1 + 2 * (i % 2), SCALES[i % len(SCALES)])
    for i, (hd, causal, (sq, sk)) in enumerate(itertools.product([64, 128], [False, True], SEQLENS))
]
# More of the reference's (sq, sk) pairs (test_flash_attn.py:59-140), batch 1.
EXTRA_SEQLENS = [(113, 203), (1, 1025), (1024, 1023), (897, 1025), (1536, 1536)]
CASES += [
    (128 if i % 2 == 0 else 64, i != 1, sq, sk, HEADS[i % len(HEADS)], 1, SCALES[i % len(SCALES)])
    for i, (sq, sk) in enumerate(EXTRA_SEQLENS)
]


def _oracles(q, k, v, do, s, causal):
    o_ref, l_ref = attention_fwd(q, k, v, s, causal)
    grads_ref = attention_bwd(q, k, v, o_ref, l_ref, do, s, causal)
    o_tw, l_tw = fwd_twin(q, k, v, s, causal)
    grads_tw = bwd_twin(q, k, v, o_tw, l_tw, do, s, causal)
    noise = bwd_fp32_noise(q, k, v, o_ref, l_ref, do, s, causal)
    return grads_ref, grads_tw, noise


def _check_grads(tag, q, k, v, do, grads, s, causal):
    """Gradients (any layout: packed slices, caller tensors) against the oracle."""
    qc, kc, vc, doc = (t.detach().cpu() for t in (q, k, v, do))
    g_ref, g_tw, noise = _oracles(qc, kc, vc, doc, s, causal)
    for name, got, r, t, n in zip(("dq", "dk", "dv"), grads, g_ref, g_tw, noise):
        assert_2x(f"{tag} {name}", got, r, t, n)


@pytest.mark.gpu
@pytest.mark.parametrize("hd,causal,sq,sk,heads,batch,scale", CASES)
def test_bwd_parity(device, hd, causal, sq, sk, heads, batch, scale):
    h, hk = heads
    g = torch.Generator().manual_seed(2000 + sq * 7 + sk * 13 + hd + int(causal))
    q = randn16((batch, sq, h, hd), g)
    k = randn16((batch, sk, hk, hd), g)
    v = randn16((batch, sk, hk, hd), g)
    do = randn16((batch, sq, h, hd), g)
    s = hd ** -0.5 if scale is None else scale
    qd, kd, vd = (t.to(device).requires_grad_() for t in (q, k, v))
    out = fai.flash_attn_func(qd, kd, vd, softmax_scale=scale, causal=causal)
    out.backward(do.to(device))
    torch.cuda.synchronize()
    (dq_r, dk_r, dv_r), (dq_t, dk_t, dv_t), (nq, nk, nv) = _oracles(q, k, v, do, s, causal)
    assert kd.grad.shape == k.shape and vd.grad.shape == v.shape
    assert_2x("dq", qd.grad, dq_r, dq_t, nq)
    assert_2x("dk", kd.grad, dk_r, dk_t, nk)
    assert_2x("dv", vd.grad, dv_r, dv_t, nv)


@pytest.mark.gpu
def test_bwd_packed_matches_unpacked(device):
    g = torch.Generator().manual_seed(21)
    qkv = randn16((2, 160, 3, 2, 64), g).to(device).requires_grad_()
    do = randn16((2, 160, 2, 64), g).to(device)
    fai.flash_attn_qkvpacked_func(qkv, causal=True).backward(do)
    q, k, v = (qkv.detach()[:, :, i].clone().requires_grad_() for i in range(3))
    fai.flash_attn_func(q, k, v, causal=True).backward(do)
    assert torch.equal(qkv.grad[:, :, 0], q.grad)
    assert torch.equal(qkv.grad[:, :, 1], k.grad)
    assert torch.equal(qkv.grad[:, :, 2], v.grad)
    _check_grads("qkvpacked", q, k, v, do, [qkv.grad[:, :, i] for i in range(3)], 64 ** -0.5, True)


@pytest.mark.gpu
def test_bwd_deterministic(device):
    g = torch.Generator().manual_seed(22)
    q, k, v = (randn16((1, 600, 4, 128), g).to(device).requires_grad_() for _ in range(3))
    do = randn16((1, 600, 4, 128), g).to(device)
    res = []
    for _ in range(2):
        for t in (q, k, v):
            t.grad = None
        fai.flash_attn_func(q, k, v, causal=True).backward(do)
        res.append([t.grad.clone() for t in (q, k, v)])
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_kvpacked_bwd_matches_unpacked(device):
    # GQA kv packed (b, s, 2, hk, d): dkv is one tensor written slice by slice.
    g = torch.Generator().manual_seed(23)
    q = randn16((2, 150, 4, 128), g).to(device).requires_grad_()
    kv = randn16((2, 170, 2, 2, 128), g).to(device).requires_grad_()
    do = randn16((2, 150, 4, 128), g).to(device)
    fai.flash_attn_kvpacked_func(q, kv, causal=True).backward(do)
    qr = q.detach().clone().requires_grad_()
    k, v = (kv.detach()[:, :, i].clone().requires_grad_() for i in range(2))
    fai.flash_attn_func(qr, k, v, causal=True).backward(do)
    assert torch.equal(q.grad, qr.grad)
    assert torch.equal(kv.grad[:, :, 0], k.grad)
    assert torch.equal(kv.grad[:, :, 1], v.grad)
    _check_grads("kvpacked", q, k, v, do, [q.grad, kv.grad[:, :, 0], kv.grad[:, :, 1]], 128 ** -0.5, True)


@pytest.mark.gpu
def test_bwd_into_given_tensors(device):
    # Gradients written into caller tensors: strided slices in place (same
    # storage returned), and a view whose base is not 16-byte aligned through
    # a temporary; both equal the freshly allocated result.
    g = torch.Generator().manual_seed(24)
    q, k, v = (randn16((1, 96, 2, 64), g).to(device) for _ in range(3))
    do = randn16((1, 96, 2, 64), g).to(device)
    s = 64 ** -0.5
    out, lse = fai._flash_attn_forward(q, k, v, s, True)
    ref = fai._flash_attn_backward(do, q, k, v, out, lse, s, True)
    packed = torch.full((1, 96, 3, 2, 64), 7.0, dtype=torch.float16, device=device)
    views = tuple(packed[:, :, i] for i in range(3))
    got = fai._flash_attn_backward(do, q, k, v, out, lse, s, True, *views)
    for r, x, w in zip(ref, got, views):
        assert x.data_ptr() == w.data_ptr()
        assert torch.equal(x, r)
    _check_grads("into packed slices", q, k, v, do, got, s, True)
    buf = torch.zeros(1 * 96 * 2 * 64 + 4, dtype=torch.float16, device=device)
    odd = buf[4:].view(1, 96, 2, 64)  # base 8 bytes past a 16-byte boundary
    dq, _, _ = fai._flash_attn_backward(do, q, k, v, out, lse, s, True, odd, None, None)
    assert dq.data_ptr() == odd.data_ptr() and torch.equal(dq, ref[0])
    assert torch.equal(buf[:4], torch.zeros(4, dtype=torch.float16, device=device))
    with pytest.raises(RuntimeError, match="dk must have the shape of its input"):
        fai._flash_attn_backward(do, q, k, v, out, lse, s, True, None, views[1][:, :50], None)
