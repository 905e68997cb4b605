"""KV-cache parity on the GPU.

* append: the cache after the call equals the oracle append (Python slice /
  page-table writes, interface.py:642-685) bit for bit, for contiguous,
  cache_batch_idx-remapped and paged caches;
* attention: output vs the fp32 split-KV oracle (interface.py:731-776),
  bounded by 2x the reference's own error (its KV kernels are fp32 until the
  final fp16 rounding, so the twin is the rounded oracle); LSE to fp32
  precision with -inf reported as 0;
* layout invariance: paged, shuffled-paged and remapped caches give outputs
  bit-identical to the same logical contiguous cache.
Case list after test_flash_attn.py:1104-1964.
"""

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, assert_lse, kv_oracle, randn16
from oracle import kvcache as okv


def _paged_from_contiguous(kc, vc, lens, page, gen, shuffle=True):
    """Scatter a contiguous cache [b, cap, hk, d] into pages with a random
    (or identity) block table (builder after test_flash_attn.py:540-609)."""
    b, cap, hk, d = kc.shape
    nb = cap // page
    total = b * nb
    perm = torch.randperm(total, generator=gen) if shuffle else torch.arange(total)
    table = perm.reshape(b, nb).to(torch.int32)
    kp = torch.zeros((total, page, hk, d), dtype=kc.dtype)
    vp = torch.zeros_like(kp)
    for bi in range(b):
        for j in range(nb):
            kp[table[bi, j]] = kc[bi, j * page : (j + 1) * page]
            vp[table[bi, j]] = vc[bi, j * page : (j + 1) * page]
    return kp, vp, table


def _run(device, q, kc, vc, k, v, seqlens, batch_idx, table, causal, splits, scale=None):
    args = dict(
        cache_seqlens=seqlens.to(device),
        cache_batch_idx=None if batch_idx is None else batch_idx.to(device),
        block_table=None if table is None else table.to(device),
        causal=causal,
        num_splits=splits,
        return_softmax_lse=True,
        softmax_scale=scale,
    )
    kcd, vcd = kc.clone().to(device), vc.clone().to(device)
    out, lse = fai.flash_attn_with_kvcache(
        q.to(device), kcd, vcd, None if k is None else k.to(device), None if v is None else v.to(device), **args
    )
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), kcd.cpu(), vcd.cpu()


_oracle = kv_oracle


CASES = [
    # b, sq, h, hk, hd, cap, new, causal, splits, paged, remap
    (4, 1, 8, 2, 128, 1024, 1, True, 0, True, False),
    (4, 1, 8, 2, 128, 1024, 1, True, 8, True, False),
    (3, 1, 6, 1, 64, 768, 1, True, 3, True, False),
    (3, 1, 4, 4, 64, 512, 0, False, 1, False, False),
    (4, 4, 16, 16, 64, 2048, 4, True, 16, False, True),
    (4, 4, 16, 16, 64, 2048, 4, True, 0, False, True),
    (4, 4, 16, 16, 64, 2048, 4, True, 1, False, True),
    (2, 3, 6, 2, 128, 512, 3, True, 2, False, False),
    (2, 3, 6, 2, 128, 512, 3, False, 0, True, False),
    (2, 40, 4, 4, 128, 512, 0, True, 0, False, False),
    (2, 9, 8, 2, 64, 512, 2, True, 5, True, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,h,hk,hd,cap,new,causal,splits,paged,remap", CASES)
def test_kvcache_parity(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap):
    g = torch.Generator().manual_seed(4000 + b * 31 + sq * 7 + hd + splits)
    rows = b + 2 if remap else b
    kc = randn16((rows, cap, hk, hd), g)
    vc = randn16((rows, cap, hk, hd), g)
    q = randn16((b, sq, h, hd), g)
    k = randn16((b, new, hk, hd), g) if new else None
    v = randn16((b, new, hk, hd), g) if new else None
    seqlens = torch.randint(0, cap - new + 1, (b,), generator=g, dtype=torch.int32)
    seqlens[0] = cap - new  # one sequence at full capacity
    batch_idx = torch.randperm(rows, generator=g)[:b].to(torch.int32) if remap else None
    table = None
    if paged:
        kc, vc, table = _paged_from_contiguous(kc, vc, seqlens, 256, g)
    out, lse, kc_after, vc_after = _run(device, q, kc, vc, k, v, seqlens, batch_idx, table, causal, splits)
    o_ref, l_ref, kc_ref, vc_ref = _oracle(q, kc, vc, k, v, seqlens, batch_idx, table, causal, splits, None)
    assert torch.equal(kc_after, kc_ref), "k_cache after append differs from the oracle append"
    assert torch.equal(vc_after, vc_ref), "v_cache after append differs from the oracle append"
    assert_2x("out", out, o_ref, o_ref.to(torch.float16))
    assert_lse(lse, l_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("hd,sq,splits", [(128, 1, 8), (128, 1, 0), (64, 4, 16), (64, 2, 3)])
def test_kvcache_layout_invariance(device, hd, sq, splits):
    """Paged (identity and shuffled tables), remapped and contiguous caches holding
    the same logical tokens give bit-identical outputs."""
    g = torch.Generator().manual_seed(5000 + hd + sq)
    b, h, hk, cap = 3, 8, 2, 1024
    kc = randn16((b, cap, hk, hd), g)
    vc = randn16((b, cap, hk, hd), g)
    q = randn16((b, sq, h, hd), g)
    k = randn16((b, 1, hk, hd), g)
    v = randn16((b, 1, hk, hd), g)
    seqlens = torch.tensor([1000, 1, 517], dtype=torch.int32)
    ref = _run(device, q, kc, vc, k, v, seqlens, None, None, True, splits)
    for shuffle in (False, True):
        kp, vp, table = _paged_from_contiguous(kc, vc, seqlens, 256, g, shuffle=shuffle)
        got = _run(device, q, kp, vp, k, v, seqlens, None, table, True, splits)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    # remap: put the rows in a larger cache at permuted positions
    rows = torch.tensor([4, 0, 2], dtype=torch.int32)
    kr = randn16((5, cap, hk, hd), g)
    vr = randn16((5, cap, hk, hd), g)
    kr[rows.long()], vr[rows.long()] = kc, vc
    got = _run(device, q, kr, vr, k, v, seqlens, rows, None, True, splits)
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])


@pytest.mark.gpu
def test_kvcache_empty_cache_and_int_seqlens(device):
    g = torch.Generator().manual_seed(51)
    q = randn16((2, 1, 4, 64), g).to(device)
    kc = randn16((2, 256, 2, 64), g).to(device)
    vc = randn16((2, 256, 2, 64), g).to(device)
    out, lse = fai.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=0, causal=True, return_softmax_lse=True)
    assert torch.all(out == 0) and torch.all(lse == 0)
    out_int = fai.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=100, causal=True)
    out_t = fai.flash_attn_with_kvcache(
        q, kc, vc, cache_seqlens=torch.full((2,), 100, dtype=torch.int32, device=device), causal=True
    )
    assert torch.equal(out_int, out_t)
    out_full = fai.flash_attn_with_kvcache(q, kc, vc)  # cache_seqlens None -> full capacity
    o_ref, _ = okv.splitkv_attention(q.cpu(), kc.cpu(), vc.cpu(), torch.full((2,), 256), 0.125, False, 1)
    assert_2x("out", out_full, o_ref, o_ref.to(torch.float16))


@pytest.mark.gpu
@pytest.mark.parametrize("page,hd,splits,scale", [(512, 128, 4, None), (768, 64, 0, -0.2), (1024, 128, 7, 0.05)])
def test_kvcache_page_sizes_and_scales(device, page, hd, splits, scale):
    """Pages larger than 256 tokens (any multiple of 256 is accepted), negative and
    non-default scales: append bit-exact, attention vs the oracle, and, where the
    contiguous cache takes the same split-KV kernel (explicit splits > 1; a
    contiguous multi-token chunk otherwise runs the tiled forward kernel, as in
    the reference's routing, flash_api.cpp:668), the same output bit for bit."""
    g = torch.Generator().manual_seed(6000 + page + hd)
    b, sq, h, hk, cap, new = 3, 2, 8, 2, 3 * page, 2
    kc = randn16((b, cap, hk, hd), g)
    vc = randn16((b, cap, hk, hd), g)
    q = randn16((b, sq, h, hd), g)
    k = randn16((b, new, hk, hd), g)
    v = randn16((b, new, hk, hd), g)
    seqlens = torch.tensor([cap - new, page - 1, 5], dtype=torch.int32)  # full, straddling a page end, short
    kp, vp, table = _paged_from_contiguous(kc, vc, seqlens, page, g)
    out, lse, kp_after, vp_after = _run(device, q, kp, vp, k, v, seqlens, None, table, True, splits, scale)
    o_ref, l_ref, kp_ref, vp_ref = _oracle(q, kp, vp, k, v, seqlens, None, table, True, splits, scale)
    assert torch.equal(kp_after, kp_ref) and torch.equal(vp_after, vp_ref)
    assert_2x("out", out, o_ref, o_ref.to(torch.float16))
    assert_lse(lse, l_ref)
    if splits > 1:
        contiguous = _run(device, q, kc, vc, k, v, seqlens, None, None, True, splits, scale)
        assert torch.equal(contiguous[0], out) and torch.equal(contiguous[1], lse)


@pytest.mark.gpu
@pytest.mark.parametrize("b,h,hk,hd", [(64, 16, 16, 64), (32, 16, 16, 64), (64, 32, 8, 128)])
def test_kvcache_heads_per_item(device, b, h, hk, hd):
    """Decode calls with enough work items (8192 / 4096 / 4096 with 8 splits on
    a 256-CU MI355X: at least four per resident workgroup after the grouping)
    that the split kernel gives each item 4, 2 and 2 adjacent KV heads of a
    head-interleaved cache: append bit-exact and attention within 2x the
    reference's error against the oracle; the paged copy of the cache (also
    head-interleaved, so the same grouping) bit-identical; the same logical
    cache stored heads-major (one head per item) within the same bound."""
    g = torch.Generator().manual_seed(7000 + b + hk + hd)
    cap, splits = 1024, 8
    kc = randn16((b, cap, hk, hd), g)
    vc = randn16((b, cap, hk, hd), g)
    q = randn16((b, 1, h, hd), g)
    k = randn16((b, 1, hk, hd), g)
    v = randn16((b, 1, hk, hd), g)
    seqlens = torch.randint(256, cap, (b,), generator=g, dtype=torch.int32)
    seqlens[0] = cap - 1
    out, lse, kc_after, vc_after = _run(device, q, kc, vc, k, v, seqlens, None, None, True, splits)
    o_ref, l_ref, kc_ref, vc_ref = _oracle(q, kc, vc, k, v, seqlens, None, None, True, splits, None)
    assert torch.equal(kc_after, kc_ref) and torch.equal(vc_after, vc_ref)
    assert_2x("out", out, o_ref, o_ref.to(torch.float16))
    assert_lse(lse, l_ref)
    kp, vp, table = _paged_from_contiguous(kc, vc, seqlens, 256, g)
    paged = _run(device, q, kp, vp, k, v, seqlens, None, table, True, splits)
    assert torch.equal(paged[0], out) and torch.equal(paged[1], lse)
    # [b][hk][cap][d] storage seen as a strided [b][cap][hk][d] cache
    kh = kc.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    vh = vc.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    assert kh.stride(2) == cap * hd
    heads_major = _run(device, q, kh, vh, k, v, seqlens, None, None, True, splits)
    assert torch.equal(heads_major[2], kc_ref) and torch.equal(heads_major[3], vc_ref)
    assert_2x("out (heads-major cache)", heads_major[0], o_ref, o_ref.to(torch.float16))
    assert_lse(heads_major[1], l_ref)
