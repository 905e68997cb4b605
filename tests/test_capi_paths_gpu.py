"""Entry points and kernel instances of the C ABI that the drop-in Python API
does not reach, against the oracle (through the ctypes binding, fa_capi):

* fa_bwd_preprocess followed by fa_bwd_dkdv: the standalone dO.O row-sum
  kernel (the counterpart of flash_bwd_preprocess_kernel.h:23-96) feeding the
  dK/dV kernel, instead of the row sums the dQ kernel writes;
* fa_kv_append + fa_kv_splitkv + fa_kv_combine without the batch_order
  workspace: the split kernel's natural-order instances (one workgroup per
  work item, no device work counter), plain and with the options instance;
* a paged split whose keys span more than the 1024 page ids the split kernel
  stages in LDS: the fallback that reads the block table per tile
  (the reference handles any length, kvcache_native.cu:1061-1062);
* the split kernel's own combine (split counts), against the combine kernel
  and the oracle.
"""

import ctypes

import pytest
import torch

import fa_capi
import flash_attention_interface as fai
from helpers import assert_2x, assert_lse, check_fwd_bwd, check_varlen, cu_from_lengths, kv_oracle, randn16
from oracle import kvcache as okv
from oracle.attention import attention_fwd


@pytest.mark.gpu
@pytest.mark.parametrize("varlen,hd,causal,heads", [(False, 128, True, (8, 2)), (False, 64, False, (4, 4)),
                                                    (True, 128, True, (6, 3)), (True, 64, False, (4, 1))])
def test_preprocess_then_dkdv(device, varlen, hd, causal, heads):
    h, hk = heads
    g = torch.Generator().manual_seed(9100 + hd + 2 * varlen + causal)
    if varlen:
        lens = [300, 1, 517, 64]
        cu = cu_from_lengths(lens)
        tot, mx = int(cu[-1]), max(lens)
        q, do = randn16((tot, h, hd), g), randn16((tot, h, hd), g)
        k, v = randn16((tot, hk, hd), g), randn16((tot, hk, hd), g)
        lse_shape = (len(lens), h, mx)
    else:
        b, sq = 2, 390
        q, do = randn16((b, sq, h, hd), g), randn16((b, sq, h, hd), g)
        k, v = randn16((b, sq, hk, hd), g), randn16((b, sq, hk, hd), g)
        lse_shape = (b, h, sq)
    s = hd ** -0.5
    qd, kd, vd, dod = (t.to(device) for t in (q, k, v, do))
    o = torch.empty_like(qd)
    lse = torch.empty(lse_shape, dtype=torch.float32, device=device)
    cud = cu.to(device) if varlen else None
    mq = mx if varlen else 0
    fa_capi.call("fa_fwd", fa_capi.fwd_args(qd, kd, vd, o, lse, s, causal, cud, cud, mq, mq))
    dq, dk, dv = torch.zeros_like(qd), torch.full_like(kd, 7.0), torch.full_like(vd, 7.0)
    dsum = torch.full((2,) + lse_shape, 3.0, dtype=torch.float32, device=device)
    ba = fa_capi.bwd_args(qd, kd, vd, o, lse, dod, dq, dk, dv, dsum, s, causal, cud, cud, mq, mq)
    print(f"case varlen={varlen} hd={hd} causal={causal} heads={heads}", flush=True)
    fa_capi.call("fa_bwd_preprocess", ba)
    fa_capi.call("fa_bwd_dkdv", ba)
    torch.cuda.synchronize()
    # The row sums: -D = -sum_d O * dO (fp32), and LSE * log2(e); 0 on padding rows.
    of, dof = o.float().cpu(), do.float()
    if varlen:
        d_ref = torch.zeros(lse_shape)
        for bi in range(len(lens)):
            a0, a1 = int(cu[bi]), int(cu[bi + 1])
            d_ref[bi, :, : a1 - a0] = (of[a0:a1] * dof[a0:a1]).sum(-1).T
    else:
        d_ref = (of * dof).sum(-1).permute(0, 2, 1)
    assert torch.allclose(-dsum[0].cpu(), d_ref, rtol=1e-5, atol=1e-5)
    assert torch.allclose(dsum[1].cpu(), lse.cpu() * 1.4426950408889634, rtol=1e-6, atol=1e-6)
    # dK / dV against the oracle (dQ is not part of this path; pass the oracle's own).
    if varlen:
        from oracle.attention import varlen_bwd, varlen_fwd

        o_ref, l_ref = varlen_fwd(q, k, v, cu, cu, mx, s, causal)
        dq_ref = varlen_bwd(q, k, v, o_ref, l_ref, do, cu, cu, s, causal)[0]
        check_varlen("preprocess+dkdv", cu, cu, q, k, v, do, o.cpu(), None, (dq_ref, dk.cpu(), dv.cpu()), s, causal)
    else:
        from oracle.attention import attention_bwd

        o_ref, l_ref = attention_fwd(q, k, v, s, causal)
        dq_ref = attention_bwd(q, k, v, o_ref, l_ref, do, s, causal)[0]
        check_fwd_bwd("preprocess+dkdv", q, k, v, do, o.cpu(), lse.cpu(), (dq_ref, dk.cpu(), dv.cpu()), s, causal)


def _kv_inputs(g, b, sq, h, hk, hd, cap, new, paged, page=256):
    q = randn16((b, sq, h, hd), g)
    kc, vc = randn16((b, cap, hk, hd), g), randn16((b, cap, hk, hd), g)
    k = randn16((b, new, hk, hd), g) if new else None
    v = randn16((b, new, hk, hd), g) if new else None
    table = None
    if paged:
        nb = cap // page
        table = torch.randperm(b * nb, generator=g).reshape(b, nb).to(torch.int32)
        kp = torch.empty((b * nb, page, hk, hd), dtype=torch.float16)
        vp = torch.empty_like(kp)
        for bi in range(b):
            for j in range(nb):
                kp[table[bi, j]] = kc[bi, j * page:(j + 1) * page]
                vp[table[bi, j]] = vc[bi, j * page:(j + 1) * page]
        kc, vc = kp, vp
    return q, kc, vc, k, v, table


def _kv_capi(device, q, kc, vc, k, v, seqlens, table, causal, splits, window=(-1, -1), order=False, fused=False,
             calls=("fa_kv_append", "fa_kv_splitkv", "fa_kv_combine"), cache_batch_idx=None, status=None):
    """The decode entry points ``calls`` through the C ABI; batch_order only when
    ``order``, split counts (the split kernel's own combine) only when ``fused``."""
    qd, kcd, vcd = q.to(device), kc.clone().to(device), vc.clone().to(device)
    kd = None if k is None else k.to(device)
    vd = None if v is None else v.to(device)
    o = torch.full_like(qd, 5.0)
    b, sq, h, hd = q.shape
    lse = torch.full((b, h, sq), 5.0, dtype=torch.float32, device=device)
    rows = b * h * sq
    acc = torch.empty((splits * rows * (hd + 1),), dtype=torch.float32, device=device)
    border = torch.full((b + 1,), -3, dtype=torch.int32, device=device)
    counts = torch.full((max(1, b * h * ((sq + 31) // 32)),), -3, dtype=torch.int32, device=device)
    a = fa_capi.kvcache_args(qd, kcd, vcd, o, lse, seqlens.to(device), hd ** -0.5, causal, splits, kd, vd,
                             block_table=None if table is None else table.to(device),
                             cache_batch_idx=None if cache_batch_idx is None else cache_batch_idx.to(device),
                             out_accum=acc if splits > 1 else None,
                             lse_accum=acc[splits * rows * hd:] if splits > 1 else None,
                             batch_order=border if order else None, window=window,
                             split_count=counts if fused else None, status=status)
    assert fa_capi.load().fa_kv_workspace_bytes(ctypes.byref(a)) <= acc.numel() * 4
    assert fa_capi.load().fa_kv_split_count_len(ctypes.byref(a)) <= counts.numel()
    for name in calls:
        fa_capi.call(name, a)
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu(), kcd.cpu(), vcd.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,h,hk,hd,cap,new,paged,splits,window", [
    (5, 1, 8, 2, 128, 1024, 1, True, 4, (-1, -1)),
    (3, 4, 8, 8, 64, 2048, 4, False, 6, (-1, -1)),
    (4, 1, 8, 2, 128, 1024, 1, False, 1, (-1, -1)),
    (3, 2, 4, 1, 64, 768, 2, True, 3, (100, -1)),  # options instance
])
def test_splitkv_natural_order(device, b, sq, h, hk, hd, cap, new, paged, splits, window):
    g = torch.Generator().manual_seed(9200 + b + sq + hd + splits)
    q, kc, vc, k, v, table = _kv_inputs(g, b, sq, h, hk, hd, cap, new, paged)
    seqlens = torch.randint(0, cap - new + 1, (b,), generator=g, dtype=torch.int32)
    seqlens[0] = cap - new
    print(f"case b={b} sq={sq} hd={hd} paged={paged} splits={splits} window={window}", flush=True)
    out, lse, kca, vca = _kv_capi(device, q, kc, vc, k, v, seqlens, table, True, splits, window)
    if window == (-1, -1):
        o_ref, l_ref, kc_ref, vc_ref = kv_oracle(q, kc, vc, k, v, seqlens, None, table, True, splits, None)
    else:
        _, _, kc_ref, vc_ref = kv_oracle(q, kc, vc, k, v, seqlens, None, table, True, splits, None)
        ends = seqlens + new
        ku, vu = okv.materialize(kc_ref, vc_ref, ends, None, table)
        o_ref, l_ref = okv.splitkv_attention(q, ku, vu, ends, hd ** -0.5, True, splits, window=window)
    assert torch.equal(kca, kc_ref) and torch.equal(vca, vc_ref), "append differs from the oracle"
    assert_2x("out", out, o_ref, o_ref.to(torch.float16))
    assert_lse(lse, l_ref)
    # Same bits as the longest-first resident grid (the order does not change any item's arithmetic).
    got = _kv_capi(device, q, kc, vc, k, v, seqlens, table, True, splits, window, order=True)
    assert torch.equal(got[0], out) and torch.equal(got[1], lse)


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,h,hk,hd,cap,new,paged,splits,window,remap", [
    (7, 1, 32, 8, 128, 2048, 1, True, 8, (-1, -1), False),   # c4's form: GQA group of 4 rows, paged
    (4, 4, 16, 16, 64, 4096, 4, False, 16, (-1, -1), True),  # c5's form: MHA, 4 query rows, remapped
    (3, 5, 16, 2, 128, 1024, 5, False, 3, (-1, -1), False),  # 40 rows of a kv head: two row tiles
    (5, 2, 8, 2, 64, 768, 2, True, 5, (200, -1), False),     # options instance (local window)
    (3, 3, 32, 1, 64, 1024, 3, False, 70, (-1, -1), False),   # 96 rows (three tiles), 70 splits (> 64)
])
def test_fused_combine(device, b, sq, h, hk, hd, cap, new, paged, splits, window, remap):
    """With batch_order and split counts the split kernel combines its partials
    itself (the last split item of each row tile to finish) and fa_fwd_kvcache
    is two launches: the same bits as the combine kernel, the oracle's values,
    and a second call right after (other lengths) starts from counts the
    ordering workgroup zeroed again.  An invalid sequence (cache overflow) is
    reported and gets O = 0, LSE = 0 through the fused path too."""
    g = torch.Generator().manual_seed(9250 + b + sq + hd + splits)
    q, kc, vc, k, v, table = _kv_inputs(g, b, sq, h, hk, hd, cap, new, paged)
    rows_c = b + 2 if remap else b
    if remap:
        kc = torch.cat([kc, randn16((2,) + tuple(kc.shape[1:]), g)])
        vc = torch.cat([vc, randn16((2,) + tuple(vc.shape[1:]), g)])
    idx = torch.randperm(rows_c, generator=g)[:b].to(torch.int32) if remap else None
    for call in range(2):
        seqlens = torch.randint(0, cap - new + 1, (b,), generator=g, dtype=torch.int32)
        seqlens[call] = cap - new
        seqlens[-1] = cap - new + 1  # overflows the cache after the append: invalid
        print(f"case fused b={b} sq={sq} hd={hd} splits={splits} call={call}", flush=True)
        st_f = torch.zeros(1, dtype=torch.int32, device=device)
        ref = _kv_capi(device, q, kc, vc, k, v, seqlens, table, True, splits, window, order=True,
                       cache_batch_idx=idx)
        got = _kv_capi(device, q, kc, vc, k, v, seqlens, table, True, splits, window, order=True, fused=True,
                       calls=("fa_fwd_kvcache",), cache_batch_idx=idx, status=st_f)
        for n, r, x in zip(("out", "lse", "k_cache", "v_cache"), ref, got):
            assert torch.equal(r, x), f"{n}: fused combine differs from the combine kernel"
        # The three entry points with counts: fa_kv_splitkv combines, fa_kv_combine has nothing left to do.
        three = _kv_capi(device, q, kc, vc, k, v, seqlens, table, True, splits, window, order=True, fused=True,
                         cache_batch_idx=idx)
        assert torch.equal(three[0], ref[0]) and torch.equal(three[1], ref[1])
        assert int(st_f.item()) == 1, "the overflowing sequence is reported"
        out, lse = got[0], got[1]
        assert not out[-1].any() and not lse[-1].any(), "an invalid sequence gets O = 0, LSE = 0"
        valid = slice(0, b - 1)
        sl = seqlens[valid]
        kcv, vcv = (kc, vc)
        kv_idx = None if idx is None else idx[valid]
        tab = None if table is None else table[valid]
        if window == (-1, -1):
            o_ref, l_ref, _, _ = kv_oracle(q[valid], kcv, vcv, k[valid], v[valid], sl, kv_idx, tab, True, splits,
                                           None)
        else:
            _, _, kc_ref, vc_ref = kv_oracle(q[valid], kcv, vcv, k[valid], v[valid], sl, kv_idx, tab, True, splits,
                                             None)
            ku, vu = okv.materialize(kc_ref, vc_ref, sl + new, kv_idx, tab)
            o_ref, l_ref = okv.splitkv_attention(q[valid], ku, vu, sl + new, hd ** -0.5, True, splits, window=window)
        assert_2x("out", out[valid], o_ref, o_ref.to(torch.float16))
        assert_lse(lse[valid], l_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("splits,order", [(1, False), (1, True), (2, True)])
def test_paged_split_over_1024_pages(device, splits, order):
    """1100 shuffled pages of 256 tokens in one sequence (hk 1, d 64): with one
    split the kernel walks more page ids than it stages in LDS and reads the
    block table per tile; two splits of ~550 pages stage them in LDS."""
    g = torch.Generator().manual_seed(9300)
    pages, page, h, hk, hd = 1100, 256, 4, 1, 64
    cap = pages * page
    q = randn16((1, 1, h, hd), g)
    kn, vn = randn16((1, 1, hk, hd), g), randn16((1, 1, hk, hd), g)
    gd = torch.Generator(device=device).manual_seed(9301)
    kp = torch.randn((pages, page, hk, hd), generator=gd, device=device, dtype=torch.float16)
    vp = torch.randn((pages, page, hk, hd), generator=gd, device=device, dtype=torch.float16)
    table = torch.randperm(pages, generator=g).reshape(1, pages).to(torch.int32)
    seqlens = torch.tensor([cap - 7], dtype=torch.int32)
    print(f"case splits={splits} order={order}: {cap - 6} keys over {pages} pages", flush=True)
    out, lse, kpa, vpa = _kv_capi(device, q, kp.cpu(), vp.cpu(), kn, vn, seqlens, table, True, splits, order=order)
    o_ref, l_ref, kp_ref, vp_ref = kv_oracle(q, kp.cpu(), vp.cpu(), kn, vn, seqlens, None, table, True, splits, None)
    assert torch.equal(kpa, kp_ref) and torch.equal(vpa, vp_ref)
    assert_2x("out", out, o_ref, o_ref.to(torch.float16))
    assert_lse(lse, l_ref)
    # The drop-in API takes the same fallback with num_splits=1.
    kpd, vpd = kp.clone(), vp.clone()
    o2 = fai.flash_attn_with_kvcache(q.to(device), kpd, vpd, kn.to(device), vn.to(device),
                                     cache_seqlens=seqlens.to(device), block_table=table.to(device), causal=True,
                                     num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(o2.cpu(), out)


def _len_bucket(n):
    """The order kernel's key-count bucket: exact below 32, then 32 per power of two."""
    if n < 32:
        return n
    msb = n.bit_length() - 1
    return (msb - 4) * 32 + ((n >> (msb - 5)) & 31)


@pytest.mark.gpu
def test_order_kernel_large_batch(device):
    """2500 sequences (more than one order-kernel round of 1024 threads): the
    batch_order list is a permutation, sequences by non-increasing key-count
    bucket, and the decode over that order matches the oracle (one invalid
    sequence included: it sorts as empty and gets O = 0, LSE = 0)."""
    g = torch.Generator().manual_seed(9400)
    b, sq, h, hk, hd, cap, new, splits = 2500, 1, 4, 2, 64, 96, 1, 2
    q, kc, vc, k, v, _ = _kv_inputs(g, b, sq, h, hk, hd, cap, new, False)
    seqlens = torch.randint(0, cap - new + 1, (b,), generator=g, dtype=torch.int32)
    seqlens[7] = cap  # cap + new > cap: invalid
    qd, kcd, vcd = q.to(device), kc.clone().to(device), vc.clone().to(device)
    o = torch.full_like(qd, 5.0)
    lse = torch.full((b, h, sq), 5.0, dtype=torch.float32, device=device)
    rows = b * h * sq
    acc = torch.empty((splits * rows * (hd + 1),), dtype=torch.float32, device=device)
    border = torch.full((b + 1,), -3, dtype=torch.int32, device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    a = fa_capi.kvcache_args(qd, kcd, vcd, o, lse, seqlens.to(device), hd ** -0.5, True, splits, k.to(device),
                             v.to(device), out_accum=acc, lse_accum=acc[splits * rows * hd:], batch_order=border,
                             status=status)
    print(f"case order kernel b={b}", flush=True)
    for name in ("fa_kv_append", "fa_kv_splitkv", "fa_kv_combine"):
        fa_capi.call(name, a)
    torch.cuda.synchronize()
    order = border.cpu().tolist()
    assert sorted(order[:b]) == list(range(b)), "batch_order must list every sequence once"
    ends = [0 if i == 7 else int(n) + new for i, n in enumerate(seqlens.tolist())]
    keys = [_len_bucket(ends[i]) for i in order[:b]]
    assert all(x >= y for x, y in zip(keys, keys[1:])), "sequences must come most keys first"
    assert order[b] > 0, "the work counter is reset, then counts the claimed items"
    assert int(status.item()) == 1, "the invalid sequence is reported as a capacity error"
    valid = [i for i in range(b) if i != 7]
    sl = seqlens.clone()
    sl[7] = 0
    o_ref, l_ref, _, _ = kv_oracle(q[valid], kc[valid], vc[valid], k[valid], v[valid], sl[valid], None, None, True,
                                   splits, None)
    assert_2x("out", o.cpu()[valid], o_ref, o_ref.to(torch.float16))
    assert_lse(lse.cpu()[valid], l_ref)
    assert not o.cpu()[7].any() and not lse.cpu()[7].any()
