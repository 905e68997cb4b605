"""Varlen work orders: the optional work_order workspaces of fa_bwd_args (dK/dV
and dQ lists) and fa_fwd_args.

With the workspace, fa_bwd lists the (sequence, key block) items on the device,
most query rows first, and launches the dK/dV workgroups in that order (and the
dQ kernel its (sequence, block of query positions) items, most keys first).  Every
item is computed independently, so dQ, dK and dV must be bit-identical to the
natural-order launch; the list itself must hold every item with keys exactly
once, in non-increasing 64-row buckets of the rows that see the key block
(causal: min(sq, sk - 128 nb), else sq), then -1 for the items with no keys.
Cases: mixed lengths with empty and one-token sequences, sq != sk, GQA,
head_dim 64 and 128, causal and not."""

import ctypes

import pytest
import torch

import fa_capi
from helpers import check_varlen, cu_from_lengths, randn16

CASES = [
    # lengths_q, lengths_k, h, hk, hd, causal
    ([1838, 2357, 653, 3709, 463, 1, 0, 552], None, 8, 2, 128, True),
    ([200, 17, 90, 0, 700], [100, 300, 90, 5, 640], 6, 3, 128, False),
    ([300, 17, 1000, 129], [129, 300, 1000, 17], 4, 1, 64, True),
    ([64, 128, 256, 1000], None, 4, 4, 64, False),
]


def _bucket_rows(lq, lk, nb, causal):
    k0 = 128 * nb
    if k0 >= lk:
        return None
    rows = max(0, min(lq, lk - k0)) if causal else lq
    return min(rows // 64, 1023)


@pytest.mark.gpu
@pytest.mark.parametrize("lens_q,lens_k,h,hk,hd,causal", CASES)
def test_work_order_same_results_and_sorted(device, lens_q, lens_k, h, hk, hd, causal):
    lens_k = lens_k or lens_q
    g = torch.Generator().manual_seed(6100 + sum(lens_q) + hd)
    cu_q, cu_k = cu_from_lengths(lens_q), cu_from_lengths(lens_k)
    tq, tk = int(cu_q[-1]), int(cu_k[-1])
    mq, mk = max(lens_q), max(lens_k)
    q, do = randn16((tq, h, hd), g).to(device), randn16((tq, h, hd), g).to(device)
    k, v = randn16((tk, hk, hd), g).to(device), randn16((tk, hk, hd), g).to(device)
    cq, ck = cu_q.to(device), cu_k.to(device)
    o = torch.empty_like(q)
    lse = torch.empty((len(lens_q), h, mq), dtype=torch.float32, device=device)
    s = hd ** -0.5
    fa = fa_capi.fwd_args(q, k, v, o, lse, s, causal, cq, ck, mq, mk)
    fa_capi.call("fa_fwd", fa)  # raises on a non-zero code
    grads = {}
    for ordered in (False, True):
        dq, dk, dv = torch.full_like(q, 7.0), torch.full_like(k, 7.0), torch.full_like(v, 7.0)
        dsum = torch.empty((2,) + tuple(lse.shape), dtype=torch.float32, device=device)
        ba = fa_capi.bwd_args(q, k, v, o, lse, do, dq, dk, dv, dsum, s, causal, cq, ck, mq, mk)
        n = fa_capi.load().fa_bwd_order_len(ctypes.byref(ba))
        # dQ blocks hold P = 128 / gp positions of gp heads of a GQA group.
        nnb, p_dq = (mk + 127) // 128, 128 // _head_pack(h, hk, 128)
        nmb = (mq + p_dq - 1) // p_dq
        assert n == len(lens_q) * (nnb + (mq + 31) // 32)
        order = torch.full((n,), -7, dtype=torch.int32, device=device)
        if ordered:
            ba.work_order = order.data_ptr()
        print(f"case lens_q={lens_q} hd={hd} causal={causal} ordered={ordered}", flush=True)
        fa_capi.call("fa_bwd", ba)
        torch.cuda.synchronize()
        grads[ordered] = (dq.cpu(), dk.cpu(), dv.cpu())
        if ordered:
            got = order.cpu().tolist()[: len(lens_q) * nnb]  # the dK/dV list
            expect = {}
            for b in range(len(lens_q)):
                for nb in range(nnb):
                    bk = _bucket_rows(lens_q[b], lens_k[b], nb, causal)
                    if bk is not None:
                        expect[b * nnb + nb] = bk
            live = got[: len(expect)]
            assert sorted(live) == sorted(expect), "the list must hold every item with keys once"
            assert all(x == -1 for x in got[len(expect):]), "the rest of the list must be -1"
            buckets = [expect[i] for i in live]
            assert all(x >= y for x, y in zip(buckets, buckets[1:])), "items must come most rows first"
            # The dQ list (second part): query blocks by the keys their last row sees.
            got_q = order.cpu().tolist()[len(lens_q) * nnb: len(lens_q) * (nnb + nmb)]
            expect_q = {}
            for b in range(len(lens_q)):
                for mb in range(nmb):
                    m0 = p_dq * mb
                    if m0 < lens_q[b]:
                        keys = max(0, min(lens_k[b], m0 + p_dq + lens_k[b] - lens_q[b])) if causal else lens_k[b]
                        expect_q[b * nmb + mb] = min(keys // 64, 1023)
            live_q = got_q[: len(expect_q)]
            assert sorted(live_q) == sorted(expect_q) and all(x == -1 for x in got_q[len(expect_q):])
            bq = [expect_q[i] for i in live_q]
            assert all(x >= y for x, y in zip(bq, bq[1:])), "query blocks must come most keys first"
    for a, b, name in zip(grads[False], grads[True], ("dq", "dk", "dv")):
        assert torch.equal(a, b), f"{name} differs between the natural and the device-built order"
    # Both orders' results (bit-identical) against the per-sequence oracle.
    check_varlen("work order", cu_q, cu_k, q.cpu(), k.cpu(), v.cpu(), do.cpu(), o.cpu(), lse.cpu(), grads[True], s,
                 causal)


def _head_pack(h, hk, bm):
    """Query heads per forward or dQ workgroup: the largest power of two dividing
    the GQA group that leaves whole 32-row tiles per head."""
    gp = 1
    while 2 * gp <= bm // 32 and (h // hk) % (2 * gp) == 0:
        gp *= 2
    return gp


def _fwd_bucket(lq, lk, mb, bm, causal):
    m0 = bm * mb
    if m0 >= lq:
        return None
    rows = min(bm, lq - m0)
    keys = max(0, min(lk, m0 + bm + lk - lq)) if causal else lk
    return min(rows * keys // (bm * 64), 1023)


@pytest.mark.gpu
@pytest.mark.parametrize("lens_q,lens_k,h,hk,hd,causal", CASES)
def test_fwd_work_order_same_results_and_sorted(device, lens_q, lens_k, h, hk, hd, causal):
    """fa_fwd with the work_order workspace: the same output and LSE bits as the
    natural order, and a list holding every (sequence, query block) item once,
    non-empty ones by non-increasing work, then the blocks past each sequence."""
    lens_k = lens_k or lens_q
    g = torch.Generator().manual_seed(6200 + sum(lens_q) + hd)
    cu_q, cu_k = cu_from_lengths(lens_q), cu_from_lengths(lens_k)
    tq, tk = int(cu_q[-1]), int(cu_k[-1])
    mq, mk = max(lens_q), max(lens_k)
    q = randn16((tq, h, hd), g).to(device)
    k, v = randn16((tk, hk, hd), g).to(device), randn16((tk, hk, hd), g).to(device)
    cq, ck = cu_q.to(device), cu_k.to(device)
    s = hd ** -0.5
    res = {}
    for ordered in (False, True):
        o = torch.full_like(q, 7.0)
        lse = torch.full((len(lens_q), h, mq), 7.0, dtype=torch.float32, device=device)
        fa = fa_capi.fwd_args(q, k, v, o, lse, s, causal, cq, ck, mq, mk)
        n = fa_capi.load().fa_fwd_order_len(ctypes.byref(fa))
        assert n == len(lens_q) * ((mq + 31) // 32)
        order = torch.full((n,), -7, dtype=torch.int32, device=device)
        if ordered:
            fa.work_order = order.data_ptr()
        print(f"case lens_q={lens_q} hd={hd} causal={causal} ordered={ordered}", flush=True)
        fa_capi.call("fa_fwd", fa)
        torch.cuda.synchronize()
        res[ordered] = (o.cpu(), lse.cpu())
        if ordered:
            cus = torch.cuda.get_device_properties(0).multi_processor_count
            # Positions per workgroup: 256 rows (ping-pong) or 128, over gp heads.
            gp = _head_pack(h, hk, 256)
            pp_grid = -(-mq * gp // 256) * len(lens_q) * (h // gp)
            bm = 256 // gp if hd == 128 and pp_grid >= 2 * cus and mq >= 2048 else 128 // _head_pack(h, hk, 128)
            nmb = (mq + bm - 1) // bm
            got = order.cpu().tolist()[: len(lens_q) * nmb]
            assert sorted(got) == list(range(len(lens_q) * nmb)), "every item exactly once"
            bk = [_fwd_bucket(lens_q[i // nmb], lens_k[i // nmb], i % nmb, bm, causal) for i in got]
            n_live = sum(x is not None for x in bk)
            assert all(x is not None for x in bk[:n_live]) and all(x is None for x in bk[n_live:])
            assert all(x >= y for x, y in zip(bk[:n_live], bk[1:n_live])), "items must come most work first"
    assert torch.equal(res[False][0][:tq], res[True][0][:tq]) and torch.equal(res[False][1], res[True][1])
    check_varlen("fwd work order", cu_q, cu_k, q.cpu(), k.cpu(), v.cpu(), None, res[True][0], res[True][1], None, s,
                 causal)
