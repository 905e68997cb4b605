"""The synchronisation-free KV-cache mode (validate=False) on the GPU.

* For valid inputs it gives the default mode's outputs, LSE and cache bit for
  bit (contiguous, remapped, paged; split kernel and chunk route).
* Out-of-range inputs that the default mode rejects on the host (capacity,
  interface.py:855 / test_flash_attn.py:2084-2093; cache rows,
  flash_api.cpp:634-641) are caught by the kernels: the sequence is neither
  appended to nor attended over (O = 0, LSE = 0), the other sequences are
  unaffected, and flash_attn_kvcache_check() raises the default mode's error.
* A decode step (append + split-KV + combine) captured in a HIP graph replays
  correctly with new lengths written between replays, each replay checked
  against an eager call on the same inputs.
"""

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, assert_lse, kv_oracle, randn16


def _inputs(b, sq, h, hk, hd, cap, new, gen, paged=False, page=256):
    q = randn16((b, sq, h, hd), gen)
    kc = randn16((b, cap, hk, hd), gen)
    vc = randn16((b, cap, hk, hd), gen)
    k = randn16((b, new, hk, hd), gen) if new else None
    v = randn16((b, new, hk, hd), gen) if new else None
    table = None
    if paged:
        nb = cap // page
        table = torch.randperm(b * nb, generator=gen).reshape(b, nb).to(torch.int32)
        kc = kc.reshape(b * nb, page, hk, hd)
        vc = vc.reshape(b * nb, page, hk, hd)
    return q, kc, vc, k, v, table


def _call(device, q, kc, vc, k, v, seqlens, table=None, batch_idx=None, splits=0, validate=True):
    kcd, vcd = kc.clone().to(device), vc.clone().to(device)
    out, lse = fai.flash_attn_with_kvcache(
        q.to(device), kcd, vcd, None if k is None else k.to(device), None if v is None else v.to(device),
        cache_seqlens=seqlens.to(device), cache_batch_idx=None if batch_idx is None else batch_idx.to(device),
        block_table=None if table is None else table.to(device), causal=True, num_splits=splits,
        return_softmax_lse=True, validate=validate,
    )
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), kcd.cpu(), vcd.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize(
    "b,sq,h,hk,hd,cap,new,paged,remap,splits",
    [
        (4, 1, 8, 2, 128, 1024, 1, True, False, 0),   # paged decode, heuristic splits
        (3, 1, 4, 1, 64, 768, 1, True, False, 3),
        (3, 1, 4, 4, 64, 512, 0, False, False, 1),    # no append
        (4, 4, 8, 8, 64, 1024, 4, False, True, 1),    # remapped chunk: tiled forward kernel
        (4, 4, 8, 8, 64, 1024, 4, False, True, 4),
    ],
)
def test_nosync_matches_default(device, b, sq, h, hk, hd, cap, new, paged, remap, splits):
    gen = torch.Generator().manual_seed(7000 + b * 10 + sq + hd + splits)
    q, kc, vc, k, v, table = _inputs(b + (2 if remap else 0), sq, h, hk, hd, cap, new, gen, paged)
    q = q[:b]
    if k is not None:
        k, v = k[:b], v[:b]
    batch_idx = torch.randperm(b + 2, generator=gen)[:b].to(torch.int32) if remap else None
    seqlens = torch.randint(0, cap - new + 1, (b,), generator=gen, dtype=torch.int32)
    if table is not None:
        table = table[:b]
    fai.flash_attn_kvcache_check(device)
    ref = _call(device, q, kc, vc, k, v, seqlens, table, batch_idx, splits, validate=True)
    got = _call(device, q, kc, vc, k, v, seqlens, table, batch_idx, splits, validate=False)
    for name, r, x in zip(("out", "lse", "k_cache", "v_cache"), ref, got):
        assert torch.equal(r, x), name
    fai.flash_attn_kvcache_check(device)  # nothing recorded
    # The sync-free results against the oracle directly.
    o_ref, l_ref, kc_ref, vc_ref = kv_oracle(q, kc, vc, k, v, seqlens, batch_idx, table, True, splits, None)
    assert torch.equal(got[2], kc_ref) and torch.equal(got[3], vc_ref), "append differs from the oracle"
    assert_2x("out", got[0], o_ref, o_ref.to(torch.float16))
    assert_lse(got[1], l_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("route", ["paged", "contiguous_decode", "chunk"])
def test_nosync_out_of_range_caught_on_device(device, route):
    gen = torch.Generator().manual_seed(7100 + len(route))
    paged = route == "paged"
    sq, new, splits = (4, 4, 1) if route == "chunk" else (1, 1, 2)
    b, h, hk, hd, cap = 3, 4, 2, 64, 512
    q, kc, vc, k, v, table = _inputs(b, sq, h, hk, hd, cap, new, gen, paged)
    good = torch.tensor([100, 200, 50], dtype=torch.int32)
    ref = _call(device, q, kc, vc, k, v, good, table, None, splits, validate=True)
    # Oracle rows for the sequences kept valid (0 and 2); the invalid one must read as no keys.
    o_ref, l_ref, _, _ = kv_oracle(q, kc, vc, k, v, good, None, table, True, splits, None)
    fai.flash_attn_kvcache_check(device)
    for bad_len in (cap - new + 1, -1):
        seqlens = good.clone()
        seqlens[1] = bad_len
        if bad_len > 0:  # the host check (a maximum) passes negative lengths; the kernels do not
            with pytest.raises(ValueError, match="cache capacity is insufficient"):
                _call(device, q, kc, vc, k, v, seqlens, table, None, splits, validate=True)
        out, lse, kcd, vcd = _call(device, q, kc, vc, k, v, seqlens, table, None, splits, validate=False)
        assert not out[1].any() and not lse[1].any()
        for bi in (0, 2):
            assert_2x(f"out[{bi}]", out[bi], o_ref[bi], o_ref[bi].to(torch.float16))
            assert_lse(lse[bi], l_ref[bi])
        assert torch.equal(out[0], ref[0][0]) and torch.equal(out[2], ref[0][2])
        assert torch.equal(lse[0], ref[1][0]) and torch.equal(lse[2], ref[1][2])
        if paged:
            untouched = table[1].long()
            assert torch.equal(kcd[untouched], kc[untouched]) and torch.equal(vcd[untouched], vc[untouched])
            for bi in (0, 2):
                rows = table[bi].long()
                assert torch.equal(kcd[rows], ref[2][rows]) and torch.equal(vcd[rows], ref[3][rows])
        else:
            assert torch.equal(kcd[1], kc[1]) and torch.equal(vcd[1], vc[1])
            assert torch.equal(kcd[0], ref[2][0]) and torch.equal(kcd[2], ref[2][2])
        with pytest.raises(ValueError, match="cache capacity is insufficient for the requested append length"):
            fai.flash_attn_kvcache_check(device)
        fai.flash_attn_kvcache_check(device)  # cleared


@pytest.mark.gpu
@pytest.mark.parametrize("splits,sq", [(2, 1), (1, 4)])
def test_nosync_cache_row_out_of_range(device, splits, sq):
    gen = torch.Generator().manual_seed(7200 + splits)
    b, h, hk, hd, cap, new = 3, 4, 2, 64, 512, sq
    q, kc, vc, k, v, _ = _inputs(b + 1, sq, h, hk, hd, cap, new, gen)
    q, k, v = q[:b], k[:b], v[:b]
    seqlens = torch.tensor([10, 20, 30], dtype=torch.int32)
    fai.flash_attn_kvcache_check(device)
    for bad in (b + 1, -1):
        idx = torch.tensor([2, bad, 0], dtype=torch.int32)
        with pytest.raises(RuntimeError, match="cache_batch_idx entries must be within cache batch bounds"):
            _call(device, q, kc, vc, k, v, seqlens, None, idx, splits, validate=True)
        out, lse, kcd, vcd = _call(device, q, kc, vc, k, v, seqlens, None, idx, splits, validate=False)
        assert not out[1].any() and not lse[1].any()
        # Sequences 0 and 2 (cache rows 2 and 0) against the oracle.
        keep = torch.tensor([0, 2])
        o_ref, l_ref, _, _ = kv_oracle(q[keep], kc, vc, k[keep], v[keep], seqlens[keep], idx[keep], None, True,
                                       splits, None)
        for j, bi in enumerate((0, 2)):
            assert_2x(f"out[{bi}]", out[bi], o_ref[j], o_ref[j].to(torch.float16))
            assert_lse(lse[bi], l_ref[j])
        assert torch.equal(kcd[1], kc[1]) and torch.equal(kcd[3], kc[3])  # rows no valid sequence uses
        with pytest.raises(RuntimeError, match="cache_batch_idx entries must be within cache batch bounds"):
            fai.flash_attn_kvcache_check(device)
        fai.flash_attn_kvcache_check(device)


@pytest.mark.gpu
def test_nosync_decode_step_in_hip_graph(device):
    gen = torch.Generator().manual_seed(7300)
    b, h, hk, hd, cap, page = 4, 8, 2, 128, 1024, 256
    q0, kc0, vc0, k0, v0, table = _inputs(b, 1, h, hk, hd, cap, 1, gen, paged=True)
    q, k, v = q0.to(device), k0.to(device), v0.to(device)
    kc, vc, tbl = kc0.to(device), vc0.to(device), table.to(device)
    seqlens = torch.tensor([5, 300, 1000, 0], dtype=torch.int32, device=device)
    fai.flash_attn_kvcache_check(device)  # allocates the status word before capture
    args = dict(block_table=tbl, causal=True, num_splits=0, return_softmax_lse=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the graph
        fai.flash_attn_with_kvcache(q, kc.clone(), vc.clone(), k, v, cache_seqlens=seqlens, validate=False, **args)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, lse_g = fai.flash_attn_with_kvcache(q, kc, vc, k, v, cache_seqlens=seqlens, validate=False, **args)
    steps = [[5, 300, 1000, 0], [6, 301, 700, 1], [1023, 2, 512, 256], [7, 1024, 3, 9]]
    for i, lens in enumerate(steps):
        seqlens.copy_(torch.tensor(lens, dtype=torch.int32))
        q.copy_(randn16(tuple(q.shape), gen))
        k.copy_(randn16(tuple(k.shape), gen))
        v.copy_(randn16(tuple(v.shape), gen))
        kc_before, vc_before = kc.clone(), vc.clone()
        graph.replay()
        torch.cuda.synchronize()
        kr, vr = kc_before.clone(), vc_before.clone()
        # Each replay against the oracle (append + split-KV over the logical cache).
        ok = [i for i, n in enumerate(lens) if n + 1 <= cap]
        sel = torch.tensor(ok)
        o_ref, l_ref, _, _ = kv_oracle(q.cpu()[sel], kc_before.cpu(), vc_before.cpu(), k.cpu()[sel], v.cpu()[sel],
                                       torch.tensor(lens, dtype=torch.int32)[sel], None, tbl.cpu()[sel], True, 0, None)
        for j, bi in enumerate(ok):
            assert_2x(f"replay {i} out[{bi}]", out_g[bi].cpu(), o_ref[j], o_ref[j].to(torch.float16))
            assert_lse(lse_g[bi].cpu(), l_ref[j])
        if max(lens) + 1 <= cap:
            out_r, lse_r = fai.flash_attn_with_kvcache(q, kr, vr, k, v, cache_seqlens=seqlens, **args)
            torch.cuda.synchronize()
            assert torch.equal(out_g, out_r) and torch.equal(lse_g, lse_r), f"replay {i}"
            assert torch.equal(kc, kr) and torch.equal(vc, vr), f"replay {i}"
            fai.flash_attn_kvcache_check(device)
        else:
            # Sequence 1 would overflow: untouched and zero, the rest as before.
            assert not out_g[1].any() and not lse_g[1].any()
            with pytest.raises(ValueError, match="cache capacity is insufficient"):
                fai.flash_attn_kvcache_check(device)
