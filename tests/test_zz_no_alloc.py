"""fa_fwd_kvcache_noalloc (the allocation-free decode entry point) through the
C ABI (collected last: it must pass alone and after every other test): same
outputs, LSE and appended cache, bit for bit, as fa_fwd_kvcache with a caller
workspace, on two calls in a row (the second smaller, so it runs over the
first call's leftover scratch contents), with one split (no accumulators) and
with splits; the process's first call made inside a HIP graph capture (the
device's scratch address is looked up then) and the graph replayed with new
cache lengths; a request beyond the static scratch returns FA_ERR_SCRATCH
without launching anything."""

import ctypes

import pytest
import torch

import fa_capi
from helpers import randn16


def _inputs(g, b, sq, h, hk, hd, cap, paged, page=256):
    q = randn16((b, sq, h, hd), g)
    k, v = randn16((b, sq, hk, hd), g), randn16((b, sq, hk, hd), g)
    if paged:
        nb = cap // page
        kc, vc = randn16((b * nb, page, hk, hd), g), randn16((b * nb, page, hk, hd), g)
        table = torch.randperm(b * nb, generator=g).reshape(b, nb).to(torch.int32)
    else:
        kc, vc = randn16((b, cap, hk, hd), g), randn16((b, cap, hk, hd), g)
        table = None
    lens = torch.randint(0, cap - sq + 1, (b,), generator=g, dtype=torch.int32)
    lens[0] = cap - sq
    return q, k, v, kc, vc, table, lens


def _call(device, name, inp, splits, workspace):
    q, k, v, kc, vc, table, lens = inp
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    kcd, vcd = kc.to(device), vc.to(device)
    o = torch.full_like(qd, 3.0)
    b, sq, h, hd = q.shape
    lse = torch.full((b, h, sq), 3.0, dtype=torch.float32, device=device)
    rows = b * h * sq
    acc = oa = la = order = counts = None
    if workspace:
        acc = torch.empty((max(splits, 1) * rows * (hd + 1),), dtype=torch.float32, device=device)
        oa, la = (acc, acc[splits * rows * hd:]) if splits > 1 else (None, None)
        order = torch.empty((b + 1,), dtype=torch.int32, device=device)
        counts = torch.empty((b * h * ((sq + 31) // 32),), dtype=torch.int32, device=device)
    a = fa_capi.kvcache_args(qd, kcd, vcd, o, lse, lens.to(device), hd ** -0.5, True, splits, kd, vd,
                             block_table=None if table is None else table.to(device), out_accum=oa, lse_accum=la,
                             batch_order=order, split_count=counts)
    if workspace:
        assert fa_capi.load().fa_kv_split_count_len(ctypes.byref(a)) <= counts.numel()
    print(f"{name}: b={b} sq={sq} h={h} hd={hd} splits={splits}", flush=True)
    fa_capi.call(name, a)
    torch.cuda.synchronize()
    return o.cpu(), lse.cpu(), kcd.cpu(), vcd.cpu()


@pytest.mark.gpu
def test_noalloc_first_call_under_graph_capture(device):
    # Defined first in the last-collected file: the process's first noalloc call
    # happens inside the capture (nothing else calls it).  Paged decode, 8
    # sequences, 32 / 8 heads, 4 splits; the graph is replayed three times with
    # new lengths (eager copies and a synchronisation between replays), each
    # replay against fa_fwd_kvcache with a caller workspace on the same inputs.
    g = torch.Generator().manual_seed(9902)
    q, k, v, kc, vc, table, lens = _inputs(g, 8, 1, 32, 8, 128, 2048, True)
    splits = 4
    qd, kd, vd, td = q.to(device), k.to(device), v.to(device), table.to(device)
    kc0, vc0 = kc.to(device), vc.to(device)
    kcd, vcd = kc0.clone(), vc0.clone()
    seq_d = lens.to(device)
    o = torch.zeros_like(qd)
    lse = torch.zeros((8, 32, 1), dtype=torch.float32, device=device)
    a = fa_capi.kvcache_args(qd, kcd, vcd, o, lse, seq_d, 128 ** -0.5, True, splits, kd, vd, block_table=td)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("noalloc: first call inside torch.cuda.graph capture", flush=True)
    with torch.cuda.graph(graph):
        fa_capi.call("fa_fwd_kvcache_noalloc", a)
    torch.cuda.synchronize()
    for rep in range(3):
        new_lens = torch.randint(0, 2048, (8,), generator=g, dtype=torch.int32)
        new_lens[rep] = 2047
        seq_d.copy_(new_lens.to(device))
        kcd.copy_(kc0)
        vcd.copy_(vc0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = _call(device, "fa_fwd_kvcache", (q, k, v, kc, vc, table, new_lens), splits, True)
        for n, r, x in zip(("out", "lse", "k_cache", "v_cache"), ref, (o.cpu(), lse.cpu(), kcd.cpu(), vcd.cpu())):
            assert torch.equal(r, x), f"replay {rep}: {n} differs from fa_fwd_kvcache"
    del graph


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(device):
    g = torch.Generator().manual_seed(9900)
    # First call: paged decode, 64 sequences, 8 splits (8.5 MB of accumulators); then a
    # smaller contiguous multi-token call over the same scratch; then one split.
    runs = [
        (_inputs(g, 64, 1, 32, 8, 128, 4096, True), 8),
        (_inputs(g, 3, 4, 8, 8, 64, 1024, False), 3),
        (_inputs(g, 2, 1, 8, 2, 128, 512, True), 1),
    ]
    for inp, splits in runs:
        ref = _call(device, "fa_fwd_kvcache", inp, splits, True)
        got = _call(device, "fa_fwd_kvcache_noalloc", inp, splits, False)
        for n, r, x in zip(("out", "lse", "k_cache", "v_cache"), ref, got):
            assert torch.equal(r, x), f"{n} differs from fa_fwd_kvcache"


@pytest.mark.gpu
def test_noalloc_rejects_requests_beyond_the_scratch(device):
    # 128 splits x 64 x 32 rows x 129 floats = 135 MB > 16 MiB: refused before any launch.
    g = torch.Generator().manual_seed(9901)
    q, k, v, kc, vc, table, lens = _inputs(g, 64, 1, 32, 8, 128, 1024, True)
    o = torch.zeros_like(q).to(device)
    lse = torch.zeros((64, 32, 1), dtype=torch.float32, device=device)
    a = fa_capi.kvcache_args(q.to(device), kc.to(device), vc.to(device), o, lse, lens.to(device), 0.1, True, 128,
                             k.to(device), v.to(device), block_table=table.to(device))
    rc = fa_capi.load().fa_fwd_kvcache_noalloc(ctypes.byref(a), ctypes.c_void_p(fa_capi.stream_handle()))
    assert rc == fa_capi.FA_ERR_SCRATCH
    assert b"static scratch" in fa_capi.load().fa_error_string(rc)
    torch.cuda.synchronize()
    assert not o.any()
