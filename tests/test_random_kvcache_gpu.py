"""Seeded random KV-cache calls on the GPU against the oracle.

The KV-cache tests follow the reference's case list (test_flash_attn.py:1104-1964);
these draw the call instead: batch, query tokens, appended tokens, query and kv
heads, head_dim, capacity, cache lengths (one sequence at full capacity, empty
ones allowed), causal or not, num_splits (0 = the heuristic), contiguous,
remapped (cache_batch_idx) or paged (shuffled block table), each case from its
own fixed seed.  Eight "large" calls have enough work items for the split
kernel to take two or four KV heads per item.  Each call is checked as the
fixed cases are: the cache after the append bit for bit against the oracle
append, the output within 2x the reference's own error, the LSE to fp32
precision.
"""

import random

import pytest
import torch

from helpers import assert_2x, assert_lse, kv_oracle, randn16
from test_kvcache_gpu import _paged_from_contiguous, _run


def _case(i, large):
    r = random.Random(7700 + i)
    hd = r.choice([64, 128])
    if large:
        b, hk, sq = r.choice([48, 64]), 8, 1
        h = hk * r.choice([1, 4])
        cap = r.choice([1024, 2048])
        splits = r.choice([8, 12, 16])
        new, causal, paged, remap = 1, True, r.random() < 0.5, False
    else:
        b = r.randint(1, 8)
        hk = r.choice([1, 2, 4, 8])
        h = hk * r.choice([1, 2, 4])
        sq = r.choice([1, 1, 1, 2, 4, r.randint(1, 16)])
        cap = r.choice([256, 512, 1024, 2048])
        new = r.randint(0, min(sq, 4))
        causal = r.random() < 0.7
        splits = r.choice([0, 0, 1, r.randint(2, 16)])
        paged = r.random() < 0.4
        remap = not paged and r.random() < 0.4
    return b, sq, h, hk, hd, cap, new, causal, splits, paged, remap


CASES = [(i, False) for i in range(40)] + [(i, True) for i in range(40, 48)]


def test_random_kv_cases_are_fixed():
    """Two draws pinned (a changed generator would change every case); the list covers
    paged, remapped and contiguous caches, appends and no appends, both head dims."""
    assert _case(0, False) == (3, 1, 8, 2, 128, 512, 0, False, 0, True, False)
    assert _case(40, True) == (48, 1, 32, 8, 128, 2048, 1, True, 16, False, False)
    cs = [_case(i, large) for i, large in CASES]
    assert any(c[9] for c in cs) and any(c[10] for c in cs) and any(not c[9] and not c[10] for c in cs)
    assert any(c[6] == 0 for c in cs) and any(c[6] > 0 for c in cs)
    assert {c[4] for c in cs} == {64, 128}


@pytest.mark.gpu
@pytest.mark.parametrize("idx,large", CASES)
def test_random_kvcache_call(device, idx, large):
    b, sq, h, hk, hd, cap, new, causal, splits, paged, remap = _case(idx, large)
    print(f"kv case {idx}: b{b} sq{sq} h{h}/{hk} d{hd} cap{cap} new{new} causal={causal} splits={splits} "
          f"paged={paged} remap={remap}", flush=True)
    g = torch.Generator().manual_seed(7800 + idx)
    rows = b + 3 if remap else b
    kc = randn16((rows, cap, hk, hd), g)
    vc = randn16((rows, cap, hk, hd), g)
    q = randn16((b, sq, h, hd), g)
    k = randn16((b, new, hk, hd), g) if new else None
    v = randn16((b, new, hk, hd), g) if new else None
    seqlens = torch.randint(0, cap - new + 1, (b,), generator=g, dtype=torch.int32)
    seqlens[0] = cap - new  # one sequence at full capacity
    if b > 2:
        seqlens[1] = 0  # and one with an empty cache
    batch_idx = torch.randperm(rows, generator=g)[:b].to(torch.int32) if remap else None
    table = None
    if paged:
        kc, vc, table = _paged_from_contiguous(kc, vc, seqlens, 256, g)
    out, lse, kc_after, vc_after = _run(device, q, kc, vc, k, v, seqlens, batch_idx, table, causal, splits)
    o_ref, l_ref, kc_ref, vc_ref = kv_oracle(q, kc, vc, k, v, seqlens, batch_idx, table, causal, splits, None)
    assert torch.equal(kc_after, kc_ref), "k_cache after append differs from the oracle append"
    assert torch.equal(vc_after, vc_ref), "v_cache after append differs from the oracle append"
    assert_2x("out", out, o_ref, o_ref.to(torch.float16))
    assert_lse(lse, l_ref)
