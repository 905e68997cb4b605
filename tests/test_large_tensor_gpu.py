"""Tensors past 2^31 elements on the GPU, against the fp32 oracle (2x-twin bound).

Q, O, dO and dQ of b2 x 262208 x 32 heads x 128 hold 2.148e9 fp16 elements each (4.3 GB), past 2^31, so
any 32-bit element offset in the forward, dQ or dK/dV kernels would wrap.  K and V have 8 heads (GQA
32 / 8), causal.  Checked against the oracle: batch row 1's last 64 query rows (every element of them lies
past 2^31), whose outputs, LSE and dQ depend only on those rows and all keys, and the last 64 keys of that
row, whose dK / dV depend only on the queries at or after them, i.e. the same 64 rows; for KV head 7 and
its query heads 28-31.  The inputs are drawn on the GPU (seeded N(0, 1) in fp16).

The KV-cache calls at the end do the same for the decode path: caches of more than 2^31 elements per
tensor, contiguous (read through cache_batch_idx, the first sequence in the last rows) and paged (the
first sequence's pages the cache's last ones).
"""

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, assert_lse

B, S, H, HK, D = 2, 262208, 32, 8, 128
TAIL = 64


def test_large_shape_is_past_2_31_elements():
    assert B * S * H * D > 2 ** 31
    # the checked rows start past element 2^31 of Q
    assert ((1 * S + S - TAIL) * H) * D > 2 ** 31


@pytest.mark.gpu
def test_fwd_bwd_past_2_31_elements(device):
    from oracle.attention import attention_bwd, attention_fwd, bwd_fp32_noise
    from oracle.twin import bwd_twin, fwd_twin

    gen = torch.Generator(device=device).manual_seed(4242)
    q = torch.randn((B, S, H, D), generator=gen, device=device, dtype=torch.float16)
    k = torch.randn((B, S, HK, D), generator=gen, device=device, dtype=torch.float16)
    v = torch.randn((B, S, HK, D), generator=gen, device=device, dtype=torch.float16)
    do = torch.randn((B, S, H, D), generator=gen, device=device, dtype=torch.float16)
    scale = D ** -0.5
    print(f"large tensors: b{B} s{S} h{H}/{HK} d{D} causal, Q {q.numel()} elements", flush=True)
    out, lse = fai._flash_attn_forward(q, k, v, scale, True)
    dq, dk, dv = fai._flash_attn_backward(do, q, k, v, out, lse, scale, True)
    torch.cuda.synchronize()

    hq, hkv, rows = slice(28, 32), slice(7, 8), slice(S - TAIL, S)
    qs = q[1:2, rows, hq].cpu()
    dos = do[1:2, rows, hq].cpu()
    ks, vs = k[1:2, :, hkv].cpu(), v[1:2, :, hkv].cpu()
    del q, k, v, do
    # 64 query rows against every key, bottom-right causal: the global mask of those rows.
    o_ref, l_ref = attention_fwd(qs, ks, vs, scale, True)
    o_tw, l_tw = fwd_twin(qs, ks, vs, scale, True)
    assert_2x("out", out[1:2, rows, hq].cpu(), o_ref, o_tw)
    assert_lse(lse[1:2, hq, rows].cpu(), l_ref)
    g_ref = attention_bwd(qs, ks, vs, o_ref, l_ref, dos, scale, True)
    g_tw = bwd_twin(qs, ks, vs, o_tw, l_tw, dos, scale, True)
    noise = bwd_fp32_noise(qs, ks, vs, o_ref, l_ref, dos, scale, True, dt=torch.float32)
    assert_2x("dq", dq[1:2, rows, hq].cpu(), g_ref[0], g_tw[0], noise[0])
    # The last TAIL keys are seen by these rows only.
    for name, got, i in (("dk", dk, 1), ("dv", dv, 2)):
        assert_2x(name, got[1:2, rows, hkv].cpu(), g_ref[i][:, rows], g_tw[i][:, rows], noise[i][:, rows])


# KV caches past 2^31 elements per tensor: 16 rows x 131328 positions x 8 heads x 128 (contiguous), and
# 8256 pages of 256 positions (paged), 2.15e9 fp16 elements (4.3 GB) each for K and V.
KV_ROWS, KV_CAP, KV_HK, KV_H, KV_D = 16, 131328, 8, 32, 128
KV_PAGES, KV_PAGE = 8256, 256


def test_large_kv_shapes_are_past_2_31_elements():
    assert KV_ROWS * KV_CAP * KV_HK * KV_D > 2 ** 31
    assert KV_PAGES * KV_PAGE * KV_HK * KV_D > 2 ** 31
    # the first sequence's append position lies past 2^31: row 15, position KV_CAP - 1 (contiguous), and
    # the last page (paged)
    assert (15 * KV_CAP + KV_CAP - 1) * KV_HK * KV_D > 2 ** 31
    assert (KV_PAGES - 1) * KV_PAGE * KV_HK * KV_D > 2 ** 31


@pytest.mark.gpu
@pytest.mark.parametrize("paged", [False, True])
def test_kvcache_past_2_31_elements(device, paged):
    """A decode call (one query token, one appended token, 16 splits, causal) on a cache past 2^31
    elements; the append, output and LSE against the oracle run on the rows / pages the call uses."""
    from helpers import kv_oracle

    gen = torch.Generator(device=device).manual_seed(4343 + int(paged))
    shape = (KV_PAGES, KV_PAGE, KV_HK, KV_D) if paged else (KV_ROWS, KV_CAP, KV_HK, KV_D)
    kc = torch.randn(shape, generator=gen, device=device, dtype=torch.float16)
    vc = torch.randn(shape, generator=gen, device=device, dtype=torch.float16)
    b = 4
    q = torch.randn((b, 1, KV_H, KV_D), generator=gen, device=device, dtype=torch.float16)
    kn = torch.randn((b, 1, KV_HK, KV_D), generator=gen, device=device, dtype=torch.float16)
    vn = torch.randn((b, 1, KV_HK, KV_D), generator=gen, device=device, dtype=torch.float16)
    seqlens = torch.tensor([KV_CAP - 1, KV_CAP - 700, 65000, 131000], dtype=torch.int32)
    print(f"large KV cache ({'paged' if paged else 'contiguous'}): {kc.numel()} elements per tensor", flush=True)
    if paged:
        # Each sequence owns KV_CAP / KV_PAGE consecutive pages; the first sequence's are the cache's last.
        per = KV_CAP // KV_PAGE
        starts = [KV_PAGES - per, 0, 2 * per, 5 * per]
        table = torch.stack([torch.arange(s0, s0 + per, dtype=torch.int32) for s0 in starts])
        used = torch.cat([table[s] for s in range(b)]).long()
        k_sub, v_sub = kc[used.to(device)].cpu(), vc[used.to(device)].cpu()  # the pages, in table order
        sub_table = torch.arange(b * per, dtype=torch.int32).reshape(b, per)
        out, lse = fai.flash_attn_with_kvcache(q, kc, vc, kn, vn, cache_seqlens=seqlens.to(device),
                                               block_table=table.to(device), causal=True, num_splits=16,
                                               return_softmax_lse=True)
        torch.cuda.synchronize()
        k_after, v_after = kc[used.to(device)].cpu(), vc[used.to(device)].cpu()
        o_ref, l_ref, k_ref, v_ref = kv_oracle(q.cpu(), k_sub, v_sub, kn.cpu(), vn.cpu(), seqlens, None,
                                               sub_table, True, 16, None)
    else:
        rows = torch.tensor([15, 14, 3, 0], dtype=torch.int32)
        k_sub, v_sub = kc[rows.long().to(device)].cpu(), vc[rows.long().to(device)].cpu()
        out, lse = fai.flash_attn_with_kvcache(q, kc, vc, kn, vn, cache_seqlens=seqlens.to(device),
                                               cache_batch_idx=rows.to(device), causal=True, num_splits=16,
                                               return_softmax_lse=True)
        torch.cuda.synchronize()
        k_after, v_after = kc[rows.long().to(device)].cpu(), vc[rows.long().to(device)].cpu()
        o_ref, l_ref, k_ref, v_ref = kv_oracle(q.cpu(), k_sub, v_sub, kn.cpu(), vn.cpu(), seqlens, None, None,
                                               True, 16, None)
    assert torch.equal(k_after, k_ref), "k_cache after append differs from the oracle append"
    assert torch.equal(v_after, v_ref), "v_cache after append differs from the oracle append"
    assert_2x("out", out.cpu(), o_ref, o_ref.to(torch.float16))
    assert_lse(lse.cpu(), l_ref)
