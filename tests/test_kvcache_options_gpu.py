"""Local windows, softcap, ALiBi, cache_leftpad and rotary embeddings in
flash_attn_with_kvcache (upstream FlashAttention semantics; the reference's
signature takes these but rejects them, flash_attention_interface.py:617-634)
against the extended CPU oracle.  Rotated keys land in the cache bit for bit
as the oracle rotates them.

Bound: as for the other KV-cache outputs (the kernels are fp32 until the final
fp16 rounding), 2x the error of the fp16-rounded oracle; LSE to fp32 precision.
Cases cover paged and contiguous / remapped caches, one and several query
tokens (several go through the split kernel too), GQA, explicit and heuristic
split counts, and a long cache whose splits mostly fall outside the window
(the kernel skips those tiles)."""

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, assert_lse, randn16
from oracle import kvcache as okv

CASES = [
    # b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, softcap
    (3, 1, 8, 2, 128, 1024, 1, True, 0, True, False, (100, -1), 0.0),
    (3, 1, 8, 2, 128, 1024, 1, True, 4, False, False, (0, 0), 0.0),
    (2, 4, 8, 8, 64, 512, 4, True, 1, False, True, (37, 0), 0.0),
    (2, 4, 8, 8, 64, 512, 4, False, 2, False, False, (5, 3), 0.0),
    (3, 1, 8, 2, 128, 1024, 1, True, 8, True, False, (-1, -1), 30.0),
    (2, 3, 6, 2, 64, 512, 3, True, 0, False, True, (64, -1), 5.0),
    (2, 1, 8, 2, 128, 4096, 1, True, 16, True, False, (300, -1), 0.0),
    (2, 5, 4, 1, 128, 768, 0, True, 3, False, False, (2000, 1), 1.5),
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,h,hk,hd,cap,new,causal,splits,paged,remap,window,softcap", CASES)
def test_kvcache_window_softcap(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, softcap):
    _check(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, softcap, None, False)


CASES_ALIBI_LEFTPAD = [
    # b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, softcap, alibi, leftpad
    (3, 1, 8, 2, 128, 1024, 1, True, 0, True, False, (-1, -1), 0.0, "h", False),
    (2, 4, 8, 8, 64, 512, 4, False, 2, False, True, (-1, -1), 0.0, "bh", False),
    (3, 1, 8, 2, 128, 1024, 1, True, 4, False, False, (-1, -1), 0.0, None, True),
    (2, 4, 6, 2, 64, 512, 4, True, 1, False, True, (-1, -1), 0.0, None, True),
    (2, 3, 8, 2, 128, 768, 3, True, 3, True, False, (50, -1), 10.0, "h", True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,h,hk,hd,cap,new,causal,splits,paged,remap,window,softcap,alibi,leftpad",
                         CASES_ALIBI_LEFTPAD)
def test_kvcache_alibi_leftpad(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, softcap,
                               alibi, leftpad):
    _check(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, softcap, alibi, leftpad)


CASES_ROTARY = [
    # b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, rotary_dim, interleaved, leftpad
    (3, 1, 8, 2, 128, 1024, 1, True, 0, True, False, (-1, -1), 128, False, False),
    (3, 1, 8, 2, 128, 1024, 1, True, 4, False, True, (-1, -1), 64, True, False),
    (2, 4, 8, 8, 64, 512, 4, True, 1, False, False, (-1, -1), 64, False, False),
    (2, 4, 8, 8, 64, 512, 4, False, 2, True, False, (-1, -1), 32, True, False),
    (2, 3, 6, 2, 64, 512, 2, False, 0, False, True, (40, 7), 48, False, True),
    (2, 5, 4, 1, 128, 768, 5, True, 3, True, False, (-1, -1), 80, True, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("b,sq,h,hk,hd,cap,new,causal,splits,paged,remap,window,rotary_dim,interleaved,leftpad",
                         CASES_ROTARY)
def test_kvcache_rotary(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, rotary_dim,
                        interleaved, leftpad):
    _check(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, 0.0, None, leftpad,
           rotary=(rotary_dim, interleaved))


@pytest.mark.gpu
@pytest.mark.parametrize("interleaved", [False, True])
def test_kvcache_rotary_column_sliced_tables(device, interleaved):
    """cos / sin passed as column slices of wider tables (rows not packed): the
    host layer hands the kernels packed copies, so the angles are the slices'."""
    _check(device, 3, 2, 8, 2, 128, 1024, 2, True, 2, True, False, (-1, -1), 0.0, None, False,
           rotary=(64, interleaved), sliced=True)


@pytest.mark.gpu
def test_kvcache_rotary_needs_new_keys(device):
    q = torch.zeros((1, 1, 4, 64), dtype=torch.float16, device=device)
    kc = torch.zeros((1, 256, 1, 64), dtype=torch.float16, device=device)
    tab = torch.zeros((256, 16), dtype=torch.float16, device=device)
    with pytest.raises(RuntimeError, match="new key / value to be appended"):
        fai.flash_attn_with_kvcache(q, kc, kc.clone(), rotary_cos=tab, rotary_sin=tab,
                                    cache_seqlens=torch.ones(1, dtype=torch.int32, device=device))
    k = torch.zeros((1, 1, 1, 64), dtype=torch.float16, device=device)
    with pytest.raises(RuntimeError, match="divisible by 16"):
        fai.flash_attn_with_kvcache(q, kc, kc.clone(), k, k, rotary_cos=tab[:, :12], rotary_sin=tab[:, :12],
                                    cache_seqlens=torch.ones(1, dtype=torch.int32, device=device))


def _check(device, b, sq, h, hk, hd, cap, new, causal, splits, paged, remap, window, softcap, alibi, leftpad,
           rotary=None, sliced=False):
    g = torch.Generator().manual_seed(8000 + b * 13 + sq + hd + cap // 256 + (alibi is not None) + 2 * leftpad
                                      + (0 if rotary is None else rotary[0]))
    rows = b + 2 if remap else b
    kc = randn16((rows, cap, hk, hd), g)
    vc = randn16((rows, cap, hk, hd), g)
    q = randn16((b, sq, h, hd), g)
    k = randn16((b, new, hk, hd), g) if new else None
    v = randn16((b, new, hk, hd), g) if new else None
    seqlens = torch.randint(max(0, sq - new), cap - new + 1, (b,), generator=g, dtype=torch.int32)
    seqlens[0] = cap - new
    batch_idx = torch.randperm(rows, generator=g)[:b].to(torch.int32) if remap else None
    slopes = None
    if alibi == "h":
        slopes = torch.rand((h,), generator=g) * 0.5
    elif alibi == "bh":
        slopes = torch.rand((b, h), generator=g) * 0.5
    lpad = torch.randint(0, 64, (b,), generator=g, dtype=torch.int32) if leftpad else None
    cos = sin = None
    if rotary is not None:
        ang = torch.rand((cap, rotary[0] // 2), generator=g, dtype=torch.float64) * 2 * torch.pi
        cos, sin = torch.cos(ang).to(torch.float16), torch.sin(ang).to(torch.float16)
    cos_d = sin_d = None
    if cos is not None:
        cos_d, sin_d = cos.to(device), sin.to(device)
        if sliced:  # the first rotary_dim / 2 columns of tables 16 columns wider
            wide = torch.zeros((2, cap, rotary[0] // 2 + 16), dtype=torch.float16, device=device)
            wide[0, :, : rotary[0] // 2], wide[1, :, : rotary[0] // 2] = cos_d, sin_d
            cos_d, sin_d = wide[0, :, : rotary[0] // 2], wide[1, :, : rotary[0] // 2]
            assert not cos_d.is_contiguous()
    table = None
    kcp, vcp = kc, vc
    if paged:
        nb = cap // 256
        table = torch.randperm(b * nb, generator=g).reshape(b, nb).to(torch.int32)
        kcp = torch.zeros((b * nb, 256, hk, hd), dtype=torch.float16)
        vcp = torch.zeros_like(kcp)
        for bi in range(b):
            for j in range(nb):
                kcp[table[bi, j]] = kc[bi, j * 256 : (j + 1) * 256]
                vcp[table[bi, j]] = vc[bi, j * 256 : (j + 1) * 256]
    kcd, vcd = kcp.clone().to(device), vcp.clone().to(device)
    out, lse = fai.flash_attn_with_kvcache(
        q.to(device), kcd, vcd, None if k is None else k.to(device), None if v is None else v.to(device),
        cache_seqlens=seqlens.to(device), cache_batch_idx=None if batch_idx is None else batch_idx.to(device),
        block_table=None if table is None else table.to(device), causal=causal, num_splits=splits,
        window_size=window, softcap=softcap, return_softmax_lse=True,
        alibi_slopes=None if slopes is None else slopes.to(device),
        cache_leftpad=None if lpad is None else lpad.to(device),
        rotary_cos=cos_d, rotary_sin=sin_d,
        rotary_interleaved=True if rotary is None else rotary[1],
    )
    torch.cuda.synchronize()
    # Oracle: append, materialise the logical caches, attend.
    kr, vr = kcp.clone(), vcp.clone()
    # Upstream's normalisation of bounds at least the capacity.
    w = tuple(-1 if x >= cap else x for x in window)
    if rotary is not None:
        k = okv.rotary_embed(k, cos, sin, okv.rotary_positions(seqlens, new, True), rotary[1])
        q = okv.rotary_embed(q, cos, sin, okv.rotary_positions(seqlens, sq, causal or w != (-1, -1)), rotary[1])
    if k is not None:
        if table is None:
            okv.append_contiguous(kr, vr, k, v, seqlens, batch_idx)
        else:
            okv.append_paged(kr, vr, k, v, seqlens, table)
    assert torch.equal(kcd.cpu(), kr) and torch.equal(vcd.cpu(), vr), "append differs from the oracle"
    ends = seqlens + new
    ku, vu = okv.materialize(kr, vr, ends, batch_idx, table)
    o_ref, l_ref = okv.splitkv_attention(q, ku, vu, ends, hd ** -0.5, causal, max(splits, 1), window=w,
                                         softcap=softcap, alibi_slopes=slopes, leftpad=lpad)
    assert_2x("out", out.cpu(), o_ref, o_ref.to(torch.float16))
    assert_lse(lse.cpu(), l_ref)
