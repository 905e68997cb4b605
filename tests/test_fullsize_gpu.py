"""Parity at the BASELINE configurations' full sizes (c1-c5), on the GPU.

The kernels run on the whole workload; the fp32 oracle and the
rounding-point twin are evaluated on the CPU for the parts that finish in
seconds there:

* c1 (b2 s512 h8 d64, non-causal forward): every element;
* c2 (b4 s4096 h16 d128 causal, forward + backward): every element of batch
  rows 0 and 3 (rows of a batch are independent, so each is the full
  computation of that row at the full sequence length and head count);
* c3 (16 packed causal sequences, 32/8 heads): every element of the shortest,
  the median-length and the longest sequence;
* c4 (paged decode with append, 64 sequences up to 32k keys, 8 splits) and c5
  (4 remapped rows of an 8 x 131072 contiguous cache, 4 new tokens, 16 splits):
  every output and LSE, the appended K/V bit-exact, and every other cache
  position unchanged.

Bounds as in the small-size tests: 2x the twin's error (+ the fp32 noise
floor for the backward), LSE to 2e-5 relative, bit-exact cache writes.
"""

import time

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, assert_lse, cu_from_lengths, randn16, varlen_lengths
from oracle import kvcache as okv
from oracle.attention import attention_bwd, attention_fwd, bwd_fp32_noise
from oracle.twin import bwd_twin, fwd_twin


def _log(msg):
    print(f"[fullsize] {msg}", flush=True)


def _check_fwd_bwd(tag, q, k, v, do, out, dq, dk, dv, scale, causal):
    t = time.time()
    o_ref, l_ref = attention_fwd(q, k, v, scale, causal)
    o_tw, l_tw = fwd_twin(q, k, v, scale, causal)
    assert_2x(f"{tag} out", out, o_ref, o_tw)
    if dq is None:
        _log(f"{tag}: forward checked in {time.time() - t:.1f} s")
        return o_ref, l_ref
    g_ref = attention_bwd(q, k, v, o_ref, l_ref, do, scale, causal)
    g_tw = bwd_twin(q, k, v, o_tw, l_tw, do, scale, causal)
    noise = bwd_fp32_noise(q, k, v, o_ref, l_ref, do, scale, causal, dt=torch.float32)
    for name, got, r, tw, nz in zip(("dq", "dk", "dv"), (dq, dk, dv), g_ref, g_tw, noise):
        assert_2x(f"{tag} {name}", got, r, tw, nz)
    _log(f"{tag}: forward and backward checked in {time.time() - t:.1f} s")
    return o_ref, l_ref


@pytest.mark.gpu
def test_c1_full_forward(device):
    g = torch.Generator().manual_seed(11)
    q, k, v = (randn16((2, 512, 8, 64), g) for _ in range(3))
    _log("c1: b2 s512 h8 d64 non-causal")
    out, lse = fai._flash_attn_forward(q.to(device), k.to(device), v.to(device), 64 ** -0.5, False)
    torch.cuda.synchronize()
    _, l_ref = _check_fwd_bwd("c1", q, k, v, None, out.cpu(), None, None, None, 64 ** -0.5, False)
    assert_lse(lse.cpu(), l_ref)


@pytest.mark.gpu
def test_c2_full_forward_backward(device):
    b, s, h, d = 4, 4096, 16, 128
    g = torch.Generator().manual_seed(12)
    q, k, v, do = (randn16((b, s, h, d), g) for _ in range(4))
    _log("c2: b4 s4096 h16 d128 causal fwd + bwd on the GPU")
    qd, kd, vd = (t.to(device).requires_grad_() for t in (q, k, v))
    out = fai.flash_attn_func(qd, kd, vd, causal=True)
    out.backward(do.to(device))
    # The same forward again for its LSE (the kernels are deterministic).
    out2, lse = fai._flash_attn_forward(qd.detach(), kd.detach(), vd.detach(), d ** -0.5, True)
    torch.cuda.synchronize()
    assert torch.equal(out2, out.detach())
    assert all(torch.isfinite(t).all() for t in (out, qd.grad, kd.grad, vd.grad))
    for r in (0, 3):  # checked batch rows
        sl = slice(r, r + 1)
        _, l_ref = _check_fwd_bwd(
            f"c2 row {r}", q[sl], k[sl], v[sl], do[sl], out.detach()[sl].cpu(), qd.grad[sl].cpu(),
            kd.grad[sl].cpu(), vd.grad[sl].cpu(), d ** -0.5, True,
        )
        assert_lse(lse[sl].cpu(), l_ref)


@pytest.mark.gpu
def test_c3_full_varlen_gqa(device):
    h, hk, d = 32, 8, 128
    lens = varlen_lengths(16, 128, 4096, seed=13)
    cu = cu_from_lengths(lens)
    total, mx = int(cu[-1]), max(lens)
    g = torch.Generator().manual_seed(14)
    q = randn16((total, h, d), g)
    k = randn16((total, hk, d), g)
    v = randn16((total, hk, d), g)
    do = randn16((total, h, d), g)
    _log(f"c3: 16 packed causal sequences ({total} tokens, max {mx}), 32/8 heads, fwd + bwd on the GPU")
    qd, kd, vd = (t.to(device).requires_grad_() for t in (q, k, v))
    cud = cu.to(device)
    out = fai.flash_attn_varlen_func(qd, kd, vd, cud, cud, mx, mx, causal=True)
    out.backward(do.to(device))
    out2, lse = fai._flash_attn_varlen_forward(qd.detach(), kd.detach(), vd.detach(), cud, cud, mx, mx, d ** -0.5, True)
    torch.cuda.synchronize()
    assert torch.equal(out2, out.detach())
    order = sorted(range(16), key=lambda i: lens[i])
    for i in (order[0], order[8], order[-1]):
        a, e = int(cu[i]), int(cu[i + 1])
        _, l_ref = _check_fwd_bwd(
            f"c3 seq {i} (n={e - a})", q[a:e][None], k[a:e][None], v[a:e][None], do[a:e][None],
            out.detach()[a:e][None].cpu(), qd.grad[a:e][None].cpu(), kd.grad[a:e][None].cpu(), vd.grad[a:e][None].cpu(),
            d ** -0.5, True,
        )
        assert_lse(lse[i : i + 1, :, : e - a].cpu(), l_ref)


def _check_kvcache(tag, device, q, k_cache, v_cache, k_new, v_new, seqlens, batch_idx, table, splits):
    """Run flash_attn_with_kvcache on the device-resident cache and check the
    append (bit-exact, nothing else touched) and the attention (vs the oracle)."""
    kc0, vc0 = k_cache.clone(), v_cache.clone()
    t = time.time()
    out, lse = fai.flash_attn_with_kvcache(
        q.to(device), k_cache, v_cache, k_new.to(device), v_new.to(device), cache_seqlens=seqlens.to(device),
        cache_batch_idx=None if batch_idx is None else batch_idx.to(device),
        block_table=None if table is None else table.to(device), causal=True, num_splits=splits,
        return_softmax_lse=True,
    )
    torch.cuda.synchronize()
    _log(f"{tag}: kernels done in {time.time() - t:.2f} s")
    # Append: the written positions hold k_new / v_new bit for bit, the rest is unchanged.
    n_new = k_new.shape[1]
    written = torch.zeros(k_cache.shape[:2], dtype=torch.bool, device=device)
    for bi, start in enumerate(int(x) for x in seqlens.tolist()):
        for tt in range(n_new):
            pos = start + tt
            if table is not None:
                page = k_cache.shape[1]
                row, off = int(table[bi, pos // page]), pos % page
            else:
                row, off = (int(batch_idx[bi]) if batch_idx is not None else bi), pos
            written[row, off] = True
            assert torch.equal(k_cache[row, off], k_new[bi, tt].to(device)), f"{tag}: k_new {bi},{tt} not appended"
            assert torch.equal(v_cache[row, off], v_new[bi, tt].to(device)), f"{tag}: v_new {bi},{tt} not appended"
    for name, after, before in (("k", k_cache, kc0), ("v", v_cache, vc0)):
        changed = (after != before).flatten(2).any(dim=2)
        assert not (changed & ~written).any(), f"{tag}: {name}_cache changed outside the appended positions"
    del kc0, vc0
    # Attention over the appended cache, every sequence and head.
    t = time.time()
    ends = seqlens + n_new
    ku, vu = okv.materialize(k_cache.cpu(), v_cache.cpu(), ends, batch_idx, table)
    o_ref, l_ref = okv.splitkv_attention(q, ku, vu, ends, q.shape[-1] ** -0.5, True, splits)
    assert_2x(f"{tag} out", out.cpu(), o_ref, o_ref.to(torch.float16))
    assert_lse(lse.cpu(), l_ref)
    _log(f"{tag}: oracle checked in {time.time() - t:.1f} s")


@pytest.mark.gpu
def test_c4_full_paged_decode(device):
    b, h, hk, d, page, splits = 64, 32, 8, 128, 256, 8
    g = torch.Generator().manual_seed(15)
    lens = torch.randint(1024, 32769, (b,), generator=g, dtype=torch.int32)
    nblk = [(int(x) + 1 + page - 1) // page for x in lens]
    perm = torch.randperm(sum(nblk), generator=g)
    table = torch.zeros((b, max(nblk)), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[off : off + n].to(torch.int32)
        off += n
    q = randn16((b, 1, h, d), g)
    k_new = randn16((b, 1, hk, d), g)
    v_new = randn16((b, 1, hk, d), g)
    gd = torch.Generator(device=device).manual_seed(15)
    k_cache = torch.randn((sum(nblk), page, hk, d), generator=gd, device=device, dtype=torch.float16)
    v_cache = torch.randn((sum(nblk), page, hk, d), generator=gd, device=device, dtype=torch.float16)
    _log(f"c4: paged decode, 64 sequences, {int(lens.sum()) + b} keys, {sum(nblk)} pages of 256")
    _check_kvcache("c4", device, q, k_cache, v_cache, k_new, v_new, lens, None, table, splits)


@pytest.mark.gpu
def test_c5_full_long_context(device):
    rows, cap, h, d, b, sq, splits = 8, 131072, 16, 64, 4, 4, 16
    g = torch.Generator().manual_seed(16)
    batch_idx = torch.randperm(rows, generator=g)[:b].to(torch.int32)
    lens = torch.randint(65536, 131069, (b,), generator=g, dtype=torch.int32)
    q = randn16((b, sq, h, d), g)
    k_new = randn16((b, sq, h, d), g)
    v_new = randn16((b, sq, h, d), g)
    gd = torch.Generator(device=device).manual_seed(16)
    k_cache = torch.randn((rows, cap, h, d), generator=gd, device=device, dtype=torch.float16)
    v_cache = torch.randn((rows, cap, h, d), generator=gd, device=device, dtype=torch.float16)
    _log(f"c5: contiguous 8 x 131072 cache, rows {batch_idx.tolist()}, lengths {lens.tolist()}")
    _check_kvcache("c5", device, q, k_cache, v_cache, k_new, v_new, lens, batch_idx, None, splits)
