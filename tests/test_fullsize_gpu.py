"""Parity at the BASELINE configurations' full sizes (c1-c5) and at the
north-star point (causal b4 s8192 h16 d128), on the GPU.

The kernels run on the whole workload; the fp32 oracle and the
rounding-point twin are evaluated on the CPU for the parts that finish in
seconds there:

* c1 (b2 s512 h8 d64, non-causal forward): every element;
* c2 (b4 s4096 h16 d128 causal, forward + backward), the s8192 point and its
  head_dim 64 counterpart (b4 s8192 h16 d64 causal, one 8-head half of rows 0 and 3):
  every element of batch rows 0 and 3 (rows of a batch are independent, so
  each is the full computation of that row at the full sequence length and
  head count), checked four KV heads at a time (the s8192 rows as two tests
  of eight heads each); the reference's longest published length (b4 s16000
  h16 d128 causal): two heads of rows 0 and 3;
* c3 (16 packed causal sequences, 32/8 heads): every element of the shortest,
  the median-length and the longest sequence;
* c4 (paged decode with append, 64 sequences up to 32k keys, 8 splits) and c5
  (4 remapped rows of an 8 x 131072 contiguous cache, 4 new tokens, 16 splits):
  every output and LSE, the appended K/V bit-exact, and every other cache
  position unchanged.

The inputs are the ones bench.py times: the same seeds and draw order (c2 seed 1,
s8192 seed 5, the sweep's shapes seed 7, c3 seed 2, c4 seed 3, c5 seed 4; c1,
which bench.py does not time, seed 0).

Bounds as in the small-size tests: 2x the twin's error (+ the fp32 noise
floor for the backward), LSE to 2e-5 relative, bit-exact cache writes.  The
twin's error on these exact inputs is committed in tests/golden/ref_error.json
(tests/golden/make_ref_error.py); each test checks that the twin still
reproduces it (within 5 %), so a change to the twin's rounding points cannot
silently move the bound, and that the fp32-noise widening of the backward
bound stays below a tenth of the 2x bound.
"""

import json
import os
import time

import pytest
import torch

import flash_attention_interface as fai
from helpers import (FULLSIZE, FULLSIZE_KV_CHUNK, assert_2x, assert_lse, c1_inputs, c3_checked_sequences, c3_inputs,
                     check_fwd_bwd, dense_inputs, randn16, unit_key)
from oracle import kvcache as okv

REF_ERROR = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_error.json")))
TWIN_REL_TOL = 0.05  # the twin's error on the committed inputs, recomputed on another host's BLAS
NOISE_FRAC = 0.1  # largest fp32-noise widening allowed, as a fraction of the 2x bound


def _log(msg):
    print(f"[fullsize] {msg}", flush=True)


def _check_against_fixture(key, stats):
    """The twin's error equals the committed one; the noise widening is small; log the margins."""
    fx = REF_ERROR[key]
    for n, s in stats.items():
        if n == "lse":
            continue
        want = fx["err_ref"][n]
        assert abs(s["err_ref"] - want) <= TWIN_REL_TOL * want, (
            f"{key} {n}: twin error {s['err_ref']:.4e} differs from the committed {want:.4e}"
        )
        if s["noise_max"]:
            assert s["noise_max"] <= NOISE_FRAC * s["bound"], (
                f"{key} {n}: fp32-noise widening {s['noise_max']:.3e} above {NOISE_FRAC} of the bound {s['bound']:.3e}"
            )
    _log(f"{key} margins (err / 2x bound): " + ", ".join(
        f"{n} {s['err'] / s['bound']:.2f}" for n, s in stats.items() if n != "lse"))


@pytest.mark.gpu
def test_c1_full_forward(device):
    q, k, v = c1_inputs()
    _log("c1: b2 s512 h8 d64 non-causal")
    out, lse = fai._flash_attn_forward(q.to(device), k.to(device), v.to(device), 64 ** -0.5, False)
    torch.cuda.synchronize()
    stats = check_fwd_bwd("c1", q, k, v, None, out.cpu(), lse.cpu(), None, 64 ** -0.5, False)
    _check_against_fixture("c1", stats)


_DENSE = {}


def _dense_run(device, name):
    """Forward (autograd) + backward of a full-size dense configuration on the GPU, once per module."""
    if name not in _DENSE:
        b, s, h, d, seed, causal, _ = FULLSIZE[name]
        q, k, v, do = dense_inputs(b, s, h, d, seed)
        _log(f"{name}: b{b} s{s} h{h} d{d} causal={causal} fwd + bwd on the GPU")
        qd, kd, vd = (t.to(device).requires_grad_() for t in (q, k, v))
        out = fai.flash_attn_func(qd, kd, vd, causal=causal)
        out.backward(do.to(device))
        # The same forward again for its LSE (the kernels are deterministic).
        out2, lse = fai._flash_attn_forward(qd.detach(), kd.detach(), vd.detach(), d ** -0.5, causal)
        torch.cuda.synchronize()
        assert torch.equal(out2, out.detach())
        assert all(torch.isfinite(t).all() for t in (out, qd.grad, kd.grad, vd.grad))
        _DENSE.clear()  # one configuration's tensors at a time
        _DENSE[name] = (q, k, v, do, out.detach().cpu(), lse.cpu(), qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu())
    return _DENSE[name]


def _check_dense_unit(device, name, unit):
    b, s, h, d, seed, causal, _ = FULLSIZE[name]
    q, k, v, do, out, lse, dq, dk, dv = _dense_run(device, name)
    r, hs = slice(unit[0], unit[0] + 1), slice(unit[1], unit[2])
    key = unit_key(name, unit)
    t = time.time()
    stats = check_fwd_bwd(key, q[r, :, hs], k[r, :, hs], v[r, :, hs], do[r, :, hs], out[r, :, hs], lse[r, hs],
                          (dq[r, :, hs], dk[r, :, hs], dv[r, :, hs]), d ** -0.5, causal,
                          kv_chunk=FULLSIZE_KV_CHUNK.get(name, 4), log=_log)
    _log(f"{key}: forward and backward checked in {time.time() - t:.1f} s")
    _check_against_fixture(key, stats)


@pytest.mark.gpu
@pytest.mark.parametrize("unit", FULLSIZE["c2"][6])
def test_c2_full_forward_backward(device, unit):
    _check_dense_unit(device, "c2", unit)


@pytest.mark.gpu
@pytest.mark.parametrize("unit", FULLSIZE["s8192"][6])
def test_s8192_north_star_forward_backward(device, unit):
    """The shape the north star's MFMA targets are quoted on (benchmark.sh:17-21)."""
    _check_dense_unit(device, "s8192", unit)


@pytest.mark.gpu
@pytest.mark.parametrize("unit", FULLSIZE["hd64_s8192"][6])
def test_hd64_s8192_forward_backward(device, unit):
    """benchmark.sh's head_dim 64 shape at seqlen 8192, causal (benchmark.sh:17-23): the
    head_dim 64 forms of the forward (softmax without the row maximum) and dQ (dP from -D)."""
    _check_dense_unit(device, "hd64_s8192", unit)


@pytest.mark.gpu
@pytest.mark.parametrize("unit", FULLSIZE["s16000"][6])
def test_s16000_forward_backward(device, unit):
    """The reference's longest published point (benchmark.sh:21; README.md:30 quotes its speedups at
    s = 16000 / 16384): b4 s16000 h16 d128 causal, the sweep's seed; two heads of rows 0 and 3."""
    _check_dense_unit(device, "s16000", unit)


@pytest.mark.gpu
def test_c3_full_varlen_gqa(device):
    lens, cu, q, k, v, do = c3_inputs()
    total, mx, d = int(cu[-1]), max(lens), q.shape[-1]
    _log(f"c3: 16 packed causal sequences ({total} tokens, max {mx}), 32/8 heads, fwd + bwd on the GPU")
    qd, kd, vd = (t.to(device).requires_grad_() for t in (q, k, v))
    cud = cu.to(device)
    out = fai.flash_attn_varlen_func(qd, kd, vd, cud, cud, mx, mx, causal=True)
    out.backward(do.to(device))
    out2, lse = fai._flash_attn_varlen_forward(qd.detach(), kd.detach(), vd.detach(), cud, cud, mx, mx, d ** -0.5, True)
    torch.cuda.synchronize()
    assert torch.equal(out2, out.detach())
    out, lse = out.detach().cpu(), lse.cpu()
    dq, dk, dv = qd.grad.cpu(), kd.grad.cpu(), vd.grad.cpu()
    for i in c3_checked_sequences(lens):
        a, e = int(cu[i]), int(cu[i + 1])
        stats = check_fwd_bwd(
            f"c3 seq {i} (n={e - a})", q[a:e][None], k[a:e][None], v[a:e][None], do[a:e][None], out[a:e][None],
            lse[i : i + 1, :, : e - a], (dq[a:e][None], dk[a:e][None], dv[a:e][None]), d ** -0.5, True, kv_chunk=4,
        )
        _check_against_fixture(f"c3_seq{i}", stats)


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
    """Config c4 drawn exactly as bench.py draws it (seed 3; the cache on the device generator)."""
    b, h, hk, d, page, splits = 64, 32, 8, 128, 256, 8
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(1024, 32769, (b,), generator=g)
    nblk = [(int(x) + 1 + page - 1) // page for x in lens]
    perm = torch.randperm(sum(nblk), generator=g)
    table = torch.zeros((b, max(nblk)), dtype=torch.int32)
    off = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[off : off + n].to(torch.int32)
        off += n
    gd = torch.Generator(device=device).manual_seed(3)
    k_cache = torch.randn((sum(nblk), page, hk, d), generator=gd, device=device, dtype=torch.float16)
    v_cache = torch.randn((sum(nblk), page, hk, d), generator=gd, device=device, dtype=torch.float16)
    q = randn16((b, 1, h, d), g)
    k_new = randn16((b, 1, hk, d), g)
    v_new = randn16((b, 1, hk, d), g)
    _log(f"c4: paged decode, 64 sequences, {int(lens.sum()) + b} keys, {sum(nblk)} pages of 256")
    _check_kvcache("c4", device, q, k_cache, v_cache, k_new, v_new, lens.to(torch.int32), None, table, splits)


@pytest.mark.gpu
def test_c5_full_long_context(device):
    """Config c5 drawn exactly as bench.py draws it (seed 4; the cache on the device generator)."""
    rows, cap, h, d, b, sq, splits = 8, 131072, 16, 64, 4, 4, 16
    g = torch.Generator().manual_seed(4)
    batch_idx = torch.randperm(rows, generator=g)[:b].to(torch.int32)
    lens = torch.randint(65536, 131069, (b,), generator=g)
    gd = torch.Generator(device=device).manual_seed(4)
    k_cache = torch.randn((rows, cap, h, d), generator=gd, device=device, dtype=torch.float16)
    v_cache = torch.randn((rows, cap, h, d), generator=gd, device=device, dtype=torch.float16)
    q = randn16((b, sq, h, d), g)
    k_new = randn16((b, sq, h, d), g)
    v_new = randn16((b, sq, h, d), g)
    _log(f"c5: contiguous 8 x 131072 cache, rows {batch_idx.tolist()}, lengths {lens.tolist()}")
    _check_kvcache("c5", device, q, k_cache, v_cache, k_new, v_new, lens.to(torch.int32), batch_idx, None, splits)
