"""Pins the CPU oracle before it is trusted as the parity reference.

The reference ships no golden vectors for this path (its tests compare against
runtime SDPA on unseeded inputs), so every oracle function is checked against
something independent of its own formula:
  * closed forms: sq = sk = 1, constant keys (uniform softmax), a dominant key,
    fully masked rows, the bottom-right causal alignment with sq != sk;
  * float64 brute force written as plain loops over the definitions;
  * torch.autograd of an independently written expression, and central finite
    differences, for the backward;
  * exact invariants for the cache functions (slice writes, page-table
    round trips, split-KV == unsplit, a hand-computed combine).
"""

import math

import pytest
import torch

from oracle import kvcache as okv
from oracle import twin
from oracle.attention import attention_bwd, attention_fwd, bwd_fp32_noise, causal_keep, varlen_bwd, varlen_fwd

D64 = torch.float64


def _rand(shape, seed, dtype=D64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def _brute_fwd(q, k, v, scale, causal):
    """Plain loops over the definition of softmax attention (bottom-right causal)."""
    b, sq, h, d = q.shape
    sk, hk = k.shape[1], k.shape[2]
    grp = h // hk
    out = torch.zeros(b, sq, h, d, dtype=D64)
    lse = torch.zeros(b, h, sq, dtype=D64)
    for bi in range(b):
        for hi in range(h):
            kh = hi // grp
            for i in range(sq):
                logits = []
                for j in range(sk):
                    if causal and j > i + sk - sq:
                        continue
                    dot = sum(float(q[bi, i, hi, t]) * float(k[bi, j, kh, t]) for t in range(d))
                    logits.append((j, dot * scale))
                if not logits:
                    continue
                m = max(x for _, x in logits)
                z = sum(math.exp(x - m) for _, x in logits)
                lse[bi, hi, i] = m + math.log(z)
                for j, x in logits:
                    out[bi, i, hi] += math.exp(x - m) / z * v[bi, j, kh].double()
    return out, lse


def test_fwd_single_token_closed_form():
    q, k, v = _rand((1, 1, 2, 8), 1), _rand((1, 1, 2, 8), 2), _rand((1, 1, 2, 8), 3)
    out, lse = attention_fwd(q, k, v, 0.37, False, dtype=D64)
    assert torch.allclose(out, v, atol=1e-14)
    assert torch.allclose(lse[0, :, 0], 0.37 * (q[0, 0] * k[0, 0]).sum(-1), atol=1e-14)


def test_fwd_constant_keys_give_prefix_means_bottom_right():
    # Identical keys -> uniform weights over the visible keys.  sq=2, sk=3 causal:
    # row 0 sees keys 0..1, row 1 sees keys 0..2 (bottom-right, mask.h:52).
    q = _rand((1, 2, 1, 4), 4)
    k = _rand((1, 1, 1, 4), 5).expand(1, 3, 1, 4).contiguous()
    v = _rand((1, 3, 1, 4), 6)
    out, _ = attention_fwd(q, k, v, 1.0, True, dtype=D64)
    assert torch.allclose(out[0, 0, 0], v[0, :2, 0].mean(0), atol=1e-14)
    assert torch.allclose(out[0, 1, 0], v[0, :3, 0].mean(0), atol=1e-14)
    out_nc, _ = attention_fwd(q, k, v, 1.0, False, dtype=D64)
    assert torch.allclose(out_nc[0, 0, 0], v[0, :, 0].mean(0), atol=1e-14)


def test_fwd_dominant_key():
    q = torch.zeros(1, 1, 1, 4, dtype=D64)
    q[..., 0] = 1.0
    k = torch.zeros(1, 5, 1, 4, dtype=D64)
    k[0, 3, 0, 0] = 80.0
    v = _rand((1, 5, 1, 4), 7)
    out, lse = attention_fwd(q, k, v, 1.0, False, dtype=D64)
    assert torch.allclose(out[0, 0, 0], v[0, 3, 0], atol=1e-12)
    assert abs(lse.item() - 80.0) < 1e-12


def test_fwd_fully_masked_rows_are_zero():
    q, k, v = _rand((1, 5, 2, 4), 8), _rand((1, 2, 1, 4), 9), _rand((1, 2, 1, 4), 10)
    out, lse = attention_fwd(q, k, v, 0.5, True, dtype=D64)
    assert torch.all(out[0, :3] == 0) and torch.all(lse[0, :, :3] == 0)
    assert torch.all(out[0, 3:] != 0)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(3, 4), (4, 3), (1, 5), (5, 5)])
def test_fwd_matches_brute_force(causal, sq, sk):
    q, k, v = _rand((2, sq, 4, 6), 11), _rand((2, sk, 2, 6), 12), _rand((2, sk, 2, 6), 13)
    out, lse = attention_fwd(q, k, v, 0.41, causal, dtype=D64)
    bo, bl = _brute_fwd(q, k, v, 0.41, causal)
    assert torch.allclose(out, bo, atol=1e-12)
    assert torch.allclose(lse, bl, atol=1e-12)


def _autograd_ref(q, k, v, do, scale, causal):
    """An independent expression (softmax + matmul, repeat for GQA) differentiated by autograd."""
    q, k, v = (t.clone().requires_grad_() for t in (q, k, v))
    grp = q.shape[2] // k.shape[2]
    kk = k.repeat_interleave(grp, dim=2)
    vv = v.repeat_interleave(grp, dim=2)
    s = torch.einsum("bihd,bjhd->bhij", q, kk) * scale
    if causal:
        s = s.masked_fill(~causal_keep(q.shape[1], k.shape[1]), float("-inf"))
    p = torch.softmax(s, dim=-1).nan_to_num(0.0)
    o = torch.einsum("bhij,bjhd->bihd", p, vv)
    o.backward(do)
    return q.grad, k.grad, v.grad


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk,h,hk", [(5, 7, 2, 1), (7, 5, 4, 2), (6, 6, 3, 3)])
def test_bwd_matches_autograd(causal, sq, sk, h, hk):
    q, k, v = _rand((2, sq, h, 8), 14), _rand((2, sk, hk, 8), 15), _rand((2, sk, hk, 8), 16)
    do = _rand((2, sq, h, 8), 17)
    out, lse = attention_fwd(q, k, v, 0.3, causal, dtype=D64)
    dq, dk, dv = attention_bwd(q, k, v, out, lse, do, 0.3, causal, dtype=D64)
    rq, rk, rv = _autograd_ref(q, k, v, do, 0.3, causal)
    assert torch.allclose(dq, rq, atol=1e-12)
    assert torch.allclose(dk, rk, atol=1e-12)
    assert torch.allclose(dv, rv, atol=1e-12)


def test_bwd_finite_differences():
    q, k, v = _rand((1, 4, 2, 4), 18), _rand((1, 6, 1, 4), 19), _rand((1, 6, 1, 4), 20)
    do = _rand((1, 4, 2, 4), 21)
    out, lse = attention_fwd(q, k, v, 0.7, True, dtype=D64)
    grads = attention_bwd(q, k, v, out, lse, do, 0.7, True, dtype=D64)

    def loss(qq, kk, vv):
        return (attention_fwd(qq, kk, vv, 0.7, True, dtype=D64)[0] * do).sum().item()

    eps = 1e-6
    for gi, t in enumerate((q, k, v)):
        for idx in [(0, 1, 0, 2), (0, 3, 0, 0), (0, 2, 0, 3)]:
            if idx[2] >= t.shape[2]:
                continue
            tp, tm = t.clone(), t.clone()
            tp[idx] += eps
            tm[idx] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[gi], args_m[gi] = tp, tm
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(fd - grads[gi][idx].item()) < 1e-7


@pytest.mark.parametrize("sq,sk,h,hk,causal", [(37, 1, 6, 1, False), (50, 40, 4, 2, True)])
def test_bwd_noise_floor_covers_fp32_and_stays_small(sq, sk, h, hk, causal):
    """The fp32 noise scale covers what fp32 arithmetic in another summation
    order does (here: the fp32 closed form vs float64), including the single
    key case where dP == D and dK is pure rounding noise, and stays far below
    the gradients' own size, so a dropped term or wrong index cannot hide in it."""
    g = torch.Generator().manual_seed(23)
    q, k, v, do = (torch.randn(s, generator=g).half() for s in ((2, sq, h, 128), (2, sk, hk, 128), (2, sk, hk, 128), (2, sq, h, 128)))
    o64, l64 = attention_fwd(q, k, v, 0.3, causal, dtype=D64)
    g64 = attention_bwd(q, k, v, o64, l64, do, 0.3, causal, dtype=D64)
    g32 = attention_bwd(q, k, v, o64.float(), l64.float(), do, 0.3, causal)
    noise = bwd_fp32_noise(q, k, v, o64, l64, do, 0.3, causal)
    for a, b, n in zip(g32, g64, noise):
        assert torch.all((a.double() - b).abs() <= n.double())
    if sk > 1:
        for b, n in zip(g64, noise):
            assert n.max().item() < 1e-3 * b.abs().max().item()


def test_varlen_equals_dense_per_sequence():
    lens = [3, 5, 1]
    cu = torch.tensor([0, 3, 8, 9], dtype=torch.int32)
    q, k, v = _rand((9, 2, 4), 22), _rand((9, 1, 4), 23), _rand((9, 1, 4), 24)
    do = _rand((9, 2, 4), 25)
    out, lse = varlen_fwd(q, k, v, cu, cu, 5, 0.5, True, dtype=D64)
    assert lse.shape == (3, 2, 5)
    assert torch.all(lse[0, :, 3:] == 0) and torch.all(lse[2, :, 1:] == 0)
    grads = varlen_bwd(q, k, v, out, lse, do, cu, cu, 0.5, True, dtype=D64)
    for bi, (a, n) in enumerate(zip([0, 3, 8], lens)):
        bo, bl = _brute_fwd(q[a : a + n][None], k[a : a + n][None], v[a : a + n][None], 0.5, True)
        assert torch.allclose(out[a : a + n], bo[0], atol=1e-12)
        assert torch.allclose(lse[bi, :, :n], bl[0], atol=1e-12)
        rq, rk, rv = _autograd_ref(q[a : a + n][None], k[a : a + n][None], v[a : a + n][None], do[a : a + n][None], 0.5, True)
        assert torch.allclose(grads[0][a : a + n], rq[0], atol=1e-12)
        assert torch.allclose(grads[1][a : a + n], rk[0], atol=1e-12)


# --------------------------------------------------------------------------- kv cache


def test_append_contiguous_and_remap_are_slice_writes():
    kc = torch.zeros(4, 10, 2, 8, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    k = _rand((2, 3, 2, 8), 26, torch.float16)
    v = _rand((2, 3, 2, 8), 27, torch.float16)
    okv.append_contiguous(kc, vc, k, v, torch.tensor([2, 7], dtype=torch.int32), torch.tensor([3, 0], dtype=torch.int32))
    assert torch.equal(kc[3, 2:5], k[0]) and torch.equal(kc[0, 7:10], k[1]) and torch.equal(vc[0, 7:10], v[1])
    assert kc[1].abs().sum() == 0 and kc[2].abs().sum() == 0 and kc[3, :2].abs().sum() == 0


def test_append_paged_roundtrip_equals_contiguous():
    g = torch.Generator().manual_seed(28)
    b, cap, page = 3, 768, 256
    kc = _rand((b, cap, 1, 8), 29, torch.float16)
    vc = _rand((b, cap, 1, 8), 30, torch.float16)
    lens = torch.tensor([0, 255, 700], dtype=torch.int32)
    k = _rand((b, 4, 1, 8), 31, torch.float16)
    v = _rand((b, 4, 1, 8), 32, torch.float16)
    perm = torch.randperm(b * 3, generator=g)
    table = perm.reshape(b, 3).to(torch.int32)
    kp = torch.zeros(b * 3, page, 1, 8, dtype=torch.float16)
    vp = torch.zeros_like(kp)
    for bi in range(b):
        for j in range(3):
            kp[table[bi, j]] = kc[bi, j * page : (j + 1) * page]
            vp[table[bi, j]] = vc[bi, j * page : (j + 1) * page]
    okv.append_contiguous(kc, vc, k, v, lens, None)
    okv.append_paged(kp, vp, k, v, lens, table)
    a = okv.materialize(kc, vc, lens + 4, None, None)
    bmat = okv.materialize(kp, vp, lens + 4, None, table)
    assert torch.equal(a[0], bmat[0]) and torch.equal(a[1], bmat[1])
    # position 255 + t crosses the page boundary 255 | 256
    assert torch.equal(bmat[0][1, 255:259], k[1])


def test_split_bounds_partition():
    for L in [0, 1, 7, 1000, 4097]:
        for S in [1, 3, 8, 16]:
            bnd = okv.split_bounds(L, S)
            assert bnd[0][0] == 0 and bnd[-1][1] == L
            assert all(bnd[i][1] == bnd[i + 1][0] for i in range(S - 1))


def test_combine_known_answer():
    # Two splits with lse a, b: weights e^a / (e^a + e^b), e^b / (e^a + e^b).
    out_parts = torch.tensor([[[1.0, 0.0]], [[0.0, 3.0]]], dtype=D64)
    lse_parts = torch.tensor([[math.log(1.0)], [math.log(3.0)]], dtype=D64)
    out, lse = okv.combine(out_parts, lse_parts)
    assert torch.allclose(out[0], torch.tensor([0.25, 2.25], dtype=D64), atol=1e-15)
    assert abs(lse.item() - math.log(4.0)) < 1e-15
    # an empty split (-inf) has weight 0; an all-empty row reports 0 / 0
    out, lse = okv.combine(torch.ones(2, 2, 2, dtype=D64), torch.tensor([[0.0, -math.inf], [-math.inf, -math.inf]], dtype=D64))
    assert torch.allclose(out[0], torch.ones(2, dtype=D64)) and torch.all(out[1] == 0) and lse[1] == 0


@pytest.mark.parametrize("causal", [False, True])
def test_splitkv_equals_unsplit_and_dense(causal):
    q = _rand((3, 2, 4, 8), 33)
    ku, vu = _rand((3, 40, 2, 8), 34), _rand((3, 40, 2, 8), 35)
    lens = torch.tensor([40, 1, 23], dtype=torch.int32)
    o1, l1 = okv.splitkv_attention(q, ku, vu, lens, 0.3, causal, 1, dtype=D64)
    for S in (2, 5, 16, 64):
        oS, lS = okv.splitkv_attention(q, ku, vu, lens, 0.3, causal, S, dtype=D64)
        assert torch.allclose(oS, o1, atol=1e-12) and torch.allclose(lS, l1, atol=1e-12)
    for bi, n in enumerate(lens.tolist()):
        bo, bl = _brute_fwd(q[bi : bi + 1], ku[bi : bi + 1, :n], vu[bi : bi + 1, :n], 0.3, causal)
        assert torch.allclose(o1[bi], bo[0], atol=1e-12) and torch.allclose(l1[bi], bl[0], atol=1e-12)


def test_splitkv_window_closed_forms():
    # Window (0, 0): each query sees exactly the key at its own aligned
    # position i + L - sq, so O is that key's V and LSE its scaled score.
    q = _rand((2, 3, 2, 8), 40)
    ku, vu = _rand((2, 20, 2, 8), 41), _rand((2, 20, 2, 8), 42)
    lens = torch.tensor([20, 7], dtype=torch.int32)
    o, l = okv.splitkv_attention(q, ku, vu, lens, 0.4, False, 3, dtype=D64, window=(0, 0))
    for bi, n in enumerate(lens.tolist()):
        for i in range(3):
            j = i + n - 3
            assert torch.allclose(o[bi, i], vu[bi, j], atol=1e-12)
            sc = (q[bi, i] * ku[bi, j]).sum(-1) * 0.4
            assert torch.allclose(l[bi, :, i], sc, atol=1e-12)
    # A left window of w with causal on equals plain attention over the last
    # w + 1 keys (one query): the window is a slice of the cache.
    q1 = _rand((2, 1, 2, 8), 43)
    for w in (0, 3, 19, 100):
        ow, lw = okv.splitkv_attention(q1, ku, vu, lens, 0.4, True, 2, dtype=D64, window=(w, -1))
        for bi, n in enumerate(lens.tolist()):
            lo = max(0, n - 1 - w)
            kk, vv = ku[bi : bi + 1, lo:n], vu[bi : bi + 1, lo:n]
            bo, bl = _brute_fwd(q1[bi : bi + 1], kk, vv, 0.4, True)
            assert torch.allclose(ow[bi], bo[0], atol=1e-12) and torch.allclose(lw[bi], bl[0], atol=1e-12)
    # A right bound of 0 is causal; wide windows change nothing.
    oc, lc = okv.splitkv_attention(q, ku, vu, lens, 0.4, True, 2, dtype=D64)
    or_, lr = okv.splitkv_attention(q, ku, vu, lens, 0.4, False, 2, dtype=D64, window=(-1, 0))
    ow_, lw_ = okv.splitkv_attention(q, ku, vu, lens, 0.4, True, 2, dtype=D64, window=(50, 50))
    assert torch.allclose(oc, or_, atol=1e-12) and torch.allclose(lc, lr, atol=1e-12)
    assert torch.allclose(oc, ow_, atol=1e-12) and torch.allclose(lc, lw_, atol=1e-12)


def test_splitkv_softcap_known_answers():
    # One key: O = V whatever the cap; LSE = c * tanh(s * scale / c).
    q = torch.tensor([[[[1.0, 2.0]]]], dtype=D64)
    k = torch.tensor([[[[3.0, -0.5]], [[0.0, 0.0]]]], dtype=D64)
    v = torch.tensor([[[[1.0, 5.0]], [[-2.0, 4.0]]]], dtype=D64)
    o, l = okv.splitkv_attention(q, k, v, torch.tensor([1], dtype=torch.int32), 0.5, False, 1, dtype=D64, softcap=0.7)
    assert torch.allclose(o[0, 0, 0], v[0, 0, 0]) and abs(l.item() - 0.7 * math.tanh(2.0 * 0.5 / 0.7)) < 1e-15
    # Two keys with scores 2 and 0: weights exp(c tanh(2 * .5 / c)) : exp(0).
    o, l = okv.splitkv_attention(q, k, v, torch.tensor([2], dtype=torch.int32), 0.5, False, 2, dtype=D64, softcap=0.7)
    a = math.exp(0.7 * math.tanh(1.0 / 0.7))
    assert torch.allclose(o[0, 0, 0], torch.tensor([(a * 1.0 - 2.0) / (a + 1), (a * 5.0 + 4.0) / (a + 1)], dtype=D64))
    assert abs(l.item() - math.log(a + 1.0)) < 1e-14
    # A huge cap is no cap.
    qq, kk, vv = _rand((2, 3, 4, 8), 44), _rand((2, 30, 2, 8), 45), _rand((2, 30, 2, 8), 46)
    lens = torch.tensor([30, 11], dtype=torch.int32)
    o1, l1 = okv.splitkv_attention(qq, kk, vv, lens, 0.3, True, 3, dtype=D64)
    o2, l2 = okv.splitkv_attention(qq, kk, vv, lens, 0.3, True, 3, dtype=D64, softcap=1e7)
    assert torch.allclose(o1, o2, atol=1e-9) and torch.allclose(l1, l2, atol=1e-9)


def test_splitkv_alibi_and_leftpad_known_answers():
    # ALiBi with all scores 0 (q = 0), causal, one query at position L - 1:
    # weights exp(-slope * (L - 1 - j)), a geometric sequence.
    L, slope = 5, 0.7
    q = torch.zeros((1, 1, 2, 4), dtype=D64)
    k = _rand((1, L, 1, 4), 47)
    v = _rand((1, L, 1, 4), 48)
    slopes = torch.tensor([slope, 0.0], dtype=D64)
    o, l = okv.splitkv_attention(q, k, v, torch.tensor([L], dtype=torch.int32), 0.5, True, 2, dtype=D64,
                                 alibi_slopes=slopes)
    w = torch.tensor([math.exp(-slope * (L - 1 - j)) for j in range(L)], dtype=D64)
    assert torch.allclose(o[0, 0, 0], (w[:, None] * v[0, :, 0]).sum(0) / w.sum(), atol=1e-13)
    assert abs(l[0, 0, 0].item() - math.log(w.sum().item())) < 1e-13
    assert torch.allclose(o[0, 0, 1], v[0, :, 0].mean(0), atol=1e-13)  # slope 0: plain mean
    # Per-batch slopes [b, h] equal the per-head form row by row; non-causal
    # bias is symmetric in |i + L - sq - j|.
    qq, kk, vv = _rand((2, 3, 4, 8), 49), _rand((2, 12, 2, 8), 50), _rand((2, 12, 2, 8), 51)
    lens = torch.tensor([12, 6], dtype=torch.int32)
    sl2 = torch.rand((2, 4), generator=torch.Generator().manual_seed(52), dtype=D64)
    ob, lb = okv.splitkv_attention(qq, kk, vv, lens, 0.3, False, 3, dtype=D64, alibi_slopes=sl2)
    for bi in range(2):
        oh, lh = okv.splitkv_attention(qq[bi : bi + 1], kk[bi : bi + 1], vv[bi : bi + 1], lens[bi : bi + 1], 0.3,
                                       False, 1, dtype=D64, alibi_slopes=sl2[bi])
        assert torch.allclose(ob[bi], oh[0], atol=1e-12) and torch.allclose(lb[bi], lh[0], atol=1e-12)
    # cache_leftpad: keys before leftpad[b] do not exist; positions stay, so a
    # causal query sees the slice [leftpad, i + L - sq].
    lp = torch.tensor([4, 0], dtype=torch.int32)
    o1, l1 = okv.splitkv_attention(qq, kk, vv, lens, 0.3, True, 2, dtype=D64, leftpad=lp)
    for bi, n in enumerate(lens.tolist()):
        a = int(lp[bi])
        bo, bl = _brute_fwd(qq[bi : bi + 1], kk[bi : bi + 1, a:n], vv[bi : bi + 1, a:n], 0.3, True)
        assert torch.allclose(o1[bi], bo[0], atol=1e-12) and torch.allclose(l1[bi], bl[0], atol=1e-12)


def _rope_tables(seqlen, rd, dtype=D64, base=10000.0):
    # cos / sin of the angles p * base^(-2j / rd), the usual rotary schedule.
    inv = base ** (-torch.arange(0, rd, 2, dtype=D64) / rd)
    ang = torch.arange(seqlen, dtype=D64)[:, None] * inv[None, :]
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


@pytest.mark.parametrize("interleaved", [False, True])
def test_rotary_special_angles_and_tail(interleaved):
    x = _rand((2, 3, 2, 64), 60, torch.float16)
    rd, half = 32, 16
    pos = torch.zeros((2, 3), dtype=torch.long)
    one, zero = torch.ones((1, half), dtype=torch.float16), torch.zeros((1, half), dtype=torch.float16)
    # Angle 0: identity, bit for bit.
    assert torch.equal(okv.rotary_embed(x, one, zero, pos, interleaved), x)
    # Quarter turn (cos 0, sin 1): (a, b) -> (-b, a) exactly; the tail is kept.
    y = okv.rotary_embed(x, zero, one, pos, interleaved)
    if interleaved:
        assert torch.equal(y[..., 0:rd:2], -x[..., 1:rd:2]) and torch.equal(y[..., 1:rd:2], x[..., 0:rd:2])
    else:
        assert torch.equal(y[..., :half], -x[..., half:rd]) and torch.equal(y[..., half:rd], x[..., :half])
    assert torch.equal(y[..., rd:], x[..., rd:])


def test_rotary_hand_computed_and_interleaving_is_a_channel_permutation():
    x = torch.tensor([1.0, 2.0, 3.0, 4.0], dtype=D64).reshape(1, 1, 1, 4)
    c = torch.tensor([[0.6, 0.0]], dtype=D64)
    s = torch.tensor([[0.8, 1.0]], dtype=D64)
    pos = torch.zeros((1, 1), dtype=torch.long)
    y = okv.rotary_embed(x, c, s, pos, False, compute=D64).flatten().tolist()
    assert y == pytest.approx([1 * 0.6 - 3 * 0.8, 2 * 0.0 - 4 * 1.0, 1 * 0.8 + 3 * 0.6, 2 * 1.0 + 4 * 0.0], abs=1e-15)
    y = okv.rotary_embed(x, c, s, pos, True, compute=D64).flatten().tolist()
    assert y == pytest.approx([1 * 0.6 - 2 * 0.8, 1 * 0.8 + 2 * 0.6, 3 * 0.0 - 4 * 1.0, 3 * 1.0 + 4 * 0.0], abs=1e-15)
    # The interleaved form is the half-split form on channels reordered
    # (0, 2, 4, ..., 1, 3, 5, ...), bit for bit at fp16.
    xx = _rand((2, 5, 3, 64), 61, torch.float16)
    cos, sin = _rope_tables(40, 48, torch.float16)
    pos = torch.randint(0, 40, (2, 5), generator=torch.Generator().manual_seed(62))
    perm = torch.cat((torch.arange(0, 48, 2), torch.arange(1, 48, 2), torch.arange(48, 64)))
    inv = torch.argsort(perm)
    a = okv.rotary_embed(xx, cos, sin, pos, True)
    b = okv.rotary_embed(xx[..., perm], cos, sin, pos, False)[..., inv]
    assert torch.equal(a, b)


@pytest.mark.parametrize("interleaved", [False, True])
def test_rotary_scores_depend_on_relative_position_only(interleaved):
    # The defining property of rotary embeddings: <R(p) q, R(p') k> depends on
    # p - p' only, and each rotated pair keeps its length.  A wrong pairing,
    # sign or position index breaks it.
    cos, sin = _rope_tables(64, 32)
    q, k = _rand((1, 1, 1, 48), 63), _rand((1, 1, 1, 48), 64)

    def score(p, pk):
        qq = okv.rotary_embed(q, cos, sin, torch.tensor([[p]]), interleaved, compute=D64)
        kk = okv.rotary_embed(k, cos, sin, torch.tensor([[pk]]), interleaved, compute=D64)
        return float((qq * kk).sum())

    for p, pk in ((7, 3), (20, 20), (5, 30)):
        assert score(p, pk) == pytest.approx(score(p + 17, pk + 17), abs=1e-12)
        assert score(p, pk) == pytest.approx(score(p + 33, pk + 33), abs=1e-12)
    assert abs(score(7, 3) - score(8, 3)) > 1e-3  # it does depend on the offset
    r = okv.rotary_embed(q, cos, sin, torch.tensor([[11]]), interleaved, compute=D64)
    assert float((r * r).sum()) == pytest.approx(float((q * q).sum()), abs=1e-12)


def test_rotary_positions():
    seq = torch.tensor([5, 0, 9], dtype=torch.int32)
    assert okv.rotary_positions(seq, 3, True).tolist() == [[5, 6, 7], [0, 1, 2], [9, 10, 11]]
    assert okv.rotary_positions(seq, 2, False).tolist() == [[5, 5], [0, 0], [9, 9]]
    # Past the table: the last row.
    cos, sin = _rope_tables(8, 16, torch.float16)
    x = _rand((1, 2, 1, 16), 65, torch.float16)
    far = okv.rotary_embed(x, cos, sin, torch.tensor([[7, 30]]), False)
    last = okv.rotary_embed(x, cos, sin, torch.tensor([[7, 7]]), False)
    assert torch.equal(far, last)


# --------------------------------------------------------------------------- twin


def test_twin_rounds_where_the_reference_rounds():
    q, k, v = (_rand((1, 1, 1, 64), s, torch.float16) for s in (36, 37, 38))
    out, lse = twin.fwd_twin(q, k, v, 0.125, False)
    assert torch.equal(out, v)  # P = 1 exactly, O = V
    q, k, v = (_rand((2, 300, 4, 128), s, torch.float16) for s in (39, 40, 41))
    o_tw, l_tw = twin.fwd_twin(q, k, v, 128 ** -0.5, True)
    o_ref, l_ref = attention_fwd(q, k, v, 128 ** -0.5, True)
    err = (o_tw.float() - o_ref).abs().max().item()
    assert 1e-5 < err < 5e-3  # rounding points present, but small
    assert (l_tw - l_ref).abs().max().item() < 1e-4
    do = _rand((2, 300, 4, 128), 42, torch.float16)
    g_tw = twin.bwd_twin(q, k, v, o_tw, l_tw, do, 128 ** -0.5, True)
    g_ref = attention_bwd(q, k, v, o_ref, l_ref, do, 128 ** -0.5, True)
    for a, b in zip(g_tw, g_ref):
        e = (a.float() - b).abs().max().item()
        assert 1e-5 < e < 2e-2


def test_twin_error_matches_committed_fixture():
    """The twin's error on the small committed cases equals tests/golden/ref_error.json:
    a change to the twin's rounding points (an extra or a missing fp16 rounding)
    moves these errors and fails here before it can move any GPU bound."""
    import json
    import os
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, os.path.join(here, "golden"))
    import make_ref_error as mre

    fx = json.load(open(os.path.join(here, "golden", "ref_error.json")))
    for key in mre.SMALL:
        err, noise = mre.small_case(key)
        for n, e in err.items():
            want = fx[key]["err_ref"][n]
            assert abs(e - want) <= 0.05 * want, f"{key} {n}: twin error {e:.4e} vs committed {want:.4e}"
        for n, z in noise.items():
            want = fx[key]["noise_max"][n]
            assert abs(z - want) <= 0.05 * want, f"{key} {n}: noise scale {z:.4e} vs committed {want:.4e}"
