"""KV-cache oracle (CPU).  Test infrastructure only.

Restates the reference's own Python math path for ``flash_attn_with_kvcache``
(flash_attention_interface.py:642-776) and the split / combine arithmetic of
csrc/flash_attn/src/kvcache_native.cu:191-193 (split bounds), :676-729
(log-sum-exp combine) and :782-871 (paged append).

Local windows and softcap, which the reference's signature takes but rejects
(flash_attention_interface.py:617-634, "the signature matches upstream
FlashAttention"), follow upstream FlashAttention's documented semantics:
query i (aligned bottom-right, at key position i + L - sq) sees keys
[i + L - sq - left, i + L - sq + right] (a negative bound is unbounded; causal
means right = 0), softcap c > 0 replaces the scaled score s * scale by
c * tanh(s * scale / c), ALiBi adds -slope_h * |i + L - sq - j| to the score
fed to the softmax (slopes [h] or [b, h]), and cache_leftpad[b] is the first
valid key of sequence b (positions unchanged).

Rotary embeddings (``rotary_embed``) restate upstream FlashAttention's
rotary form (flash_attn/layers/rotary.py, apply_rotary_emb_torch, v2.x;
the reference's signature takes rotary_cos / rotary_sin and rejects them):
with rotary_dim = 2 * cos.shape[1], channel pairs (j, j + rotary_dim / 2)
(or (2j, 2j + 1) interleaved) are rotated by the angle whose cosine and sine
are cos[p, j], sin[p, j] at the row's position p; channels past rotary_dim are
kept.  Appended key t of sequence b sits at position cache_seqlens[b] + t, and
query i at cache_seqlens[b] + i when causal or windowed, else at
cache_seqlens[b].
"""

from typing import List, Optional, Tuple

import torch

from .attention import causal_keep


def append_contiguous(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cache_seqlens: torch.Tensor,
    cache_batch_idx: Optional[torch.Tensor] = None,
) -> None:
    """In place: k/v[b, t] -> cache row ``cache_batch_idx[b]`` (or b) at
    position ``cache_seqlens[b] + t`` (flash_attention_interface.py:642-662,
    flash_api.cpp:643-654)."""
    starts = [int(x) for x in cache_seqlens.tolist()]
    rows = (
        [int(x) for x in cache_batch_idx.tolist()]
        if cache_batch_idx is not None
        else list(range(k.shape[0]))
    )
    n = k.shape[1]
    for bi, start in enumerate(starts):
        k_cache[rows[bi], start : start + n] = k[bi]
        v_cache[rows[bi], start : start + n] = v[bi]


def append_paged(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cache_seqlens: torch.Tensor,
    block_table: torch.Tensor,
) -> None:
    """In place: logical position p = cache_seqlens[b] + t goes to physical page
    block_table[b, p // page] at offset p % page
    (flash_attention_interface.py:665-685, kvcache_native.cu:825-839)."""
    page = k_cache.shape[1]
    starts = [int(x) for x in cache_seqlens.tolist()]
    table = block_table.tolist()
    for bi, start in enumerate(starts):
        for t in range(k.shape[1]):
            pos = start + t
            blk = table[bi][pos // page]
            k_cache[blk, pos % page] = k[bi, t]
            v_cache[blk, pos % page] = v[bi, t]


def rotary_embed(
    x: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: torch.Tensor,
    interleaved: bool,
    compute: torch.dtype = torch.float32,
    out_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """Rotate the first 2 * cos.shape[1] channels of x [b, s, h, d] at
    positions [b, s] (row p of cos / sin [seqlen_ro, rotary_dim / 2]).

    compute float32 on fp16 inputs: each product is exact, so every output is
    the exact rotation rounded once to fp32, then to ``out_dtype`` (x's dtype
    by default).  A position past the table takes its last row (this package's
    choice; upstream reads past the table there)."""
    rd = 2 * cos.shape[1]
    half = rd // 2
    pos = positions.long().clamp(0, cos.shape[0] - 1)
    c = cos.to(compute)[pos][:, :, None, :]  # b s 1 half
    sn = sin.to(compute)[pos][:, :, None, :]
    xr = x[..., :rd].to(compute)
    if interleaved:
        a, bb = xr[..., 0::2], xr[..., 1::2]
    else:
        a, bb = xr[..., :half], xr[..., half:]
    ra = a * c - bb * sn
    rb = a * sn + bb * c
    if interleaved:
        rot = torch.stack((ra, rb), dim=-1).flatten(-2)
    else:
        rot = torch.cat((ra, rb), dim=-1)
    out = x.to(compute).clone()
    out[..., :rd] = rot
    return out.to(out_dtype or x.dtype)


def rotary_positions(cache_seqlens: torch.Tensor, n: int, per_row: bool) -> torch.Tensor:
    """[b, n] positions: cache_seqlens[b] + i (per_row) or cache_seqlens[b]."""
    step = torch.arange(n)[None, :] if per_row else torch.zeros((1, n), dtype=torch.int64)
    return cache_seqlens.long()[:, None] + step


def materialize(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seqlens: torch.Tensor,
    cache_batch_idx: Optional[torch.Tensor],
    block_table: Optional[torch.Tensor],
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Logical per-sequence K/V [b, max_len, hk, d] read through the remap or the
    page table, zero past each length (flash_attention_interface.py:688-728)."""
    lens = [int(x) for x in seqlens.tolist()]
    max_len = max(lens) if lens else 0
    b = len(lens)
    hk, d = k_cache.shape[2], k_cache.shape[3]
    k_out = torch.zeros((b, max_len, hk, d), dtype=k_cache.dtype)
    v_out = torch.zeros_like(k_out)
    if block_table is None:
        rows = (
            [int(x) for x in cache_batch_idx.tolist()]
            if cache_batch_idx is not None
            else list(range(b))
        )
        for bi, n in enumerate(lens):
            k_out[bi, :n] = k_cache[rows[bi], :n]
            v_out[bi, :n] = v_cache[rows[bi], :n]
        return k_out, v_out
    page = k_cache.shape[1]
    table = block_table.tolist()
    for bi, n in enumerate(lens):
        pos = 0
        while pos < n:
            blk = table[bi][pos // page]
            off = pos % page
            take = min(page - off, n - pos)
            k_out[bi, pos : pos + take] = k_cache[blk, off : off + take]
            v_out[bi, pos : pos + take] = v_cache[blk, off : off + take]
            pos += take
    return k_out, v_out


def split_bounds(seqlen_k: int, num_splits: int) -> List[Tuple[int, int]]:
    """Split s of S covers [L*s // S, L*(s+1) // S) (kvcache_native.cu:191-192,
    flash_attention_interface.py:755-756)."""
    return [((seqlen_k * s) // num_splits, (seqlen_k * (s + 1)) // num_splits) for s in range(num_splits)]


def combine(out_parts: torch.Tensor, lse_parts: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Log-sum-exp combine of split partials (kvcache_native.cu:697-727).

    out_parts [S, rows, d] (already normalised per split), lse_parts [S, rows]
    with -inf for an empty split.  Returns (out [rows, d], lse [rows]) with the
    LSE of an all-empty row reported as 0 and its output 0."""
    lse_max = lse_parts.max(dim=0).values
    finite = torch.isfinite(lse_max)
    shift = torch.where(finite, lse_max, torch.zeros_like(lse_max))
    w_sum = torch.exp(lse_parts - shift[None]).sum(dim=0)
    lse_tot = torch.where(finite & (w_sum > 0), shift + torch.log(w_sum), torch.full_like(shift, float("-inf")))
    ok = torch.isfinite(lse_tot)
    w = torch.exp(lse_parts - torch.where(ok, lse_tot, torch.zeros_like(lse_tot))[None])
    w = torch.where(ok[None], w, torch.zeros_like(w))
    out = (w[..., None] * out_parts).sum(dim=0)
    return out, torch.where(ok, lse_tot, torch.zeros_like(lse_tot))


def splitkv_attention(
    q: torch.Tensor,
    k_used: torch.Tensor,
    v_used: torch.Tensor,
    seqlens: torch.Tensor,
    softmax_scale: float,
    causal: bool,
    num_splits: int,
    dtype: torch.dtype = torch.float32,
    window: Tuple[int, int] = (-1, -1),
    softcap: float = 0.0,
    alibi_slopes: Optional[torch.Tensor] = None,
    leftpad: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Split-KV attention over materialised caches, per batch row
    (flash_attention_interface.py:731-776): each split is a separate softmax
    with its own LSE (-inf when empty), then the log-sum-exp combine.

    q [b, sq, h, d]; k_used/v_used [b, >=max_len, hk, d]; causal keeps key j for
    query i iff j <= i + L - sq with L = seqlens[b] (kvcache_native.cu:347).
    ``window`` (left, right), ``softcap``, ``alibi_slopes`` and ``leftpad`` as in
    the module docstring.
    Returns (out [b, sq, h, d] in ``dtype``, lse [b, h, sq] in ``dtype``)."""
    b, sq, h, d = q.shape
    hk = k_used.shape[2]
    groups = h // hk
    out = torch.zeros((b, sq, h, d), dtype=dtype)
    lse = torch.zeros((b, h, sq), dtype=dtype)
    for bi, n in enumerate(int(x) for x in seqlens.tolist()):
        qi = q[bi].to(dtype).transpose(0, 1)  # h sq d
        ki = k_used[bi, :n].to(dtype).repeat_interleave(groups, dim=1).transpose(0, 1)
        vi = v_used[bi, :n].to(dtype).repeat_interleave(groups, dim=1).transpose(0, 1)
        splits = max(1, min(num_splits, n)) if num_splits > 0 else 1
        keep = causal_keep(sq, n) if causal else torch.ones((sq, n), dtype=torch.bool)
        left, right = window
        if left >= 0 or right >= 0:
            pos = torch.arange(sq)[:, None] + n - sq  # the query's own key position
            j = torch.arange(n)[None, :]
            if left >= 0:
                keep = keep & (j >= pos - left)
            if right >= 0:
                keep = keep & (j <= pos + right)
        if leftpad is not None:
            keep = keep & (torch.arange(n)[None, :] >= int(leftpad[bi]))
        bias = None
        if alibi_slopes is not None:
            sl = alibi_slopes[bi] if alibi_slopes.dim() == 2 else alibi_slopes
            pos = torch.arange(sq)[:, None] + n - sq
            dist = (pos - torch.arange(n)[None, :]).abs().to(dtype)
            bias = -sl.to(dtype)[:, None, None] * dist[None]  # h sq n
        parts_o, parts_l = [], []
        for s0, s1 in split_bounds(n, splits):
            sc = torch.matmul(qi, ki[:, s0:s1].transpose(-1, -2).contiguous()) * softmax_scale
            if softcap > 0:
                sc = softcap * torch.tanh(sc / softcap)
            if bias is not None:
                sc = sc + bias[:, :, s0:s1]
            sc = sc.masked_fill(~keep[:, s0:s1], float("-inf"))
            any_row = torch.isfinite(sc).any(dim=-1, keepdim=True) if s1 > s0 else torch.zeros(
                (h, sq, 1), dtype=torch.bool
            )
            if s1 > s0:
                m = torch.where(any_row, sc.amax(dim=-1, keepdim=True), torch.zeros_like(sc[..., :1]))
                p = torch.exp(sc - m)
                l = p.sum(dim=-1, keepdim=True)
                safe = torch.where(l > 0, l, torch.ones_like(l))
                o = torch.where(any_row, torch.matmul(p / safe, vi[:, s0:s1]), torch.zeros((h, sq, d), dtype=dtype))
                lp = torch.where(any_row, m + torch.log(safe), torch.full_like(m, float("-inf"))).squeeze(-1)
            else:
                o = torch.zeros((h, sq, d), dtype=dtype)
                lp = torch.full((h, sq), float("-inf"), dtype=dtype)
            parts_o.append(o.reshape(h * sq, d))
            parts_l.append(lp.reshape(h * sq))
        o_tot, l_tot = combine(torch.stack(parts_o), torch.stack(parts_l))
        out[bi] = o_tot.reshape(h, sq, d).transpose(0, 1)
        lse[bi] = l_tot.reshape(h, sq)
    return out, lse
