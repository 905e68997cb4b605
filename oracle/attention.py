"""Math attention oracle (CPU, float32 or float64).  Test infrastructure only.

Conventions restated from the reference:

* layout q [b, sq, h, d], k/v [b, sk, hk, d]  (flash_attention_interface.py:457-462)
* GQA: q-head i reads kv-head i // (h // hk)  (flash_fwd_kernel.h:76 ``bidh / h_h_k_ratio``)
* scale applied to the fp32 scores after QK^T (flash_fwd_kernel.h:314-316)
* causal is bottom-right aligned: key j kept for query i iff j <= i + sk - sq
  (mask.h:52, 88; test_flash_attn.py:305-311)
* a row with no kept key gives O = 0 and LSE = 0 (flash_fwd_kernel.h:616-629, 645-661)
* LSE layout [b, h, sq]; varlen LSE [b, h, max_seqlen_q] indexed by the local
  row, entries past a sequence's length are 0 (flash_api.cpp:388, fwd_kernel.h:97-102)
* backward: D = rowsum(O * dO) in fp32 (flash_bwd_preprocess_kernel.h:81-84),
  P = exp(scale*S - LSE), dS = P * (dP - D), dV = P^T dO, dQ = scale * dS K,
  dK = scale * dS^T Q (flash_bwd_kernel.h:417-436, 585-588, 1066-1143, 1317-1319);
  GQA dK/dV are the sums over the q-heads of a group (flash_api.cpp:338-348).
"""

from typing import Optional, Tuple

import torch


def causal_keep(sq: int, sk: int, device=None) -> torch.Tensor:
    """Bool [sq, sk]: True where key j is visible to query i (mask.h:52, 88)."""
    i = torch.arange(sq, device=device)[:, None]
    j = torch.arange(sk, device=device)[None, :]
    return j <= i + (sk - sq)


def _expand_kv(x: torch.Tensor, groups: int) -> torch.Tensor:
    # [b, sk, hk, d] -> [b, sk, h, d]; q-head i uses kv-head i // groups.
    return x.repeat_interleave(groups, dim=2) if groups > 1 else x


def attention_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    softmax_scale: float,
    causal: bool,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dense forward.  Returns (out [b, sq, h, d] in ``dtype``, lse [b, h, sq] in ``dtype``).

    Restates the math of flash_fwd_kernel.h:23-664 (online softmax gives the
    same O and LSE as the closed form) with the zero-row convention.
    """
    b, sq, h, d = q.shape
    sk, hk = k.shape[1], k.shape[2]
    groups = h // hk
    qf = q.to(dtype).permute(0, 2, 1, 3)  # b h sq d
    kf = _expand_kv(k.to(dtype), groups).permute(0, 2, 1, 3)
    vf = _expand_kv(v.to(dtype), groups).permute(0, 2, 1, 3)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * softmax_scale  # b h sq sk
    if causal:
        keep = causal_keep(sq, sk, device=s.device)
        s = s.masked_fill(~keep, float("-inf"))
    row_any = torch.isfinite(s).any(dim=-1, keepdim=True) if sk > 0 else torch.zeros(
        (b, h, sq, 1), dtype=torch.bool
    )
    if sk == 0:
        out = torch.zeros((b, h, sq, d), dtype=dtype)
        lse = torch.zeros((b, h, sq), dtype=dtype)
    else:
        m = torch.where(row_any, s.amax(dim=-1, keepdim=True), torch.zeros_like(s[..., :1]))
        p = torch.exp(s - m)
        l = p.sum(dim=-1, keepdim=True)
        safe_l = torch.where(l > 0, l, torch.ones_like(l))
        out = torch.matmul(p / safe_l, vf)
        out = torch.where(row_any, out, torch.zeros_like(out))
        lse = torch.where(row_any, m + torch.log(safe_l), torch.zeros_like(m)).squeeze(-1)
    return out.permute(0, 2, 1, 3).contiguous(), lse.contiguous()


def attention_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    softmax_scale: float,
    causal: bool,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Closed-form dense backward from the saved (out, lse).

    Follows flash_bwd_preprocess_kernel.h:74-94 (D), flash_bwd_kernel.h:401-459
    (dQ) and :1040-1143 (dK, dV), and flash_api.cpp:338-348 for the GQA sum.
    Returns (dq, dk, dv) in ``dtype``.
    """
    b, sq, h, d = q.shape
    sk, hk = k.shape[1], k.shape[2]
    groups = h // hk
    qf = q.to(dtype).permute(0, 2, 1, 3)
    kf = _expand_kv(k.to(dtype), groups).permute(0, 2, 1, 3)
    vf = _expand_kv(v.to(dtype), groups).permute(0, 2, 1, 3)
    of = out.to(dtype).permute(0, 2, 1, 3)
    dof = dout.to(dtype).permute(0, 2, 1, 3)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * softmax_scale
    p = torch.exp(s - lse.to(dtype)[..., None])
    if causal:
        keep = causal_keep(sq, sk, device=s.device)
        p = p.masked_fill(~keep, 0.0)
    dv_full = torch.matmul(p.transpose(-1, -2).contiguous(), dof)  # b h sk d
    dp = torch.matmul(dof, vf.transpose(-1, -2).contiguous())
    dsum = (of * dof).sum(dim=-1, keepdim=True)
    ds = p * (dp - dsum)
    dq = torch.matmul(ds, kf) * softmax_scale
    dk_full = torch.matmul(ds.transpose(-1, -2).contiguous(), qf) * softmax_scale
    dk = dk_full.reshape(b, hk, groups, sk, d).sum(dim=2)
    dv = dv_full.reshape(b, hk, groups, sk, d).sum(dim=2)
    return (
        dq.permute(0, 2, 1, 3).contiguous(),
        dk.permute(0, 2, 1, 3).contiguous(),
        dv.permute(0, 2, 1, 3).contiguous(),
    )


def _seq_slices(cu: torch.Tensor):
    cu_list = [int(x) for x in cu.tolist()]
    return [(cu_list[i], cu_list[i + 1]) for i in range(len(cu_list) - 1)]


def varlen_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    softmax_scale: float,
    causal: bool,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Packed varlen forward: per-sequence loop as in _varlen_reference
    (test_flash_attn.py:467-503).  LSE is [b, h, max_seqlen_q] with zeros past
    each sequence's length (flash_api.cpp:388; fwd_kernel.h:97-102)."""
    h = q.shape[1]
    qs, ks = _seq_slices(cu_seqlens_q), _seq_slices(cu_seqlens_k)
    out = torch.zeros(q.shape, dtype=dtype)
    lse = torch.zeros((len(qs), h, max_seqlen_q), dtype=dtype)
    for bi, ((q0, q1), (k0, k1)) in enumerate(zip(qs, ks)):
        o_i, l_i = attention_fwd(
            q[q0:q1][None], k[k0:k1][None], v[k0:k1][None], softmax_scale, causal, dtype
        )
        out[q0:q1] = o_i[0]
        lse[bi, :, : q1 - q0] = l_i[0]
    return out, lse


def varlen_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    softmax_scale: float,
    causal: bool,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Packed varlen backward, per-sequence closed form (flash_api.cpp:418-506)."""
    qs, ks = _seq_slices(cu_seqlens_q), _seq_slices(cu_seqlens_k)
    dq = torch.zeros(q.shape, dtype=dtype)
    dk = torch.zeros(k.shape, dtype=dtype)
    dv = torch.zeros(v.shape, dtype=dtype)
    for bi, ((q0, q1), (k0, k1)) in enumerate(zip(qs, ks)):
        g = attention_bwd(
            q[q0:q1][None],
            k[k0:k1][None],
            v[k0:k1][None],
            out[q0:q1][None],
            lse[bi : bi + 1, :, : q1 - q0],
            dout[q0:q1][None],
            softmax_scale,
            causal,
            dtype,
        )
        dq[q0:q1], dk[k0:k1], dv[k0:k1] = g[0][0], g[1][0], g[2][0]
    return dq, dk, dv



def bwd_fp32_noise(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    softmax_scale: float,
    causal: bool,
    growth: float = 4.0,
    dt: torch.dtype = torch.float64,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-element fp32 rounding-noise scale of (dq, dk, dv), in float32.

    First-order error model of any fp32 evaluation of the backward (the
    reference's MMA dP and warp-shuffle D, flash_bwd_kernel.h:385-436 and
    preprocess.h:74-94, as much as a HIP kernel), with eps = fp32 epsilon:
      * P = exp(scale*S - LSE): relative error rho_ij = eps * (|scale| (|Q||K|^T)_ij + |LSE_i| + 1);
      * dP - D: absolute error eps * A_ij, A_ij = (|dO||V|^T)_ij + sum_d |O_id dO_id|;
      * dS = P (dP - D): P rho |dP - D| + eps P A;
      * dV = P^T dO, dQ = scale dS K, dK = scale dS^T Q: the above pushed
        through absolute values, plus eps times the sum of |terms|;
    times ``growth`` for accumulation-order effects.  Where dP == D in real
    arithmetic (a row with one visible key, O = v) dS is pure noise of this
    size, which the twin's fp16 rounding points cannot show.  ``dt`` is the
    evaluation type (every term is a sum of non-negative products, so float32
    is enough for the full-size tests; float64 by default).
    """
    eps = torch.finfo(torch.float32).eps
    b, sq, h, d = q.shape
    sk, hk = k.shape[1], k.shape[2]
    groups = h // hk
    sc = abs(softmax_scale)
    qa = q.to(dt).permute(0, 2, 1, 3)
    ka = _expand_kv(k.to(dt), groups).permute(0, 2, 1, 3)
    va = _expand_kv(v.to(dt), groups).permute(0, 2, 1, 3)
    oa = out.to(dt).permute(0, 2, 1, 3)
    doa = dout.to(dt).permute(0, 2, 1, 3)
    l = lse.to(dt)[..., None]
    p = torch.exp(torch.matmul(qa, ka.transpose(-1, -2).contiguous()) * softmax_scale - l)
    if causal:
        p = p.masked_fill(~causal_keep(sq, sk), 0.0)
    rho = eps * (sc * torch.matmul(qa.abs(), ka.abs().transpose(-1, -2).contiguous()) + l.abs() + 1.0)
    dp_minus_d = torch.matmul(doa, va.transpose(-1, -2).contiguous()) - (oa * doa).sum(-1, keepdim=True)
    amag = torch.matmul(doa.abs(), va.abs().transpose(-1, -2).contiguous()) + (oa * doa).abs().sum(-1, keepdim=True)
    ds_abs = p * dp_minus_d.abs()
    ds_err = p * rho * dp_minus_d.abs() + eps * p * amag
    dq = sc * (torch.matmul(ds_err, ka.abs()) + eps * torch.matmul(ds_abs, ka.abs()))
    dk = sc * (torch.matmul(ds_err.transpose(-1, -2).contiguous(), qa.abs())
               + eps * torch.matmul(ds_abs.transpose(-1, -2).contiguous(), qa.abs()))
    pt = (p * (rho + eps)).transpose(-1, -2).contiguous()
    dv = torch.matmul(pt, doa.abs())
    dk = dk.reshape(b, hk, groups, sk, d).sum(dim=2)
    dv = dv.reshape(b, hk, groups, sk, d).sum(dim=2)
    return tuple((growth * x).permute(0, 2, 1, 3).contiguous().float() for x in (dq, dk, dv))
