"""Rounding-point twin of the reference CUDA kernels (CPU).  Test infrastructure only.

The reference kernels cannot be compiled or run here, so "the reference
kernel's own error against fp32 math" is estimated by re-running the
reference's arithmetic in PyTorch with fp32 everywhere except at the points
where the reference rounds to fp16:

forward (flash_fwd_kernel.h):
  * KV blocks of kBlockN = 64 (hd128) or 128 (hd64) keys, iterated from the
    last block to block 0 (:259, :455; flash_fwd_launch_template.h:97-118);
  * S scaled in fp32 after QK^T (:314-316); masked to -FLT_MAX (mask.h:88-95);
  * running max m, P = exp(S - m) in fp32 (:362-371), l summed from the fp32 P
    (:384-403), P rounded to fp16 before the PV product (:415, :578), O
    rescaled by exp(m_old - m) (:420-424);
  * epilogue O / l rounded to fp16, LSE = m + log(l), 0 for empty rows (:616-662).
backward (flash_bwd_kernel.h, flash_bwd_preprocess_kernel.h):
  * D = sum_d fp32(O) * fp32(dO) (preprocess.h:81-84);
  * P = exp(scale*S - LSE) fp32 (:417-424), P rounded to fp16 for dV (:1089-1092);
  * dS = P * (dP - D) rounded to fp16 for dQ and dK (:439-442, :1089-1105);
  * dQ = scale * dS K, dK = scale * dS^T Q, dV = P^T dO, each rounded to fp16
    (:585-592, :1317-1325); GQA: per-q-head fp16 dK/dV summed and rounded to
    fp16 again (flash_api.cpp:297-307, 338-348).
KV-cache decode / split kernels (kvcache_native.cu:577-599, 636-672, 697-724):
  fp32 scores, fp32 probabilities, fp32 partial outputs and combine; only the
  final output is rounded to fp16.  The twin is therefore the fp32 oracle
  followed by the fp16 rounding of the output.

MMA accumulation order and CUDA fast-math ``expf`` are not emulated; the twin
is an estimate of the reference's error, not a bit-exact copy.
"""

from typing import Tuple

import torch

from .attention import causal_keep

_FLT_MAX = torch.finfo(torch.float32).max


def _h(x: torch.Tensor) -> torch.Tensor:
    """Round to fp16 and return as fp32 (an fp16 rounding point)."""
    return x.to(torch.float16).to(torch.float32)


def fwd_twin(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, softmax_scale: float, causal: bool
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Returns (out fp16 [b, sq, h, d], lse fp32 [b, h, sq])."""
    b, sq, h, d = q.shape
    sk, hk = k.shape[1], k.shape[2]
    groups = h // hk
    block_n = 64 if d == 128 else 128
    qf = q.float().permute(0, 2, 1, 3)
    kf = k.float().repeat_interleave(groups, dim=2).permute(0, 2, 1, 3)
    vf = v.float().repeat_interleave(groups, dim=2).permute(0, 2, 1, 3)
    keep = causal_keep(sq, sk) if causal else torch.ones((sq, sk), dtype=torch.bool)
    m = torch.full((b, h, sq, 1), -_FLT_MAX)
    l = torch.zeros((b, h, sq, 1))
    o = torch.zeros((b, h, sq, d))
    n_blocks = (sk + block_n - 1) // block_n
    for nb in reversed(range(n_blocks)):
        j0, j1 = nb * block_n, min(sk, (nb + 1) * block_n)
        s = torch.matmul(qf, kf[:, :, j0:j1].transpose(-1, -2).contiguous()) * softmax_scale
        s = s.masked_fill(~keep[:, j0:j1], -_FLT_MAX)
        m_new = torch.maximum(m, s.amax(dim=-1, keepdim=True))
        dead = m_new == -_FLT_MAX
        p = torch.where(dead, torch.zeros_like(s), torch.exp(s - m_new))
        alpha = torch.exp(m - m_new)
        l = alpha * l + p.sum(dim=-1, keepdim=True)
        o = alpha * o + torch.matmul(_h(p), vf[:, :, j0:j1])
        m = m_new
    ok = l != 0
    out = torch.where(ok, o / torch.where(ok, l, torch.ones_like(l)), torch.zeros_like(o))
    lse = torch.where(ok, m + torch.log(torch.where(ok, l, torch.ones_like(l))), torch.zeros_like(m))
    return out.to(torch.float16).permute(0, 2, 1, 3).contiguous(), lse.squeeze(-1).contiguous()


def bwd_twin(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    dout: torch.Tensor,
    softmax_scale: float,
    causal: bool,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns fp16 (dq, dk, dv) following the reference's rounding points."""
    b, sq, h, d = q.shape
    sk, hk = k.shape[1], k.shape[2]
    groups = h // hk
    qf = q.float().permute(0, 2, 1, 3)
    kf = k.float().repeat_interleave(groups, dim=2).permute(0, 2, 1, 3)
    vf = v.float().repeat_interleave(groups, dim=2).permute(0, 2, 1, 3)
    of = out.float().permute(0, 2, 1, 3)
    dof = dout.float().permute(0, 2, 1, 3)
    dsum = (of * dof).sum(dim=-1, keepdim=True)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous())
    p = torch.exp(s * softmax_scale - lse.float()[..., None])
    if causal:
        p = p.masked_fill(~causal_keep(sq, sk), 0.0)
    dp = torch.matmul(dof, vf.transpose(-1, -2).contiguous())
    ds16 = _h(p * (dp - dsum))
    dq = _h(torch.matmul(ds16, kf) * softmax_scale)
    dk_h = _h(torch.matmul(ds16.transpose(-1, -2).contiguous(), qf) * softmax_scale)
    dv_h = _h(torch.matmul(_h(p).transpose(-1, -2).contiguous(), dof))
    if groups > 1:
        dk_h = _h(dk_h.reshape(b, hk, groups, sk, d).sum(dim=2))
        dv_h = _h(dv_h.reshape(b, hk, groups, sk, d).sum(dim=2))
    return (
        dq.to(torch.float16).permute(0, 2, 1, 3).contiguous(),
        dk_h.to(torch.float16).permute(0, 2, 1, 3).contiguous(),
        dv_h.to(torch.float16).permute(0, 2, 1, 3).contiguous(),
    )
