"""Python interface of the MI355X FlashAttention (drop-in for the reference's
flash_attention_interface.py).

Public API, argument order, defaults, validation order and error messages follow
the reference module (flash_attention_interface.py:448-922):

    flash_attn_func, flash_attn_qkvpacked_func, flash_attn_kvpacked_func,
    flash_attn_varlen_func, flash_attn_varlen_qkvpacked_func,
    flash_attn_varlen_kvpacked_func, flash_attn_with_kvcache

and the autograd classes FlashAttnFunc, FlashAttnQKVPackedFunc,
FlashAttnKVPackedFunc, FlashAttnVarlenFunc, FlashAttnVarlenQKVPackedFunc,
FlashAttnVarlenKVPackedFunc (:172-445).  Every call goes to the native
``flash_attn_turing`` extension (HIP kernels for gfx950); there is no Python
math fallback: a missing or incompatible extension raises at import or call.
"""

import math
from typing import Optional, Tuple, Union

import torch  # noqa: F401  (loads the HIP runtime before the extension)

import flash_attn_turing as flash_attn_gpu


def maybe_contiguous(x: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """Copy only tensors whose last dimension is strided (interface.py:9-10)."""
    if x is None or x.stride(-1) == 1:
        return x
    return x.contiguous()


def _default_scale(q: torch.Tensor, softmax_scale: Optional[float]) -> float:
    # interface.py:183: head_dim ** -0.5 unless given.
    return q.shape[-1] ** (-0.5) if softmax_scale is None else softmax_scale


# ---------------------------------------------------------------------------
# Thin wrappers over the extension (interface.py:13-169).


def _flash_attn_forward(q, k, v, softmax_scale: float, causal: bool):
    q, k, v = (maybe_contiguous(t) for t in (q, k, v))
    out, lse = flash_attn_gpu.fwd(q, k, v, softmax_scale, causal)
    return out, lse


def _flash_attn_backward(dout, q, k, v, out, lse, softmax_scale: float, causal: bool, dq=None, dk=None, dv=None):
    """dq / dk / dv, when given, are written in place (e.g. slices of a packed dqkv) and returned."""
    dout, q, k, v, out, lse = (maybe_contiguous(t) for t in (dout, q, k, v, out, lse))
    dq, dk, dv = flash_attn_gpu.bwd(q, k, v, out, lse, dout, softmax_scale, causal, dq, dk, dv)
    return dq, dk, dv


def _flash_attn_varlen_forward(
    q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int, softmax_scale: float, causal: bool
):
    q, k, v = (maybe_contiguous(t) for t in (q, k, v))
    out, lse = flash_attn_gpu.varlen_fwd(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal
    )
    return out, lse


def _flash_attn_varlen_backward(
    dout,
    q,
    k,
    v,
    out,
    lse,
    cu_seqlens_q,
    cu_seqlens_k,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    causal: bool,
    dq=None,
    dk=None,
    dv=None,
):
    """dq / dk / dv, when given, are written in place (rows no sequence covers are left as they are)."""
    dout, q, k, v, out, lse = (maybe_contiguous(t) for t in (dout, q, k, v, out, lse))
    dq, dk, dv = flash_attn_gpu.varlen_bwd(
        q, k, v, out, lse, dout, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal,
        dq, dk, dv,
    )
    return dq, dk, dv


def _flash_attn_kvcache_forward(
    q, k_cache, v_cache, k, v, cache_seqlens, cache_batch_idx, block_table, softmax_scale: float, causal: bool,
    num_splits: int, status: Optional[torch.Tensor] = None, window_size: Tuple[int, int] = (-1, -1),
    softcap: float = 0.0, cache_leftpad: Optional[torch.Tensor] = None, alibi_slopes: Optional[torch.Tensor] = None,
    rotary_cos: Optional[torch.Tensor] = None, rotary_sin: Optional[torch.Tensor] = None,
    rotary_interleaved: bool = True,
):
    tensors = (q, k_cache, v_cache, k, v, cache_seqlens, cache_batch_idx, block_table, cache_leftpad, alibi_slopes)
    q, k_cache, v_cache, k, v, cache_seqlens, cache_batch_idx, block_table, cache_leftpad, alibi_slopes = (
        maybe_contiguous(t) for t in tensors
    )
    # The 20-argument binding of flash_api.cpp:508-528; a preallocated out is
    # passed as "absent".
    out, lse = flash_attn_gpu.fwd_kvcache(
        q, k_cache, v_cache, k, v, cache_seqlens,
        rotary_cos, rotary_sin,
        cache_batch_idx,
        cache_leftpad,
        block_table,
        alibi_slopes,
        None,                  # out
        softmax_scale, causal,
        int(window_size[0]), int(window_size[1]),
        float(softcap),
        bool(rotary_interleaved),
        num_splits,
        status,                # device-side input checks instead of host reads, when given
    )
    return out, lse


# ---------------------------------------------------------------------------
# Autograd functions (interface.py:172-445).


class FlashAttnFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, causal, is_grad_enabled):
        softmax_scale = _default_scale(q, softmax_scale)
        out, lse = _flash_attn_forward(q, k, v, softmax_scale, causal)
        if is_grad_enabled and (q.requires_grad or k.requires_grad or v.requires_grad):
            ctx.save_for_backward(q, k, v, out, lse)
            ctx.softmax_scale, ctx.causal = softmax_scale, causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = _flash_attn_backward(dout, q, k, v, out, lse, ctx.softmax_scale, ctx.causal)
        return dq, dk, dv, None, None, None


# Packed inputs: the kernels take row and head strides, so q / k / v are
# passed as views of the packed tensor (no copies, unlike the reference's
# interface.py:208-212, 244-247), and the backward writes the gradient slices
# straight into one packed gradient (no torch.stack, interface.py:226-231).


def _unpack(packed: torch.Tensor, dim: int, n: int):
    return tuple(packed.select(dim=dim, index=i) for i in range(n))


def _packed_grad(packed, dim: int, zero: bool):
    """A gradient for a packed input (shape, dtype, device) and its slices along dim."""
    shape, dtype, device = packed
    g = (torch.zeros if zero else torch.empty)(shape, dtype=dtype, device=device)
    return g, tuple(g.select(dim=dim, index=i) for i in range(shape[dim]))


class FlashAttnQKVPackedFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, softmax_scale, causal, is_grad_enabled):
        q, k, v = _unpack(qkv, 2, 3)
        softmax_scale = _default_scale(q, softmax_scale)
        out, lse = _flash_attn_forward(q, k, v, softmax_scale, causal)
        if is_grad_enabled and qkv.requires_grad:
            ctx.save_for_backward(q, k, v, out, lse)
            ctx.packed = (qkv.shape, qkv.dtype, qkv.device)
            ctx.softmax_scale, ctx.causal = softmax_scale, causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dqkv, (dq, dk, dv) = _packed_grad(ctx.packed, 2, False)
        _flash_attn_backward(dout, q, k, v, out, lse, ctx.softmax_scale, ctx.causal, dq, dk, dv)
        return dqkv, None, None, None


class FlashAttnKVPackedFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, kv, softmax_scale, causal, is_grad_enabled):
        k, v = _unpack(kv, 2, 2)
        softmax_scale = _default_scale(q, softmax_scale)
        out, lse = _flash_attn_forward(q, k, v, softmax_scale, causal)
        if is_grad_enabled and (q.requires_grad or kv.requires_grad):
            ctx.save_for_backward(q, k, v, out, lse)
            ctx.packed = (kv.shape, kv.dtype, kv.device)
            ctx.softmax_scale, ctx.causal = softmax_scale, causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        dkv, (dk, dv) = _packed_grad(ctx.packed, 2, False)
        dq, _, _ = _flash_attn_backward(dout, q, k, v, out, lse, ctx.softmax_scale, ctx.causal, None, dk, dv)
        return dq, dkv, None, None, None


class FlashAttnVarlenFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal,
                is_grad_enabled):
        softmax_scale = _default_scale(q, softmax_scale)
        out, lse = _flash_attn_varlen_forward(
            q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal
        )
        if is_grad_enabled and (q.requires_grad or k.requires_grad or v.requires_grad):
            ctx.save_for_backward(q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k)
            ctx.max_seqlen_q, ctx.max_seqlen_k = max_seqlen_q, max_seqlen_k
            ctx.softmax_scale, ctx.causal = softmax_scale, causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k = ctx.saved_tensors
        dq, dk, dv = _flash_attn_varlen_backward(
            dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, ctx.max_seqlen_q, ctx.max_seqlen_k,
            ctx.softmax_scale, ctx.causal,
        )
        return dq, dk, dv, None, None, None, None, None, None, None


class FlashAttnVarlenQKVPackedFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, cu_seqlens, max_seqlen, softmax_scale, causal, is_grad_enabled):
        q, k, v = _unpack(qkv, 1, 3)
        softmax_scale = _default_scale(q, softmax_scale)
        out, lse = _flash_attn_varlen_forward(
            q, k, v, cu_seqlens, cu_seqlens, max_seqlen, max_seqlen, softmax_scale, causal
        )
        if is_grad_enabled and qkv.requires_grad:
            ctx.save_for_backward(q, k, v, out, lse, cu_seqlens)
            ctx.packed = (qkv.shape, qkv.dtype, qkv.device)
            ctx.max_seqlen = max_seqlen
            ctx.softmax_scale, ctx.causal = softmax_scale, causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, cu_seqlens = ctx.saved_tensors
        dqkv, (dq, dk, dv) = _packed_grad(ctx.packed, 1, True)
        _flash_attn_varlen_backward(
            dout, q, k, v, out, lse, cu_seqlens, cu_seqlens, ctx.max_seqlen, ctx.max_seqlen,
            ctx.softmax_scale, ctx.causal, dq, dk, dv,
        )
        return dqkv, None, None, None, None, None


class FlashAttnVarlenKVPackedFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal,
                is_grad_enabled):
        k, v = _unpack(kv, 1, 2)
        softmax_scale = _default_scale(q, softmax_scale)
        out, lse = _flash_attn_varlen_forward(
            q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal
        )
        if is_grad_enabled and (q.requires_grad or kv.requires_grad):
            ctx.save_for_backward(q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k)
            ctx.packed = (kv.shape, kv.dtype, kv.device)
            ctx.max_seqlen_q, ctx.max_seqlen_k = max_seqlen_q, max_seqlen_k
            ctx.softmax_scale, ctx.causal = softmax_scale, causal
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k = ctx.saved_tensors
        dkv, (dk, dv) = _packed_grad(ctx.packed, 1, True)
        dq, _, _ = _flash_attn_varlen_backward(
            dout, q, k, v, out, lse, cu_seqlens_q, cu_seqlens_k, ctx.max_seqlen_q, ctx.max_seqlen_k,
            ctx.softmax_scale, ctx.causal, None, dk, dv,
        )
        return dq, dkv, None, None, None, None, None, None, None


# ---------------------------------------------------------------------------
# Public functions (interface.py:448-614).


def flash_attn_func(q, k, v, softmax_scale: Optional[float] = None, causal: bool = False) -> torch.Tensor:
    """q (batch, seqlen_q, nheads, headdim); k, v (batch, seqlen_k, nheads_k, headdim).
    Returns out (batch, seqlen_q, nheads, headdim)."""
    return FlashAttnFunc.apply(q, k, v, softmax_scale, causal, torch.is_grad_enabled())


def flash_attn_qkvpacked_func(qkv, softmax_scale: Optional[float] = None, causal: bool = False) -> torch.Tensor:
    """qkv (batch, seqlen, 3, nheads, headdim).  Returns out (batch, seqlen, nheads, headdim)."""
    return FlashAttnQKVPackedFunc.apply(qkv, softmax_scale, causal, torch.is_grad_enabled())


def flash_attn_kvpacked_func(q, kv, softmax_scale: Optional[float] = None, causal: bool = False) -> torch.Tensor:
    """q (batch, seqlen_q, nheads, headdim); kv (batch, seqlen_k, 2, nheads_k, headdim)."""
    return FlashAttnKVPackedFunc.apply(q, kv, softmax_scale, causal, torch.is_grad_enabled())


def flash_attn_varlen_func(
    q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int,
    softmax_scale: Optional[float] = None, causal: bool = False,
) -> torch.Tensor:
    """q (total_q, nheads, headdim); k, v (total_k, nheads_k, headdim); cu_seqlens_* int32
    (batch_size + 1,).  Returns out (total_q, nheads, headdim)."""
    return FlashAttnVarlenFunc.apply(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal,
        torch.is_grad_enabled(),
    )


def flash_attn_varlen_qkvpacked_func(
    qkv, cu_seqlens, max_seqlen: int, softmax_scale: Optional[float] = None, causal: bool = False
) -> torch.Tensor:
    """qkv (total, 3, nheads, headdim); cu_seqlens int32 (batch_size + 1,)."""
    return FlashAttnVarlenQKVPackedFunc.apply(
        qkv, cu_seqlens, max_seqlen, softmax_scale, causal, torch.is_grad_enabled()
    )


def flash_attn_varlen_kvpacked_func(
    q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int,
    softmax_scale: Optional[float] = None, causal: bool = False,
) -> torch.Tensor:
    """q (total_q, nheads, headdim); kv (total_k, 2, nheads_k, headdim)."""
    return FlashAttnVarlenKVPackedFunc.apply(
        q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal,
        torch.is_grad_enabled(),
    )


# ---------------------------------------------------------------------------
# KV cache (interface.py:617-922).


def _validate_unsupported_kvcache_args(rotary_cos, rotary_sin, cache_leftpad, window_size, softcap, alibi_slopes):
    # interface.py:617-634 rejects all five; here they are supported with
    # upstream FlashAttention's semantics, so only their types are checked.
    for name, t in (("rotary_cos", rotary_cos), ("rotary_sin", rotary_sin)):
        if t is not None and (not isinstance(t, torch.Tensor) or t.dtype != torch.float16 or t.dim() != 2):
            raise TypeError(f"{name} must be a 2-D torch.float16 tensor (seqlen_ro, rotary_dim / 2)")
    if len(tuple(window_size)) != 2 or not all(isinstance(w, int) for w in window_size):
        raise TypeError("window_size must be a pair of ints")
    if not math.isfinite(softcap):
        raise ValueError("softcap must be finite")
    if cache_leftpad is not None and (not isinstance(cache_leftpad, torch.Tensor) or cache_leftpad.dtype != torch.int32):
        raise TypeError("cache_leftpad must be a torch.int32 tensor")
    if alibi_slopes is not None and (not isinstance(alibi_slopes, torch.Tensor) or alibi_slopes.dtype != torch.float32):
        raise TypeError("alibi_slopes must be a torch.float32 tensor")


def _validate_supported_head_dim(head_dim: int) -> None:
    if head_dim not in (64, 128):
        raise ValueError("Turing FlashAttention supports head_dim 64 or 128")


def _cache_capacity(k_cache: torch.Tensor, block_table: Optional[torch.Tensor]) -> int:
    return k_cache.shape[1] if block_table is None else block_table.shape[1] * k_cache.shape[1]


# Status words of the synchronisation-free KV-cache mode, one int32 per device.
_KV_STATUS = {}

# Bits of a status word and the errors the synchronous checks raise for them
# (interface.py:855-857 for the capacity, flash_api.cpp:634-641 for the rows).
_KV_STATUS_ERRORS = (
    (1, ValueError, "cache capacity is insufficient for the requested append length"),
    (2, RuntimeError, "cache_batch_idx entries must be within cache batch bounds"),
)


def _kv_status(device: torch.device) -> torch.Tensor:
    index = torch.device(device).index
    if index is None:
        index = torch.cuda.current_device()
    st = _KV_STATUS.get(index)
    if st is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                "flash_attn_with_kvcache(validate=False) needs its status word allocated before graph capture: "
                "call flash_attn_kvcache_check() once on this device first"
            )
        st = torch.zeros(1, dtype=torch.int32, device=torch.device("cuda", index))
        _KV_STATUS[index] = st
    return st


def flash_attn_kvcache_check(device: Optional[Union[torch.device, int]] = None) -> None:
    """Report what earlier flash_attn_with_kvcache(validate=False) calls on a
    device found wrong, then clear it.

    Such calls read neither cache_seqlens nor cache_batch_idx on the host; the
    kernels check them instead.  A sequence that would overflow its cache, or
    whose cache_batch_idx is outside the cache, is left unchanged in the cache
    and gets O = 0 (LSE 0); this function then raises the error the default
    (validate=True) call raises at once: ValueError for the capacity,
    RuntimeError for the cache row.  It reads the device (a synchronisation),
    so call it outside captured graphs, for instance after each replay or
    every few steps.  It also allocates the device's status word, which must
    exist before a validate=False call is captured.
    """
    st = _kv_status(torch.device("cuda", device) if isinstance(device, int) else (device or torch.device("cuda")))
    bits = int(st.item())
    if bits:
        st.zero_()
        for bit, exc, msg in _KV_STATUS_ERRORS:
            if bits & bit:
                raise exc(msg)


def flash_attn_with_kvcache(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k: Optional[torch.Tensor] = None,
    v: Optional[torch.Tensor] = None,
    rotary_cos: Optional[torch.Tensor] = None,
    rotary_sin: Optional[torch.Tensor] = None,
    cache_seqlens: Optional[Union[torch.Tensor, int]] = None,
    cache_batch_idx: Optional[torch.Tensor] = None,
    cache_leftpad: Optional[torch.Tensor] = None,
    block_table: Optional[torch.Tensor] = None,
    softmax_scale: Optional[float] = None,
    causal: bool = False,
    window_size: Tuple[int, int] = (-1, -1),
    softcap: float = 0.0,
    rotary_interleaved: bool = True,
    alibi_slopes: Optional[torch.Tensor] = None,
    num_splits: int = 0,
    return_softmax_lse: bool = False,
    validate: bool = True,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """KV-cache attention for inference (signature of upstream FlashAttention).

    Supports contiguous caches (optionally remapped by cache_batch_idx), paged
    caches via block_table, in-place append of k/v at cache_seqlens and split-KV
    (num_splits, 0 = heuristic).  Beyond the reference (which rejects them),
    rotary embeddings, window_size, softcap, alibi_slopes and cache_leftpad work
    with upstream FlashAttention's semantics: query i, at key position
    p = i + L - seqlen_q, sees keys [p - left, p + right] (-1: unbounded; causal
    caps the right side at p); softcap > 0 replaces each scaled score x by
    softcap * tanh(x / softcap); ALiBi (fp32 slopes [nheads] or [batch, nheads])
    adds -slope * |p - j| to the score of key j; keys before cache_leftpad[b]
    (int32 [batch]) do not exist.  With rotary_cos / rotary_sin (fp16
    [seqlen_ro, rotary_dim / 2]; k and v required), the first rotary_dim channels
    of new key t are rotated at position cache_seqlens[b] + t before the append,
    and q's at cache_seqlens[b] + i when causal or windowed, else at
    cache_seqlens[b]; rotary_interleaved pairs channels (2j, 2j + 1), otherwise
    (j, j + rotary_dim / 2).

    validate (after the reference's arguments): True checks the cache capacity
    and cache_batch_idx on the host, raising at once as the reference does (two
    device reads, so no graph capture).  False skips those reads: the kernels
    check every sequence themselves (an out-of-range one is neither appended to
    nor attended over) and record the error for flash_attn_kvcache_check(),
    so a decode step can be captured in a HIP graph.
    """
    # Validation order of interface.py:807-867.
    _validate_unsupported_kvcache_args(rotary_cos, rotary_sin, cache_leftpad, window_size, softcap, alibi_slopes)
    if (k is None) != (v is None):
        raise ValueError("k and v must either both be provided or both be None")
    _validate_supported_head_dim(q.shape[-1])
    batch = q.shape[0]
    if cache_seqlens is None:
        if k is not None:
            raise ValueError("cache_seqlens is required when appending k and v")
        cache_seqlens = torch.full(
            (batch,), _cache_capacity(k_cache, block_table), dtype=torch.int32, device=k_cache.device
        )
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((batch,), cache_seqlens, dtype=torch.int32, device=k_cache.device)
    elif not isinstance(cache_seqlens, torch.Tensor):
        raise TypeError("cache_seqlens must be an int or a torch.Tensor")
    elif cache_seqlens.dtype != torch.int32:
        raise TypeError("cache_seqlens must be a torch.int32 tensor")
    if cache_seqlens.dim() != 1 or cache_seqlens.numel() != batch:
        raise ValueError("cache_seqlens must have shape [batch_size]")
    if block_table is not None:
        if not isinstance(block_table, torch.Tensor):
            raise TypeError("block_table must be a torch.Tensor")
        if block_table.dtype != torch.int32:
            raise TypeError("block_table must be a torch.int32 tensor")
        if block_table.dim() != 2 or block_table.shape[0] != batch:
            raise ValueError("block_table must have shape [batch_size, max_num_blocks_per_seq]")
        if cache_batch_idx is not None:
            raise NotImplementedError("Paged KV cache does not support cache_batch_idx")
        if k_cache.shape[1] % 256 != 0:
            raise ValueError("Paged KV cache block size must be divisible by 256")
    if cache_batch_idx is not None:
        if not isinstance(cache_batch_idx, torch.Tensor):
            raise TypeError("cache_batch_idx must be a torch.Tensor")
        if cache_batch_idx.dtype != torch.int32:
            raise TypeError("cache_batch_idx must be a torch.int32 tensor")
        if cache_batch_idx.dim() != 1 or cache_batch_idx.numel() != batch:
            raise ValueError("cache_batch_idx must have shape [batch_size]")
    if num_splits < 0:
        raise ValueError("num_splits must be non-negative")
    seqlen_new = 0
    if k is not None and v is not None:
        if k.shape[0] != batch or v.shape[0] != batch:
            raise ValueError("k and v batch size must match q")
        if k.shape[1] != v.shape[1]:
            raise ValueError("k and v sequence length must match")
        seqlen_new = k.shape[1]
    if validate:
        max_cache_usage = int(cache_seqlens.max().item()) if cache_seqlens.numel() > 0 else 0
        if max_cache_usage + seqlen_new > _cache_capacity(k_cache, block_table):
            raise ValueError("cache capacity is insufficient for the requested append length")
    if not (q.is_cuda and k_cache.is_cuda and v_cache.is_cuda):
        raise RuntimeError("q, k_cache, v_cache must be CUDA tensors")
    if q.dtype != torch.float16 or k_cache.dtype != torch.float16 or v_cache.dtype != torch.float16:
        raise RuntimeError("q, k_cache, v_cache must be float16 tensors")
    if k is not None and v is not None:
        if not (k.is_cuda and v.is_cuda):
            raise RuntimeError("k and v must be CUDA tensors")
        if k.dtype != torch.float16 or v.dtype != torch.float16:
            raise RuntimeError("k and v must be float16 tensors")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** (-0.5)
    status = None if validate else _kv_status(q.device)
    out, lse = _flash_attn_kvcache_forward(
        q, k_cache, v_cache, k, v, cache_seqlens, cache_batch_idx, block_table, softmax_scale, causal, num_splits,
        status, tuple(window_size), softcap, cache_leftpad, alibi_slopes, rotary_cos, rotary_sin, rotary_interleaved,
    )
    return (out, lse) if return_softmax_lse else out
