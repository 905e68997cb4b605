"""ctypes binding of the C ABI in include/fa_mi355x.h (libfa_mi355x.so).

This is the binding a non-torch host (or a maintainer wiring the library into
another runtime) would write: plain structs of device pointers, sizes and
strides, a stream handle and an int return code.  ``bench.py`` and the
C-ABI parity tests use it to launch the kernels one by one; the drop-in
Python API goes through the ``flash_attn_turing`` extension instead, which
calls the same entry points from C++.

Tensors are passed as torch tensors only for convenience: ``tensor_desc``
reads their data pointer and strides.  Nothing here allocates device memory.
Each argument struct built here holds references to the tensors it points at
(``_keep``), so their memory stays allocated for as long as the struct is
used; a pointer assigned to a field afterwards is the caller's to keep alive.
"""

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfa_mi355x.so")

FA_OK = 0
FA_ERR_INVALID_ARG = -1
FA_ERR_UNSUPPORTED = -2
FA_ERR_WORKSPACE = -3
FA_ERR_SCRATCH = -4

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_p = ctypes.c_void_p


class FaTensor(ctypes.Structure):
    _fields_ = [("ptr", _p), ("batch_stride", _i64), ("row_stride", _i64), ("head_stride", _i64)]


class FaFwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", FaTensor), ("k", FaTensor), ("v", FaTensor), ("o", FaTensor),
        ("lse", _p), ("cu_seqlens_q", _p), ("cu_seqlens_k", _p), ("seqused_k", _p), ("k_batch_idx", _p),
        ("seqused_k_add", _i32),
        ("batch", _i32), ("seqlen_q", _i32), ("seqlen_k", _i32), ("nheads", _i32), ("nheads_k", _i32),
        ("head_dim", _i32), ("lse_seqlen", _i32), ("softmax_scale", _f32), ("causal", _i32),
        ("k_batch", _i32), ("status", _p), ("work_order", _p),
    ]


class FaBwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", FaTensor), ("k", FaTensor), ("v", FaTensor), ("o", FaTensor), ("dout", FaTensor),
        ("dq", FaTensor), ("dk", FaTensor), ("dv", FaTensor),
        ("lse", _p), ("dsum", _p), ("cu_seqlens_q", _p), ("cu_seqlens_k", _p),
        ("batch", _i32), ("seqlen_q", _i32), ("seqlen_k", _i32), ("nheads", _i32), ("nheads_k", _i32),
        ("head_dim", _i32), ("lse_seqlen", _i32), ("softmax_scale", _f32), ("causal", _i32),
        ("work_order", _p),
    ]


class FaKvcacheArgs(ctypes.Structure):
    _fields_ = [
        ("q", FaTensor), ("k_cache", FaTensor), ("v_cache", FaTensor), ("k_new", FaTensor), ("v_new", FaTensor),
        ("o", FaTensor), ("lse", _p), ("cache_seqlens", _p), ("cache_batch_idx", _p), ("block_table", _p),
        ("block_table_stride", _i64),
        ("batch", _i32), ("seqlen_q", _i32), ("nheads", _i32), ("nheads_k", _i32), ("head_dim", _i32),
        ("seqlen_new", _i32), ("page_block_size", _i32), ("num_splits", _i32), ("softmax_scale", _f32),
        ("causal", _i32), ("out_accum", _p), ("lse_accum", _p), ("batch_order", _p),
        ("cache_capacity", _i32), ("cache_batch", _i32), ("status", _p),
        ("local_window", _i32), ("window_left", _i32), ("window_right", _i32), ("softcap", _f32),
        ("cache_leftpad", _p), ("alibi_slopes", _p), ("alibi_batch_stride", _i64),
        ("rotary_cos", _p), ("rotary_sin", _p), ("rotary_dim", _i32), ("rotary_seqlen", _i32),
        ("rotary_interleaved", _i32), ("split_count", _p),
    ]


_ARGP = {
    "fa_fwd": FaFwdArgs,
    "fa_bwd_preprocess": FaBwdArgs,
    "fa_bwd_dq": FaBwdArgs,
    "fa_bwd_dkdv": FaBwdArgs,
    "fa_bwd": FaBwdArgs,
    "fa_kv_append": FaKvcacheArgs,
    "fa_kv_splitkv": FaKvcacheArgs,
    "fa_kv_combine": FaKvcacheArgs,
    "fa_fwd_kvcache": FaKvcacheArgs,
    "fa_fwd_kvcache_noalloc": FaKvcacheArgs,
}

# FA_ABI_VERSION of include/fa_mi355x.h whose struct layouts the classes above mirror.
ABI_VERSION = 3

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libfa_mi355x.so once and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built; run flash-attention-turing_amd/build.py")
    lib = ctypes.CDLL(path)
    lib.fa_abi_version.restype = ctypes.c_int
    if lib.fa_abi_version() != ABI_VERSION:
        raise ImportError(f"{path} has argument-struct layout version {lib.fa_abi_version()}, this binding "
                          f"declares version {ABI_VERSION}: rebuild the library or update fa_capi.py")
    for name, st in _ARGP.items():
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.POINTER(st), _p]
        fn.restype = ctypes.c_int
    lib.fa_kv_num_splits.argtypes = [ctypes.c_int] * 8
    lib.fa_kv_num_splits.restype = ctypes.c_int
    lib.fa_kv_workspace_bytes.argtypes = [ctypes.POINTER(FaKvcacheArgs)]
    lib.fa_kv_workspace_bytes.restype = ctypes.c_size_t
    lib.fa_kv_split_count_len.argtypes = [ctypes.POINTER(FaKvcacheArgs)]
    lib.fa_kv_split_count_len.restype = ctypes.c_size_t
    lib.fa_fwd_order_len.argtypes = [ctypes.POINTER(FaFwdArgs)]
    lib.fa_fwd_order_len.restype = ctypes.c_size_t
    lib.fa_bwd_order_len.argtypes = [ctypes.POINTER(FaBwdArgs)]
    lib.fa_bwd_order_len.restype = ctypes.c_size_t
    lib.fa_error_string.argtypes = [ctypes.c_int]
    lib.fa_error_string.restype = ctypes.c_char_p
    _lib = lib
    return lib


def tensor_desc(t, packed: bool = False) -> FaTensor:
    """[batch][row][head][d] (or packed [total][head][d]) strided view -> FaTensor."""
    if t is None:
        return FaTensor(None, 0, 0, 0)
    if packed:
        return FaTensor(t.data_ptr(), 0, t.stride(0), t.stride(1))
    return FaTensor(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(stream=None) -> int:
    """The raw hipStream_t of a torch stream (current stream by default)."""
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


def call(name: str, args, stream=None) -> None:
    """Invoke entry point ``name``; raise RuntimeError with the library's message on error."""
    lib = load()
    rc = getattr(lib, name)(ctypes.byref(args), ctypes.c_void_p(stream_handle(stream)))
    if rc != FA_OK:
        raise RuntimeError(f"{name} failed: {lib.fa_error_string(rc).decode()}")


def fwd_args(q, k, v, o, lse, softmax_scale: float, causal: bool, cu_seqlens_q=None, cu_seqlens_k=None,
             max_seqlen_q: int = 0, max_seqlen_k: int = 0, work_order=None) -> FaFwdArgs:
    packed = cu_seqlens_q is not None
    a = FaFwdArgs()
    a.q, a.k, a.v, a.o = (tensor_desc(x, packed) for x in (q, k, v, o))
    a.lse = lse.data_ptr()
    a.cu_seqlens_q, a.cu_seqlens_k = ptr(cu_seqlens_q), ptr(cu_seqlens_k)
    if packed:
        a.batch = cu_seqlens_q.numel() - 1
        a.seqlen_q, a.seqlen_k = max_seqlen_q, max_seqlen_k
        a.nheads, a.nheads_k, a.head_dim = q.shape[1], k.shape[1], q.shape[2]
        a.lse_seqlen = max_seqlen_q
    else:
        a.batch, a.seqlen_q, a.nheads, a.head_dim = q.shape
        a.seqlen_k, a.nheads_k = k.shape[1], k.shape[2]
        a.lse_seqlen = q.shape[1]
    a.softmax_scale = softmax_scale
    a.causal = int(causal)
    a.work_order = ptr(work_order)
    a._keep = (q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k, work_order)
    return a


def bwd_args(q, k, v, o, lse, dout, dq, dk, dv, dsum, softmax_scale: float, causal: bool, cu_seqlens_q=None,
             cu_seqlens_k=None, max_seqlen_q: int = 0, max_seqlen_k: int = 0, work_order=None) -> FaBwdArgs:
    packed = cu_seqlens_q is not None
    a = FaBwdArgs()
    a.q, a.k, a.v, a.o, a.dout, a.dq, a.dk, a.dv = (
        tensor_desc(x, packed) for x in (q, k, v, o, dout, dq, dk, dv)
    )
    a.lse, a.dsum = lse.data_ptr(), dsum.data_ptr()
    a.cu_seqlens_q, a.cu_seqlens_k = ptr(cu_seqlens_q), ptr(cu_seqlens_k)
    if packed:
        a.batch = cu_seqlens_q.numel() - 1
        a.seqlen_q, a.seqlen_k = max_seqlen_q, max_seqlen_k
        a.nheads, a.nheads_k, a.head_dim = q.shape[1], k.shape[1], q.shape[2]
        a.lse_seqlen = max_seqlen_q
    else:
        a.batch, a.seqlen_q, a.nheads, a.head_dim = q.shape
        a.seqlen_k, a.nheads_k = k.shape[1], k.shape[2]
        a.lse_seqlen = q.shape[1]
    a.softmax_scale = softmax_scale
    a.causal = int(causal)
    a.work_order = ptr(work_order)
    a._keep = (q, k, v, o, lse, dout, dq, dk, dv, dsum, cu_seqlens_q, cu_seqlens_k, work_order)
    return a


def kvcache_args(q, k_cache, v_cache, o, lse, cache_seqlens, softmax_scale: float, causal: bool, num_splits: int,
                 k_new=None, v_new=None, cache_batch_idx=None, block_table=None, out_accum=None,
                 lse_accum=None, batch_order=None, status=None, window=(-1, -1),
                 softcap: float = 0.0, cache_leftpad=None, alibi_slopes=None, rotary_cos=None, rotary_sin=None,
                 rotary_interleaved: bool = True, split_count=None) -> FaKvcacheArgs:
    a = FaKvcacheArgs()
    a.q, a.k_cache, a.v_cache, a.o = (tensor_desc(x) for x in (q, k_cache, v_cache, o))
    a.k_new, a.v_new = tensor_desc(k_new), tensor_desc(v_new)
    a.lse = lse.data_ptr()
    a.cache_seqlens, a.cache_batch_idx, a.block_table = ptr(cache_seqlens), ptr(cache_batch_idx), ptr(block_table)
    a.block_table_stride = block_table.stride(0) if block_table is not None else 0
    a.batch, a.seqlen_q, a.nheads, a.head_dim = q.shape
    a.nheads_k = k_cache.shape[2]
    a.seqlen_new = 0 if k_new is None else k_new.shape[1]
    a.page_block_size = k_cache.shape[1] if block_table is not None else 0
    a.num_splits = num_splits
    a.softmax_scale = softmax_scale
    a.causal = int(causal)
    a.out_accum, a.lse_accum = ptr(out_accum), ptr(lse_accum)
    a.batch_order = ptr(batch_order)
    a.cache_capacity = k_cache.shape[1] * (block_table.shape[1] if block_table is not None else 1)
    a.cache_batch = k_cache.shape[0] if block_table is None else 0
    a.status = ptr(status)
    a.local_window = int(tuple(window) != (-1, -1))
    a.window_left, a.window_right = window
    a.softcap = softcap
    a.cache_leftpad = ptr(cache_leftpad)
    a.alibi_slopes = ptr(alibi_slopes)
    a.alibi_batch_stride = alibi_slopes.stride(0) if alibi_slopes is not None and alibi_slopes.dim() == 2 else 0
    a.rotary_cos, a.rotary_sin = ptr(rotary_cos), ptr(rotary_sin)
    a.rotary_dim = 0 if rotary_cos is None else 2 * rotary_cos.shape[1]
    a.rotary_seqlen = 0 if rotary_cos is None else rotary_cos.shape[0]
    a.rotary_interleaved = int(rotary_interleaved)
    a.split_count = ptr(split_count)
    a._keep = (q, k_cache, v_cache, o, lse, cache_seqlens, k_new, v_new, cache_batch_idx, block_table, out_accum,
               lse_accum, batch_order, status, cache_leftpad, alibi_slopes, rotary_cos, rotary_sin, split_count)
    return a
