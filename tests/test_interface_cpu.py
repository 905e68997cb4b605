"""Host-only checks of the drop-in interface (no GPU needed).

Restates the reference's argument-validation tests (test_flash_attn.py:1967-2093)
with the same exception types and message regexes, plus the explicit
NotImplementedError rejections of interface.py:617-634 and the validation order
(unsupported features, then k/v pairing, then head_dim, then the rest;
capacity before device).  These run on CPU tensors, so they exercise the
Python layer only; the module still imports the compiled extension.
"""

import inspect

import pytest
import torch

import flash_attention_interface as fai
import flash_attn_turing


def _t(*shape, dtype=torch.float32):
    return torch.randn(*shape, dtype=dtype)


def test_requires_cache_seqlens_for_append():
    with pytest.raises(ValueError, match="cache_seqlens is required when appending"):
        fai.flash_attn_with_kvcache(_t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), k=_t(1, 1, 2, 64), v=_t(1, 1, 2, 64))


def test_requires_paired_kv():
    with pytest.raises(ValueError, match="k and v must either both be provided"):
        fai.flash_attn_with_kvcache(
            _t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), k=_t(1, 2, 2, 64),
            cache_seqlens=torch.tensor([4], dtype=torch.int32),
        )


def test_requires_int32_cache_seqlens():
    with pytest.raises(TypeError, match="cache_seqlens must be a torch.int32 tensor"):
        fai.flash_attn_with_kvcache(
            _t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), cache_seqlens=torch.tensor([4], dtype=torch.int64)
        )


def test_rejects_non_tensor_cache_seqlens():
    with pytest.raises(TypeError, match="cache_seqlens must be an int or a torch.Tensor"):
        fai.flash_attn_with_kvcache(_t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), cache_seqlens=[4])


def test_rejects_cpu_tensors():
    with pytest.raises(RuntimeError, match="must be CUDA tensors"):
        fai.flash_attn_with_kvcache(
            _t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), cache_seqlens=torch.tensor([4], dtype=torch.int32)
        )


def test_requires_batch_sized_cache_seqlens():
    with pytest.raises(ValueError, match=r"cache_seqlens must have shape \[batch_size\]"):
        fai.flash_attn_with_kvcache(
            _t(2, 2, 4, 64), _t(2, 8, 2, 64), _t(2, 8, 2, 64), cache_seqlens=torch.tensor([4], dtype=torch.int32)
        )


def test_rejects_unsupported_head_dim():
    with pytest.raises(ValueError, match="head_dim 64 or 128"):
        fai.flash_attn_with_kvcache(
            _t(1, 2, 4, 96), _t(1, 8, 2, 96), _t(1, 8, 2, 96), cache_seqlens=torch.tensor([4], dtype=torch.int32)
        )


def test_requires_int32_cache_batch_idx():
    with pytest.raises(TypeError, match="cache_batch_idx must be a torch.int32 tensor"):
        fai.flash_attn_with_kvcache(
            _t(1, 2, 4, 64), _t(2, 8, 2, 64), _t(2, 8, 2, 64), cache_seqlens=torch.tensor([4], dtype=torch.int32),
            cache_batch_idx=torch.tensor([1], dtype=torch.int64),
        )


def test_requires_batch_sized_cache_batch_idx():
    with pytest.raises(ValueError, match=r"cache_batch_idx must have shape \[batch_size\]"):
        fai.flash_attn_with_kvcache(
            _t(2, 2, 4, 64), _t(3, 8, 2, 64), _t(3, 8, 2, 64), cache_seqlens=torch.tensor([4, 5], dtype=torch.int32),
            cache_batch_idx=torch.tensor([1], dtype=torch.int32),
        )


def test_rejects_capacity_overrun():
    with pytest.raises(ValueError, match="cache capacity is insufficient"):
        fai.flash_attn_with_kvcache(
            _t(1, 2, 4, 64), _t(1, 5, 2, 64), _t(1, 5, 2, 64), k=_t(1, 2, 2, 64), v=_t(1, 2, 2, 64),
            cache_seqlens=torch.tensor([4], dtype=torch.int32),
        )


def test_feature_type_checks_come_first():
    # head_dim 96 and unpaired k would also be errors: the feature's own type
    # check wins, as the reference's feature rejections did (interface.py:807-812).
    with pytest.raises(TypeError, match="rotary_cos must be a 2-D torch.float16 tensor"):
        fai.flash_attn_with_kvcache(_t(1, 2, 4, 96), _t(1, 8, 2, 96), _t(1, 8, 2, 96), k=_t(1, 1, 2, 96),
                                    rotary_cos=_t(8, 32), rotary_sin=_t(8, 32))


@pytest.mark.parametrize("kwargs", [dict(window_size=(4, 0)), dict(softcap=30.0), dict(window_size=(-1, 2), softcap=5),
                                    dict(alibi_slopes=_t(4)), dict(cache_leftpad=torch.zeros(1, dtype=torch.int32)),
                                    dict(rotary_cos=_t(8, 16, dtype=torch.float16), rotary_sin=_t(8, 16, dtype=torch.float16),
                                         rotary_interleaved=False)])
def test_window_and_softcap_are_accepted(kwargs):
    # The reference rejects these (interface.py:617-634); here they pass the
    # Python checks (upstream FlashAttention's semantics) and reach the next
    # check, the device of the CPU tensors.
    with pytest.raises(RuntimeError, match="must be CUDA tensors"):
        fai.flash_attn_with_kvcache(_t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64),
                                    cache_seqlens=torch.tensor([3], dtype=torch.int32), **kwargs)
    with pytest.raises(TypeError, match="window_size must be a pair of ints"):
        fai.flash_attn_with_kvcache(_t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), window_size=(1.5, 0))
    with pytest.raises(ValueError, match="softcap must be finite"):
        fai.flash_attn_with_kvcache(_t(1, 2, 4, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), softcap=float("inf"))


def test_pairing_checked_before_head_dim():
    with pytest.raises(ValueError, match="k and v must either both be provided"):
        fai.flash_attn_with_kvcache(_t(1, 2, 4, 96), _t(1, 8, 2, 96), _t(1, 8, 2, 96), k=_t(1, 1, 2, 96))


def test_paged_validation_messages():
    q, kc = _t(2, 1, 4, 64), _t(4, 256, 2, 64)
    seq = torch.tensor([3, 4], dtype=torch.int32)
    with pytest.raises(TypeError, match="block_table must be a torch.int32 tensor"):
        fai.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=seq, block_table=torch.zeros(2, 1, dtype=torch.int64))
    with pytest.raises(ValueError, match=r"block_table must have shape \[batch_size, max_num_blocks_per_seq\]"):
        fai.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=seq, block_table=torch.zeros(3, 1, dtype=torch.int32))
    with pytest.raises(NotImplementedError, match="Paged KV cache does not support cache_batch_idx"):
        fai.flash_attn_with_kvcache(
            q, kc, kc, cache_seqlens=seq, block_table=torch.zeros(2, 1, dtype=torch.int32),
            cache_batch_idx=torch.zeros(2, dtype=torch.int32),
        )
    kc_bad = _t(4, 128, 2, 64)
    with pytest.raises(ValueError, match="Paged KV cache block size must be divisible by 256"):
        fai.flash_attn_with_kvcache(q, kc_bad, kc_bad, cache_seqlens=seq, block_table=torch.zeros(2, 1, dtype=torch.int32))
    with pytest.raises(ValueError, match="num_splits must be non-negative"):
        fai.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=seq, num_splits=-1)


def test_public_signatures_match_reference():
    # Parameter names and defaults of interface.py:448-614, 779-799.
    sig = inspect.signature(fai.flash_attn_with_kvcache)
    names = list(sig.parameters)
    assert names == [
        "q", "k_cache", "v_cache", "k", "v", "rotary_cos", "rotary_sin", "cache_seqlens", "cache_batch_idx",
        "cache_leftpad", "block_table", "softmax_scale", "causal", "window_size", "softcap", "rotary_interleaved",
        "alibi_slopes", "num_splits", "return_softmax_lse", "validate",
    ]
    # The reference's parameters, in order, then one of this build's: validate
    # (keyword, default True = the reference's host-side checks).
    assert sig.parameters["validate"].default is True
    assert sig.parameters["num_splits"].default == 0 and sig.parameters["window_size"].default == (-1, -1)
    assert list(inspect.signature(fai.flash_attn_func).parameters) == ["q", "k", "v", "softmax_scale", "causal"]
    assert list(inspect.signature(fai.flash_attn_varlen_func).parameters) == [
        "q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k", "softmax_scale", "causal",
    ]
    for name in ("flash_attn_qkvpacked_func", "flash_attn_kvpacked_func", "flash_attn_varlen_qkvpacked_func",
                 "flash_attn_varlen_kvpacked_func"):
        assert callable(getattr(fai, name))


def test_extension_exports_reference_bindings():
    for name in ("fwd", "bwd", "varlen_fwd", "varlen_bwd", "fwd_kvcache"):
        assert callable(getattr(flash_attn_turing, name))


def test_extension_rejects_cpu_tensors_with_reference_messages():
    # The C++ layer keeps flash_api.cpp's checks: rank, batch, head_dim, devices.
    with pytest.raises(RuntimeError, match="head_dim 64 or 128"):
        flash_attn_turing.fwd(_t(1, 4, 2, 96), _t(1, 4, 2, 96), _t(1, 4, 2, 96), 0.1, False)
    with pytest.raises(RuntimeError, match="num_heads_q must be divisible by num_heads_k"):
        flash_attn_turing.fwd(_t(1, 4, 3, 64), _t(1, 4, 2, 64), _t(1, 4, 2, 64), 0.1, False)
    with pytest.raises(RuntimeError, match="q, k, v must be rank-4 tensors"):
        flash_attn_turing.fwd(_t(4, 2, 64), _t(4, 2, 64), _t(4, 2, 64), 0.1, False)
    with pytest.raises(RuntimeError, match="CUDA"):
        flash_attn_turing.fwd(_t(1, 4, 2, 64).half(), _t(1, 4, 2, 64).half(), _t(1, 4, 2, 64).half(), 0.1, False)
    with pytest.raises(RuntimeError, match="q, k_cache, v_cache must be CUDA tensors"):
        flash_attn_turing.fwd_kvcache(
            _t(1, 1, 2, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), None, None, torch.zeros(1, dtype=torch.int32),
            None, None, None, None, None, None, None, 0.1, True, -1, -1, 0.0, True, 0,
        )
    with pytest.raises(RuntimeError, match="does not support a preallocated output tensor"):
        flash_attn_turing.fwd_kvcache(
            _t(1, 1, 2, 64), _t(1, 8, 2, 64), _t(1, 8, 2, 64), None, None, torch.zeros(1, dtype=torch.int32),
            None, None, None, None, None, None, _t(1, 1, 2, 64), 0.1, True, -1, -1, 0.0, True, 0,
        )


def test_packed_inputs_are_views():
    # The packed wrappers hand the kernels strided views of the packed tensor
    # (no copies); the gradient helper returns one packed tensor and its slices.
    qkv = _t(2, 5, 3, 4, 64, dtype=torch.float16)
    parts = fai._unpack(qkv, 2, 3)
    for i, t in enumerate(parts):
        assert t.data_ptr() == qkv[:, :, i].data_ptr() and t.stride() == qkv[:, :, i].stride()
    g, (a, b) = fai._packed_grad((torch.Size([7, 2, 3, 64]), torch.float16, torch.device("cpu")), 1, True)
    assert g.shape == (7, 2, 3, 64) and not g.any()
    assert a.data_ptr() == g[:, 0].data_ptr() and b.data_ptr() == g[:, 1].data_ptr()


def test_kvcache_status_errors_match_sync_checks():
    # The status bits of the synchronisation-free mode map to the exceptions and
    # texts of the synchronous checks (capacity: ValueError, as pinned by
    # test_flash_attn.py:2084-2093; cache row: the extension's RuntimeError).
    errs = dict((bit, (exc, msg)) for bit, exc, msg in fai._KV_STATUS_ERRORS)
    assert errs[1] == (ValueError, "cache capacity is insufficient for the requested append length")
    assert errs[2] == (RuntimeError, "cache_batch_idx entries must be within cache batch bounds")
    assert callable(fai.flash_attn_kvcache_check)


def test_kvcache_validate_false_skips_host_capacity_read():
    # With validate=False the capacity is not checked on the host: a CPU call
    # that would fail the capacity check reaches the device check instead.
    q, kc = _t(1, 1, 2, 64, dtype=torch.float16), _t(1, 8, 2, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="cache capacity is insufficient"):
        fai.flash_attn_with_kvcache(q, kc, kc.clone(), cache_seqlens=torch.full((1,), 9, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="must be CUDA tensors"):
        fai.flash_attn_with_kvcache(q, kc, kc.clone(), cache_seqlens=torch.full((1,), 9, dtype=torch.int32),
                                    validate=False)


def test_no_fallback_without_the_native_library(tmp_path):
    # The product path is the native library or an error: the interface cannot
    # be imported without the extension, and the C-ABI loader refuses a
    # missing library (no CPU math path behind either).
    import subprocess
    import sys

    import fa_capi

    code = (
        "import sys; sys.modules['flash_attn_turing'] = None\n"
        "try:\n"
        "    import flash_attention_interface\n"
        "except ImportError:\n"
        "    print('raised')\n"
    )
    env_path = ":".join(sys.path)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                       env={"PYTHONPATH": env_path, "PATH": "/usr/bin:/bin"}, timeout=300)
    assert r.stdout.strip() == "raised", r.stdout + r.stderr
    saved = fa_capi._lib
    try:
        fa_capi._lib = None
        with pytest.raises(ImportError, match="is not built"):
            fa_capi.load(str(tmp_path / "libfa_mi355x.so"))
    finally:
        fa_capi._lib = saved
