"""Tensors past 2^31 elements on the GPU, against the fp32 oracle (2x-twin bound).

Q, O, dO and dQ of b2 x 262208 x 32 heads x 128 hold 2.148e9 fp16 elements each (4.3 GB), past 2^31, so
any 32-bit element offset in the forward, dQ or dK/dV kernels would wrap.  K and V have 8 heads (GQA
32 / 8), causal.  Checked against the oracle: batch row 1's last 64 query rows (every element of them lies
past 2^31), whose outputs, LSE and dQ depend only on those rows and all keys, and the last 64 keys of that
row, whose dK / dV depend only on the queries at or after them, i.e. the same 64 rows; for KV head 7 and
its query heads 28-31.  The inputs are drawn on the GPU (seeded N(0, 1) in fp16).
"""

import pytest
import torch

import flash_attention_interface as fai
from helpers import assert_2x, assert_lse

B, S, H, HK, D = 2, 262208, 32, 8, 128
TAIL = 64


def test_large_shape_is_past_2_31_elements():
    assert B * S * H * D > 2 ** 31
    # the checked rows start past element 2^31 of Q
    assert ((1 * S + S - TAIL) * H) * D > 2 ** 31


@pytest.mark.gpu
def test_fwd_bwd_past_2_31_elements(device):
    from oracle.attention import attention_bwd, attention_fwd, bwd_fp32_noise
    from oracle.twin import bwd_twin, fwd_twin

    gen = torch.Generator(device=device).manual_seed(4242)
    q = torch.randn((B, S, H, D), generator=gen, device=device, dtype=torch.float16)
    k = torch.randn((B, S, HK, D), generator=gen, device=device, dtype=torch.float16)
    v = torch.randn((B, S, HK, D), generator=gen, device=device, dtype=torch.float16)
    do = torch.randn((B, S, H, D), generator=gen, device=device, dtype=torch.float16)
    scale = D ** -0.5
    print(f"large tensors: b{B} s{S} h{H}/{HK} d{D} causal, Q {q.numel()} elements", flush=True)
    out, lse = fai._flash_attn_forward(q, k, v, scale, True)
    dq, dk, dv = fai._flash_attn_backward(do, q, k, v, out, lse, scale, True)
    torch.cuda.synchronize()

    hq, hkv, rows = slice(28, 32), slice(7, 8), slice(S - TAIL, S)
    qs = q[1:2, rows, hq].cpu()
    dos = do[1:2, rows, hq].cpu()
    ks, vs = k[1:2, :, hkv].cpu(), v[1:2, :, hkv].cpu()
    del q, k, v, do
    # 64 query rows against every key, bottom-right causal: the global mask of those rows.
    o_ref, l_ref = attention_fwd(qs, ks, vs, scale, True)
    o_tw, l_tw = fwd_twin(qs, ks, vs, scale, True)
    assert_2x("out", out[1:2, rows, hq].cpu(), o_ref, o_tw)
    assert_lse(lse[1:2, hq, rows].cpu(), l_ref)
    g_ref = attention_bwd(qs, ks, vs, o_ref, l_ref, dos, scale, True)
    g_tw = bwd_twin(qs, ks, vs, o_tw, l_tw, dos, scale, True)
    noise = bwd_fp32_noise(qs, ks, vs, o_ref, l_ref, dos, scale, True, dt=torch.float32)
    assert_2x("dq", dq[1:2, rows, hq].cpu(), g_ref[0], g_tw[0], noise[0])
    # The last TAIL keys are seen by these rows only.
    for name, got, i in (("dk", dk, 1), ("dv", dv, 2)):
        assert_2x(name, got[1:2, rows, hkv].cpu(), g_ref[i][:, rows], g_tw[i][:, rows], noise[i][:, rows])
