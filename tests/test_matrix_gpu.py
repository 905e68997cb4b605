"""The reference suite's whole (seqlen_q, seqlen_k) list on the GPU.

test_flash_attn.py:59-140 lists 80 (sq, sk) pairs (58 distinct): squares,
sq < sk and sq > sk, the tile edges 63/64/65, 127/128/129, 959-961 against
1024 keys, one and two keys (1024 x 1, 1024 x 2, 128 x 1, 64 x 2) and
1025-key ragged ends.  Every distinct pair runs here at batch 1 for
head_dim 64 and 128, causal and not (test_flash_attn.py:51-56), forward
(output and LSE) and backward (dQ, dK, dV), against the fp32 oracle with the
2x-twin bound.  The head pairs (test_flash_attn.py:57) and the softmax scales
(None, 0.3; :54) rotate over the cases.
"""

import itertools

import pytest
import torch

import flash_attention_interface as fai
from helpers import check_fwd_bwd, randn16

REFERENCE_SEQLENS = [
    (64, 64), (64, 128), (64, 256), (128, 64), (256, 64), (128, 128), (1024, 1024), (128, 256), (128, 1024),
    (256, 1024), (512, 1024), (256, 128), (512, 128), (768, 128), (1024, 128), (1024, 256), (63, 63), (65, 65),
    (127, 127), (129, 129), (1, 1), (1, 2), (2, 1), (2, 2), (64, 128), (64, 256), (128, 64), (256, 64), (128, 128),
    (1024, 1024), (128, 256), (128, 1024), (256, 1024), (512, 1024), (256, 128), (512, 128), (768, 128),
    (1024, 128), (1024, 256), (64, 2), (127, 63), (129, 65), (128, 127), (128, 129), (128, 1025), (256, 1025),
    (128, 128), (1024, 1024), (128, 256), (256, 64), (897, 1024), (959, 1024), (960, 1024), (961, 1024),
    (1023, 1024), (1024, 1023), (1024, 897), (1, 64), (1, 128), (65, 64), (65, 128), (129, 64), (129, 128),
    (257, 64), (257, 128), (1, 1024), (1023, 1024), (1025, 1024), (64, 1), (128, 1), (64, 65), (128, 65),
    (64, 129), (128, 129), (64, 257), (128, 257), (1024, 1), (1024, 2), (1024, 1023), (1024, 1025),
]
SEQLENS = sorted(set(REFERENCE_SEQLENS))
HEADS = [(2, 1), (4, 2), (6, 3), (6, 1)]
SCALES = [None, 0.3]
CASES = [
    (sq, sk, hd, causal, HEADS[i % len(HEADS)], SCALES[(i // len(HEADS)) % len(SCALES)])
    for i, ((sq, sk), hd, causal) in enumerate(itertools.product(SEQLENS, [64, 128], [False, True]))
]


def test_case_list_is_the_reference_list():
    assert len(REFERENCE_SEQLENS) == 80 and len(SEQLENS) == 58
    assert len(CASES) == 4 * len(SEQLENS)


@pytest.mark.gpu
@pytest.mark.parametrize("sq,sk,hd,causal,heads,scale", CASES)
def test_reference_seqlen_matrix(device, sq, sk, hd, causal, heads, scale):
    h, hk = heads
    g = torch.Generator().manual_seed(5000 + 7 * sq + 13 * sk + hd + int(causal))
    q = randn16((1, sq, h, hd), g)
    k = randn16((1, sk, hk, hd), g)
    v = randn16((1, sk, hk, hd), g)
    do = randn16((1, sq, h, hd), g)
    s = hd ** -0.5 if scale is None else scale
    qd, kd, vd, dod = (t.to(device) for t in (q, k, v, do))
    out, lse = fai._flash_attn_forward(qd, kd, vd, s, causal)
    dq, dk, dv = fai._flash_attn_backward(dod, qd, kd, vd, out, lse, s, causal)
    torch.cuda.synchronize()
    check_fwd_bwd(f"sq={sq} sk={sk} hd={hd} causal={causal}", q, k, v, do, out.cpu(), lse.cpu(),
                  (dq.cpu(), dk.cpu(), dv.cpu()), s, causal)
