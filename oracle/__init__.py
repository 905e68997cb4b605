"""CPU oracle for the MI355X FlashAttention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the HIP library, the
``flash_attn_turing`` extension or ``flash_attention_interface``) imports,
links or executes anything in this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
use it, and only as the checker (or the timed CPU baseline), never as the
thing measured or shipped.

Contents (each function cites the reference file:line it restates):

* ``attention``  - fp32/fp64 math attention: forward with bottom-right causal
  masking, GQA and the zero-row convention; closed-form backward; varlen
  loops.  Restates ``vanilla_attention_ref`` / ``_varlen_reference``
  (test_flash_attn.py:305-368, 467-503), the mask convention of
  csrc/flash_attn/src/mask.h:52-104 and the zero-row rule of
  flash_fwd_kernel.h:616-662.
* ``kvcache``    - in-place append (contiguous, remapped, paged), paged /
  remapped materialisation, split-KV softmax with log-sum-exp combine.
  Restates flash_attention_interface.py:642-776 and
  kvcache_native.cu:191-193, 676-729, 782-871.
* ``twin``       - a rounding-point twin of the reference kernels: fp32 math
  except where the reference kernel rounds to fp16 (P before PV, dS before
  the dQ/dK GEMMs, outputs).  Used to estimate "the reference kernel's own
  error" against the fp32 oracle, because the CUDA reference cannot be built
  or run here (no nvcc, empty CUTLASS submodule, no NVIDIA GPU).

Parity pinning (see tests/test_oracle.py): every function is checked against
closed forms (sq = sk = 1, constant keys, one-hot dominant key, fully masked
rows), float64 brute force on tiny shapes, ``torch.autograd`` in float64 and
central finite differences for the backward, and exact slice / permutation
invariants for the cache functions.  The reference repository ships no golden
vectors for this path.
"""
