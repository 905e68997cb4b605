"""Write tests/golden/ref_error.json: the rounding-point twin's error against
the fp32 oracle (max-abs per tensor), and the largest fp32-noise widening of
the backward bound, for the inputs of the full-size parity tests and two
small cases a CPU test recomputes.  The GPU parity bound is 2x these errors;
committing them pins the twin (a change to its rounding points changes them).

    python tests/golden/make_ref_error.py [--only KEY ...]

CPU only (the oracle and the twin are PyTorch on the CPU).  The s8192 rows
take a few minutes."""

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
REPO = os.path.dirname(TESTS)
for p in (REPO, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

from helpers import (FULLSIZE, FULLSIZE_KV_CHUNK, c1_inputs, c3_checked_sequences, c3_inputs, dense_inputs,  # noqa: E402
                     max_abs, unit_key)
from oracle.attention import attention_bwd, attention_fwd, bwd_fp32_noise  # noqa: E402
from oracle.twin import bwd_twin, fwd_twin  # noqa: E402

OUT = os.path.join(HERE, "ref_error.json")

# Small cases the CPU suite recomputes: (b, s, h, hk, d, seed, causal).
SMALL = {
    "small_causal_b1_s1024_h4_hk2_d128": (1, 1024, 4, 2, 128, 21, True),
    "small_noncausal_b2_s300_h2_hk1_d64": (2, 300, 2, 1, 64, 22, False),
}


def twin_errors(q, k, v, do, scale, causal, kv_chunk=None):
    """{tensor: max |twin - oracle|} and {tensor: max fp32-noise widening}, chunked over KV heads."""
    hk = k.shape[2]
    groups = q.shape[2] // hk
    kv_chunk = kv_chunk or hk
    err, noise = {}, {}
    for c0 in range(0, hk, kv_chunk):
        c1 = min(hk, c0 + kv_chunk)
        hq, hkv = slice(c0 * groups, c1 * groups), slice(c0, c1)
        qc, kc, vc = q[:, :, hq], k[:, :, hkv], v[:, :, hkv]
        o_ref, l_ref = attention_fwd(qc, kc, vc, scale, causal)
        o_tw, l_tw = fwd_twin(qc, kc, vc, scale, causal)
        err["out"] = max(err.get("out", 0.0), max_abs(o_tw, o_ref))
        if do is None:
            continue
        doc = do[:, :, hq]
        g_ref = attention_bwd(qc, kc, vc, o_ref, l_ref, doc, scale, causal)
        g_tw = bwd_twin(qc, kc, vc, o_tw, l_tw, doc, scale, causal)
        nz = bwd_fp32_noise(qc, kc, vc, o_ref, l_ref, doc, scale, causal, dt=torch.float32)
        for n, r, t, z in zip(("dq", "dk", "dv"), g_ref, g_tw, nz):
            err[n] = max(err.get(n, 0.0), max_abs(t, r))
            noise[n] = max(noise.get(n, 0.0), z.max().item())
    return err, noise


def small_case(key):
    b, s, h, hk, d, seed, causal = SMALL[key]
    q, k, v, do = dense_inputs(b, s, h, d, seed, hk=hk)
    return twin_errors(q, k, v, do, d ** -0.5, causal)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", nargs="*")
    args = ap.parse_args()
    torch.set_num_threads(os.cpu_count() or 1)
    data = json.load(open(OUT)) if os.path.exists(OUT) else {}
    want = lambda key: not args.only or any(key.startswith(o) for o in args.only)  # noqa: E731

    def record(key, err, noise):
        data[key] = {"err_ref": {n: float(f"{x:.6g}") for n, x in err.items()},
                     "noise_max": {n: float(f"{x:.6g}") for n, x in noise.items()}}
        print(key, data[key], flush=True)

    for key in SMALL:
        if want(key):
            record(key, *small_case(key))
    if want("c1"):
        q, k, v = c1_inputs()
        record("c1", *twin_errors(q, k, v, None, 64 ** -0.5, False))
    for name, (b, s, h, d, seed, causal, units) in FULLSIZE.items():
        if not any(want(unit_key(name, u)) for u in units):
            continue
        q, k, v, do = dense_inputs(b, s, h, d, seed)
        for u in units:
            key = unit_key(name, u)
            if want(key):
                t = time.time()
                r, hs = slice(u[0], u[0] + 1), slice(u[1], u[2])
                record(key, *twin_errors(q[r, :, hs], k[r, :, hs], v[r, :, hs], do[r, :, hs], d ** -0.5, causal,
                                         kv_chunk=FULLSIZE_KV_CHUNK.get(name, 4)))
                print(f"  {time.time() - t:.0f} s", flush=True)
    if any(want(f"c3_seq{i}") for i in range(16)):
        lens, cu, q, k, v, do = c3_inputs()
        for i in c3_checked_sequences(lens):
            key = f"c3_seq{i}"
            if want(key):
                a, e = int(cu[i]), int(cu[i + 1])
                record(key, *twin_errors(q[a:e][None], k[a:e][None], v[a:e][None], do[a:e][None], 128 ** -0.5, True,
                                         kv_chunk=4))
    with open(OUT, "w") as f:
        json.dump(dict(sorted(data.items())), f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
