"""Writes the small golden fixtures in tests/golden/attention_cases.npz.

    python tests/golden/gen_golden.py

The reference commits no golden vectors (its tests draw fresh CUDA randoms,
test_fa_p100.py:41), so the fixtures are produced here by the float64 CPU
oracle (oracle/attention.py), which tests/test_oracle.py pins against finite
differences, torch's float64 SDPA and closed forms. Inputs are fp16 (the
kernels' input type) drawn from a seeded CPU generator; expected outputs are
float32 roundings of the float64 results. The cases cover what the reference's
suite stresses: both head dims, MHA/GQA/MQA, N of 1, below one tile, straddling
tile edges and ragged, causal and dense.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import attention as ora  # noqa: E402

# (B, Hq, Hkv, N, D, causal, input scale)
CASES = [
    (1, 2, 2, 1, 64, True, 1.0),
    (1, 2, 1, 7, 64, False, 1.0),
    (1, 4, 2, 65, 64, True, 1.0),
    (2, 2, 2, 33, 128, False, 1.0),
    (1, 2, 1, 129, 128, True, 1.0),
    (1, 1, 1, 200, 128, True, 3.0),
    (1, 2, 2, 96, 64, False, 0.05),
]


def main():
    out = {}
    for idx, (b, hq, hkv, n, d, causal, s) in enumerate(CASES):
        g = torch.Generator().manual_seed(1000 + idx)
        q = (torch.randn(b, hq, n, d, generator=g) * s).half().numpy()
        k = (torch.randn(b, hkv, n, d, generator=g) * s).half().numpy()
        v = torch.randn(b, hkv, n, d, generator=g).half().numpy()
        do = torch.randn(b, hq, n, d, generator=g).half().numpy()
        o, lse = ora.attention_fwd(q, k, v, causal)
        dq, dk, dv = ora.attention_bwd(q, k, v, do, causal)
        p = f"c{idx}_"
        out[p + "meta"] = np.array([b, hq, hkv, n, d, int(causal)], dtype=np.int64)
        for name, arr in (("q", q), ("k", k), ("v", v), ("do", do)):
            out[p + name] = arr
        for name, arr in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
            out[p + name] = arr.astype(np.float32)
    path = os.path.join(HERE, "attention_cases.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {len(CASES)} cases to {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
