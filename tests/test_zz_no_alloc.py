"""fa_bwd_noalloc, the backward entry point that allocates nothing (its two
per-row vectors live in a built-in device scratch array), against fa_bwd on
the same inputs through the C ABI, on two calls in a row, the second with a
smaller input (the scratch keeps the first call's contents), plus the float64
oracle on one (batch, head) slice at the fp16 bars, and the size limit.

dq comes out of the same phase-2 code in both entry points: bit-identical.
fa_bwd splits short causal key tiles' dK/dV work between two workgroups and
adds the two fp32 partials; fa_bwd_noalloc (no workspace slots) does not, so
dk and dv may differ in the last bits of a few elements under causal masking
and are bit-identical without it."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import GRAD_REL_L2, load_capi, make_inputs, np64
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
FA_ERR_SCRATCH = 10013


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _run(lib, q, k, v, do, causal, noalloc):
    B, Hq, N, D = q.shape
    Hkv = k.size(1)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, N, device=DEV)
    assert lib.fa_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, Hq, Hkv, N, D,
                      int(causal), 0, stream) == 0
    dq = torch.full((B, Hq, N, D), float("nan"), device=DEV)
    dk = torch.full_like(k, float("nan"))
    dv = torch.full_like(v, float("nan"))
    if noalloc:
        rc = lib.fa_bwd_noalloc(_ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(o), _ptr(lse),
                                _ptr(dq), _ptr(dk), _ptr(dv), B, Hq, Hkv, N, D, int(causal),
                                stream)
    else:
        ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        rc = lib.fa_bwd(_ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(o), _ptr(lse), _ptr(dq),
                        _ptr(dk), _ptr(dv), _ptr(ws), ws_bytes, B, Hq, Hkv, N, D, int(causal),
                        stream)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    return dq, dk, dv


def test_noalloc_matches_fa_bwd_on_two_calls_second_smaller():
    lib = load_capi()
    for B, Hq, Hkv, N, D, causal in [(1, 8, 8, 2048, 128, True), (2, 4, 2, 700, 64, False),
                                     (1, 4, 1, 1000, 64, True)]:
        print(f"case B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal}", flush=True)
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=N))
        ref = _run(lib, q, k, v, do, causal, noalloc=False)
        got = _run(lib, q, k, v, do, causal, noalloc=True)
        for name, g, r in zip(("dq", "dk", "dv"), got, ref):
            assert torch.isfinite(g).all(), name
            if name == "dq" or not causal:
                assert torch.equal(g, r), name
            else:
                d = (g.float() - r.float()).abs().max().item()
                assert d <= 2e-3 * r.float().abs().max().item(), (name, d)
                rel = ((g.float() - r.float()).norm() / r.float().norm()).item()
                assert rel <= 1e-4, (name, rel)
        # One (batch, head) slice against the float64 oracle at the fp16 bars.
        hq, hk = Hq - 1, (Hq - 1) // (Hq // Hkv)
        sl = lambda t, h: np64(t[B - 1:B, h:h + 1])
        dq_ref, dk_ref, dv_ref = ora.attention_bwd(sl(q, hq), sl(k, hk), sl(v, hk), sl(do, hq),
                                                   causal)
        assert ora.rel_l2(sl(got[0], hq), dq_ref) <= GRAD_REL_L2
        if Hq == Hkv:
            assert ora.rel_l2(sl(got[1], hk), dk_ref) <= GRAD_REL_L2
            assert ora.rel_l2(sl(got[2], hk), dv_ref) <= GRAD_REL_L2


def test_noalloc_rejects_shapes_beyond_its_scratch():
    lib = load_capi()
    q = torch.zeros(1, 1, 8, 64, dtype=torch.half, device=DEV)
    p = _ptr(q)
    dq = torch.zeros(1, 1, 8, 64, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # 2^21 + 1 rows: one more than two per-row vectors in 16 MiB allow; no
    # pointer is dereferenced (the check comes first).
    rc = lib.fa_bwd_noalloc(p, p, p, p, p, _ptr(dq), _ptr(dq), p, p, 1, 1, 1, (1 << 21) + 1, 64,
                            1, stream)
    assert rc == FA_ERR_SCRATCH
    assert b"scratch" in lib.fa_error_string(rc)
