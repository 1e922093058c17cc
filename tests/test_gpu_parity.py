"""GPU parity of the gfx950 kernels against the float64 CPU oracle.

Restates the reference's regression matrix (test_fa_p100.py:56-139) as pytest:
forward over D x (Hq, Hkv) x N x causal x precision tier, gradients over
D x (Hq, Hkv) x N x causal, and the four input regimes, plus the committed
golden fixtures, each through the public `flash_attn` op and through the C ABI.

Bars: forward max-abs <= 4e-3 and LSE max-abs <= 1e-3; dQ/dK/dV relative L2
<= 1e-2; the reference's max|err|/RMS(ref) < 6e-2 on everything.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, ROOT, load_capi,
                     make_inputs, np64)
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _fa():
    import fa_p100
    return fa_p100


def run_flash(q, k, v, do, causal, full_precision=False):
    """Forward + backward through flash_attn; returns numpy o, dq, dk, dv."""
    fa = _fa()
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa.flash_attn(qg, kg, vg, causal, full_precision)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return np64(o), np64(qg.grad), np64(kg.grad), np64(vg.grad)


def check_fwd(o, ref_o, what):
    err = ora.max_abs(o, ref_o)
    rel = ora.rel_max_rms(o, ref_o)
    assert err <= FWD_MAX_ABS and rel < REF_REL, f"{what}: max-abs {err:.3e} rel {rel:.3e}"


def check_grads(got, ref, what):
    for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
        assert np.isfinite(g).all(), f"{what} {name}: non-finite"
        if not np.any(r):
            # e.g. N=1: softmax over one key is constant, so dQ is exactly 0.
            assert np.abs(g).max() <= 1e-6, f"{what} {name}: expected zeros, max {np.abs(g).max():.3e}"
            continue
        l2 = ora.rel_l2(g, r)
        rel = ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rel < REF_REL, f"{what} {name}: rel-L2 {l2:.3e} rel {rel:.3e}"


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (8, 2), (8, 1)])
@pytest.mark.parametrize("N", [1, 7, 63, 64, 65, 333, 1023])
def test_forward_matrix(D, Hq, Hkv, N):
    """test_fa_p100.py:56-78: both causalities, both precision tiers, plus LSE."""
    fa = _fa()
    q, k, v, _ = make_inputs(1, Hq, Hkv, N, D, seed=N * 7 + D + Hkv)
    for causal in (False, True):
        ref_o, ref_lse = ora.attention_fwd(q.numpy(), k.numpy(), v.numpy(), causal)
        for fp in (False, True):
            o = fa.flash_attn(q.to(DEV), k.to(DEV), v.to(DEV), causal, fp)
            check_fwd(np64(o), ref_o, f"fwd D{D} {Hq}/{Hkv} N{N} causal={causal} fp32={fp}")
        o, lse = fa._ext.forward(q.to(DEV), k.to(DEV), v.to(DEV), causal, False)
        assert lse.dtype == torch.float32 and tuple(lse.shape) == (1, Hq, N)
        err = ora.max_abs(np64(lse), ref_lse)
        assert err <= LSE_MAX_ABS, f"lse D{D} {Hq}/{Hkv} N{N} causal={causal}: {err:.3e}"


@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 2), (8, 1)])
@pytest.mark.parametrize("N", [7, 64, 129, 333])
@pytest.mark.parametrize("causal", [False, True])
def test_gradient_matrix(D, Hq, Hkv, N, causal):
    """test_fa_p100.py:82-103, against the float64 analytic backward."""
    q, k, v, do = make_inputs(1, Hq, Hkv, N, D, seed=N * 13 + D + Hkv + causal)
    got = run_flash(q, k, v, do, causal, True)
    ref_o, _ = ora.attention_fwd(q.numpy(), k.numpy(), v.numpy(), causal)
    ref = ora.attention_bwd(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal)
    check_fwd(got[0], ref_o, "fwd")
    check_grads(got[1:], ref, f"grad D{D} {Hq}/{Hkv} N{N} causal={causal}")


@pytest.mark.parametrize("regime,scale", [("1 N(0,1)", 1.0), ("2 large x10", 10.0),
                                          ("3 near-uniform", 0.05), ("4 near-one-hot", 3.0)])
@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_input_regimes(regime, scale, D, causal):
    """test_fa_p100.py:107-139: q, k scaled, v and dO N(0,1), (1,4,256,D).

    The max-abs forward bar is stated for N(0,1)-scale inputs; every regime
    must still meet the relative bars.
    """
    q, k, v, do = make_inputs(1, 4, 4, 256, D, seed=int(scale * 100) + D + causal,
                              scale_qk=scale)
    got = run_flash(q, k, v, do, causal, True)
    ref_o, _ = ora.attention_fwd(q.numpy(), k.numpy(), v.numpy(), causal)
    ref = ora.attention_bwd(q.numpy(), k.numpy(), v.numpy(), do.numpy(), causal)
    check_fwd(got[0], ref_o, f"regime {regime} D{D} causal={causal}")
    check_grads(got[1:], ref, f"regime {regime} D{D} causal={causal}")


# ---------------------------------------------------------------------------
def _golden_cases():
    path = os.path.join(ROOT, "tests", "golden", "attention_cases.npz")
    z = np.load(path)
    n = len([k for k in z.files if k.endswith("_meta")])
    return [(i, {k[len(f"c{i}_"):]: z[k] for k in z.files if k.startswith(f"c{i}_")})
            for i in range(n)]


@pytest.mark.parametrize("idx,case", _golden_cases(), ids=lambda x: str(x) if isinstance(x, int) else "")
def test_golden_fixtures_via_op(idx, case):
    b, hq, hkv, n, d, causal = (int(x) for x in case["meta"])
    q, k, v, do = (torch.from_numpy(case[x]) for x in ("q", "k", "v", "do"))
    got = run_flash(q, k, v, do, bool(causal))
    check_fwd(got[0], case["o"], f"golden {idx}")
    check_grads(got[1:], (case["dq"], case["dk"], case["dv"]), f"golden {idx}")


@pytest.mark.parametrize("idx,case", _golden_cases(), ids=lambda x: str(x) if isinstance(x, int) else "")
def test_golden_fixtures_via_capi(idx, case):
    """Same fixtures through the C ABI (ctypes), with caller-owned buffers."""
    lib = load_capi()
    b, hq, hkv, n, d, causal = (int(x) for x in case["meta"])
    q, k, v, do = (torch.from_numpy(case[x]).to(DEV) for x in ("q", "k", "v", "do"))
    o = torch.empty_like(q)
    lse = torch.empty(b, hq, n, device=DEV, dtype=torch.float32)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = lib.fa_fwd(p(q), p(k), p(v), p(o), p(lse), b, hq, hkv, n, d, causal, 0, stream)
    assert rc == 0, lib.fa_error_string(rc)
    ws_bytes = lib.fa_bwd_workspace_bytes(b, hq, hkv, n, d)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq = torch.full((b, hq, n, d), 7.0, device=DEV)   # fa_bwd must clear it itself
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    rc = lib.fa_bwd(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                    ws_bytes, b, hq, hkv, n, d, causal, stream)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    check_fwd(np64(o), case["o"], f"capi golden {idx}")
    assert ora.max_abs(np64(lse), case["lse"]) <= LSE_MAX_ABS
    check_grads((np64(dq), np64(dk), np64(dv)), (case["dq"], case["dk"], case["dv"]),
                f"capi golden {idx}")


def test_capi_rejects_bad_arguments_without_launching():
    lib = load_capi()
    x = torch.zeros(1, 2, 8, 64, device=DEV, dtype=torch.half)
    lse = torch.zeros(1, 2, 8, device=DEV)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(0)
    assert lib.fa_fwd(p(x), p(x), p(x), p(x), p(lse), 1, 2, 2, 8, 100, 0, 0, s) == 10001
    assert lib.fa_fwd(p(x), p(x), p(x), p(x), p(lse), 1, 2, 2, 0, 64, 0, 0, s) == 10002
    assert lib.fa_fwd(p(x), p(x), p(x), p(x), p(lse), 1, 3, 2, 8, 64, 0, 0, s) == 10003
    assert lib.fa_fwd(None, p(x), p(x), p(x), p(lse), 1, 2, 2, 8, 64, 0, 0, s) == 10005
    ws = torch.zeros(16, device=DEV, dtype=torch.uint8)
    assert lib.fa_bwd(p(x), p(x), p(x), p(x), p(x), p(lse), p(lse), p(x), p(x), p(ws), 16,
                      1, 2, 2, 8, 64, 0, s) == 10006


def test_reference_error_messages_on_device():
    """The binding's TORCH_CHECKs that need device tensors (fa_p100_ext.cu:31-65, 106-113)."""
    fa = _fa()
    h = lambda *s: torch.zeros(*s, device=DEV, dtype=torch.half)
    with pytest.raises(RuntimeError, match="q must be fp16"):
        fa._ext.forward(h(1, 2, 8, 64).float(), h(1, 2, 8, 64), h(1, 2, 8, 64), False, False)
    with pytest.raises(RuntimeError, match=r"q must be \(B, H, N, D\)"):
        fa._ext.forward(h(2, 8, 64), h(1, 2, 8, 64), h(1, 2, 8, 64), False, False)
    with pytest.raises(RuntimeError, match="head dim must be a multiple of 8 from 8 to 256, got 100"):
        fa._ext.forward(h(1, 2, 8, 100), h(1, 2, 8, 100), h(1, 2, 8, 100), False, False)
    with pytest.raises(RuntimeError, match="N must be positive"):
        fa._ext.forward(h(1, 2, 0, 64), h(1, 2, 0, 64), h(1, 2, 0, 64), False, False)
    with pytest.raises(RuntimeError, match=r"query heads \(3\) must be a multiple of key/value heads \(2\)"):
        fa._ext.forward(h(1, 3, 8, 64), h(1, 2, 8, 64), h(1, 2, 8, 64), False, False)
    with pytest.raises(RuntimeError, match="k and v must match"):
        fa._ext.forward(h(1, 2, 8, 64), h(1, 2, 8, 64), h(1, 1, 8, 64), False, False)
    with pytest.raises(RuntimeError, match="k/v must be"):
        fa._ext.forward(h(1, 2, 8, 64), h(1, 2, 9, 64), h(1, 2, 9, 64), False, False)
    with pytest.raises(RuntimeError, match="query heads must be a multiple of kv heads"):
        fa._ext.backward(h(1, 3, 8, 64), h(1, 2, 8, 64), h(1, 2, 8, 64), h(1, 3, 8, 64),
                         h(1, 3, 8, 64), torch.zeros(1, 3, 8, device=DEV), False)
    with pytest.raises(RuntimeError, match="dO must be fp16"):
        fa._ext.backward(h(1, 2, 8, 64), h(1, 2, 8, 64), h(1, 2, 8, 64), h(1, 2, 8, 64).float(),
                         h(1, 2, 8, 64), torch.zeros(1, 2, 8, device=DEV), False)


def test_noncontiguous_inputs_and_current_stream():
    """Transposed-view inputs (what HF passes) and launches on a side stream."""
    fa = _fa()
    q, k, v, do = make_inputs(2, 4, 2, 77, 64, seed=5)
    ref_o, _ = ora.attention_fwd(q.numpy(), k.numpy(), v.numpy(), True)
    qv = q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    kv = k.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    vv = v.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    assert not qv.is_contiguous()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        o = fa.flash_attn(qv, kv, vv, True)
    side.synchronize()
    check_fwd(np64(o), ref_o, "strided inputs on a side stream")


def test_backward_is_deterministic():
    """No atomic adds on results (split key tiles' partials are added by
    whichever workgroup finishes second, and fp32 a + b == b + a): repeated
    runs give bit-identical gradients."""
    q, k, v, do = make_inputs(1, 8, 2, 300, 128, seed=17)
    a = run_flash(q, k, v, do, True)
    b = run_flash(q, k, v, do, True)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("Hq,Hkv,N", [(4, 4, 200), (8, 2, 333), (2, 1, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_half_dq_is_the_rounded_fp32_dq(D, Hq, Hkv, N, causal):
    """backward_half_dq (and fa_bwd_half_dq) write dq as fp16 in the kernel:
    bit-identical to the fp32 dq cast with .to(fp16), dk/dv unchanged."""
    fa = _fa()
    q, k, v, do = (t.to(DEV) for t in make_inputs(1, Hq, Hkv, N, D, seed=D + N))
    o, lse = fa._ext.forward(q, k, v, causal, False)
    dq32, dk32, dv32 = fa._ext.backward(q, k, v, do, o, lse, causal)
    dq16, dk16, dv16 = fa._ext.backward_half_dq(q, k, v, do, o, lse, causal)
    assert dq32.dtype == torch.float32 and dq16.dtype == torch.float16
    assert torch.equal(dq16, dq32.to(torch.float16))
    assert torch.equal(dk16, dk32) and torch.equal(dv16, dv32)
    # Same through the C ABI, into caller-owned buffers.
    lib = load_capi()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    ws_bytes = lib.fa_bwd_workspace_bytes(1, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq = torch.full_like(q, 7.0)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.fa_bwd_half_dq(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                            ws_bytes, 1, Hq, Hkv, N, D, int(causal), stream)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(dq, dq16) and torch.equal(dk, dk16) and torch.equal(dv, dv16)


@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("B,Hq,Hkv,N", [(1, 4, 4, 200), (2, 8, 2, 333), (1, 2, 1, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_bnhd_views_match_dense_bit_for_bit(D, B, Hq, Hkv, N, causal):
    """(B, H, N, D) views of dense (B, N, H, D) storage (what the HF hook
    passes) go through the (B, N, H, D) kernels with no copies; o and the
    gradients are bit-identical to the dense path and come back as views of
    (B, N, H, D) storage."""
    fa = _fa()
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=3 * N + D))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    assert not views[0].is_contiguous() and views[0].transpose(1, 2).is_contiguous()
    o1 = fa.flash_attn(*dense, causal)
    o2 = fa.flash_attn(*views, causal)
    assert o2.transpose(1, 2).is_contiguous()
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for a, b in zip(dense, views):
        assert torch.equal(a.grad, b.grad)


def test_bnhd_capi_matches_dense_capi():
    """fa_fwd_bnhd / fa_bwd_bnhd on (B, N, H, D) buffers against fa_fwd /
    fa_bwd_half_dq on the same logical tensors, bit for bit."""
    lib = load_capi()
    B, Hq, Hkv, N, D, causal = 2, 6, 3, 97, 128, 1
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=11))
    tb = lambda t: t.transpose(1, 2).contiguous()  # (B, N, H, D)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    o, ob = torch.empty_like(q), torch.empty_like(tb(q))
    lse, lseb = (torch.empty(B, Hq, N, device=DEV) for _ in range(2))
    assert lib.fa_fwd(p(q), p(k), p(v), p(o), p(lse), B, Hq, Hkv, N, D, causal, 0, s) == 0
    qb, kb, vb, dob = tb(q), tb(k), tb(v), tb(do)
    assert lib.fa_fwd_bnhd(p(qb), p(kb), p(vb), p(ob), p(lseb), B, Hq, Hkv, N, D, causal, s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dqb, dkb, dvb = torch.empty_like(qb), torch.empty_like(kb), torch.empty_like(vb)
    assert lib.fa_bwd_half_dq(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                              ws_bytes, B, Hq, Hkv, N, D, causal, s) == 0
    assert lib.fa_bwd_bnhd(p(qb), p(kb), p(vb), p(dob), p(ob), p(lseb), p(dqb), p(dkb), p(dvb),
                           p(ws), ws_bytes, B, Hq, Hkv, N, D, causal, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(tb(o), ob) and torch.equal(lse, lseb)
    for a, b in ((dq, dqb), (dk, dkb), (dv, dvb)):
        assert torch.equal(tb(a), b)


@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("B,Hq,Hkv,N", [(1, 4, 4, 1536), (2, 8, 2, 1000)])
def test_split_key_tiles_share_a_workspace_across_calls(D, B, Hq, Hkv, N):
    """Causal backward: the first key tiles' phase-1 work is split between two
    workgroups whose partial dK/dV meet in workspace slots. One workspace
    serves inputs A, then B, then A again, with dk/dv pre-filled with NaN
    each time: A's gradients repeat bit for bit, B's match the oracle (a
    stale, lost or doubly added partial fails one of the two), and the
    split counters are back at zero after each call."""
    lib = load_capi()
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    align = lambda n: (n + 255) // 256 * 256
    c0 = 2 * align(B * Hq * N * 4)
    n_counters = B * Hq * (((N + 127) // 128) // 2)

    def run(seed):
        q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=seed))
        o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
        assert lib.fa_fwd(p(q), p(k), p(v), p(o), p(lse), B, Hq, Hkv, N, D, 1, 0, s) == 0
        dq = torch.empty(B, Hq, N, D, device=DEV)
        dk = torch.full_like(k, float("nan"))
        dv = torch.full_like(v, float("nan"))
        rc = lib.fa_bwd(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                        ws_bytes, B, Hq, Hkv, N, D, 1, s)
        assert rc == 0, lib.fa_error_string(rc)
        torch.cuda.synchronize()
        counters = ws[c0:c0 + 4 * n_counters].view(torch.int32)
        assert int(counters.abs().sum()) == 0, "split counters not reset"
        return (q, k, v, do), (dq.clone(), dk.clone(), dv.clone())

    _, first = run(1)
    inputs_b, got_b = run(2)
    _, again = run(1)
    for x, y in zip(first, again):
        assert torch.equal(x, y)
    q, k, v, do = (t.cpu().numpy() for t in inputs_b)
    ref = ora.attention_bwd(q, k, v, do, True)
    check_grads(tuple(np64(t) for t in got_b), ref, f"split D{D} {B},{Hq}/{Hkv},N{N}")
