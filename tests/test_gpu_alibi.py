"""ALiBi slopes (beyond the reference, which has no positional bias in its
kernels): query head h adds -slope[h] * |i - j| to its scaled score of key j.
flash_attn(..., alibi_slopes=s) against the float64 oracle with the same
slopes (pinned in test_oracle.py against torch SDPA with the bias as a float
mask, the causal per-key identity, a huge-slope closed form and finite
differences), causal and not, GQA/MQA, ragged N, with key lengths and a
sliding window, in bf16, the (B, N, H, D) views and the C ABI.
Bars: the fp16 ones (helpers.py) and the bf16 ones (test_gpu_bf16.py)."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import (FWD_MAX_ABS, GRAD_REL_L2, LSE_MAX_ABS, REF_REL, fa_opts, load_capi,
                     make_inputs, np64)
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"


def slopes_for(h, steep=1.0):
    """The ALiBi paper's geometric slopes 2^(-8 i / h), i = 1 .. h, times `steep`."""
    return np.array([steep * 2.0 ** (-8.0 * (i + 1) / h) for i in range(h)])


def run(q, k, v, do, causal, slopes, lens=None, window=None):
    import fa_p100
    kv_len = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=DEV)
    al = torch.tensor(slopes, dtype=torch.float32, device=DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal, kv_len=kv_len, sliding_window=window,
                           alibi_slopes=al)
    o.backward(do.to(DEV))
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal, kv_len,
                                     window or 0, al)
    torch.cuda.synchronize()
    return o, lse, qg.grad, kg.grad, vg.grad


def check(got, q, k, v, do, causal, slopes, what, lens=None, window=None):
    o, lse, dq, dk, dv = got
    # The kernels use the fp32 slopes; so does the oracle.
    sl = np.float32(slopes).astype(np.float64)
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal, kv_len=lens, window=window, alibi=sl)
    assert ora.max_abs(np64(o), ref_o) <= FWD_MAX_ABS, what
    assert ora.rel_max_rms(np64(o), ref_o) < REF_REL, what
    seen = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(np64(lse)), seen), what
    assert ora.max_abs(np64(lse)[seen], ref_lse[seen]) <= LSE_MAX_ABS, what
    ref = ora.attention_bwd(qn, kn, vn, dn, causal, kv_len=lens, window=window, alibi=sl)
    for name, g, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref):
        g = np64(g)
        assert np.isfinite(g).all(), (what, name)
        l2, rr = ora.rel_l2(g, r), ora.rel_max_rms(g, r)
        assert l2 <= GRAD_REL_L2 and rr < REF_REL, (what, name, l2, rr)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,Hq,Hkv,N,steep", [(2, 4, 4, 300, 1.0), (1, 8, 2, 1000, 1.0),
                                               (1, 4, 1, 2048, 1.0), (1, 4, 2, 129, 16.0),
                                               (1, 2, 2, 7, 0.1)])
def test_alibi_matches_oracle(D, causal, B, Hq, Hkv, N, steep):
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=N + D + causal)
    slopes = slopes_for(Hq, steep)
    got = run(q, k, v, do, causal, slopes)
    check(got, q, k, v, do, causal, slopes,
          f"alibi x{steep} causal={causal} D{D} {B},{Hq}/{Hkv},N{N}")


@pytest.mark.parametrize("D", [64, 128])
def test_alibi_with_key_lengths_and_window(D):
    B, Hq, Hkv, N, lens = 3, 4, 2, 700, [700, 300, 5]
    q, k, v, do = make_inputs(B, Hq, Hkv, N, D, seed=3 * D)
    slopes = slopes_for(Hq)
    check(run(q, k, v, do, False, slopes, lens), q, k, v, do, False, slopes,
          f"alibi lens D{D}", lens=lens)
    check(run(q, k, v, do, True, slopes, lens, 100), q, k, v, do, True, slopes,
          f"alibi lens W100 D{D}", lens=lens, window=100)


def test_alibi_zero_slopes_equal_plain():
    """Zero slopes run the masked instantiation with a zero bias: the same
    attention as without ALiBi (to fp32 rounding, since the masked kernel's
    step order differs only at tails)."""
    import fa_p100
    q, k, v, _ = (t.to(DEV) for t in make_inputs(1, 4, 2, 384, 128, seed=5))
    o0 = fa_p100.flash_attn(q, k, v, True)
    o1 = fa_p100.flash_attn(q, k, v, True, alibi_slopes=torch.zeros(4, device=DEV))
    torch.cuda.synchronize()
    assert (o0.float() - o1.float()).abs().max().item() <= 2e-3


def test_alibi_bf16_and_bnhd_views():
    import fa_p100
    from test_gpu_bf16 import BF_FWD_MAX_ABS, BF_GRAD_REL_L2, bf16_inputs
    B, Hq, Hkv, N, D = 2, 8, 2, 500, 128
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=11))
    al = torch.tensor(slopes_for(Hq), dtype=torch.float32, device=DEV)
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True, alibi_slopes=al)
    o2 = fa_p100.flash_attn(*views, True, alibi_slopes=al)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    for a, b in zip(dense, views):
        assert torch.equal(a.grad, b.grad)
    f = lambda t: t.detach().float().cpu().double().numpy()
    sl = al.double().cpu().numpy()
    ref_o, _ = ora.attention_fwd(f(q), f(k), f(v), True, alibi=sl)
    assert ora.max_abs(f(o1), ref_o) <= BF_FWD_MAX_ABS
    ref = ora.attention_bwd(f(q), f(k), f(v), f(do), True, alibi=sl)
    for t, r in zip(dense, ref):
        assert ora.rel_l2(f(t.grad), r) <= BF_GRAD_REL_L2


def test_alibi_capi_matches_op_and_rejections():
    """fa_fwd_ex / fa_bwd_ex with alibi_slopes in the options give the op's
    results bit for bit; the binding rejects slopes of the wrong shape, type
    or device."""
    import fa_p100
    lib = load_capi()
    B, Hq, Hkv, N, D, causal = 1, 4, 2, 333, 64, 1
    q, k, v, do = (t.to(DEV) for t in make_inputs(B, Hq, Hkv, N, D, seed=8))
    al = torch.tensor(slopes_for(Hq), dtype=torch.float32, device=DEV)
    o_op, lse_op = fa_p100._ext.forward_dt(q, k, v, True, None, 0, al)
    dq_op, dk_op, dv_op = fa_p100._ext.backward_dt(q, k, v, do, o_op, lse_op, True, None, 0, al)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    opts = fa_opts(alibi_slopes=al)
    o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
    assert lib.fa_fwd_ex(p(q), p(k), p(v), p(o), p(lse), B, Hq, Hkv, N, D, causal, opts, s) == 0
    ws_bytes = lib.fa_bwd_workspace_bytes(B, Hq, Hkv, N, D)
    ws = torch.empty(ws_bytes, device=DEV, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    rc = lib.fa_bwd_ex(p(q), p(k), p(v), p(do), p(o), p(lse), p(dq), p(dk), p(dv), p(ws),
                       ws_bytes, B, Hq, Hkv, N, D, causal, opts, s)
    assert rc == 0, lib.fa_error_string(rc)
    torch.cuda.synchronize()
    for a, b in ((o, o_op), (lse, lse_op), (dq, dq_op), (dk, dk_op), (dv, dv_op)):
        assert torch.equal(a, b)
    with pytest.raises(ValueError, match="alibi_slopes"):
        fa_p100.flash_attn(q, k, v, True, alibi_slopes=al[:2])
    with pytest.raises(RuntimeError, match="alibi_slopes"):
        fa_p100._ext.forward_dt(q, k, v, True, None, 0, al.double())
    with pytest.raises(RuntimeError, match="alibi_slopes"):
        fa_p100._ext.forward_dt(q, k, v, True, None, 0, al.cpu())
