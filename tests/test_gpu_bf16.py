"""bf16 inputs (beyond the reference, which accepts fp16 only, README.md:72-75):
forward and backward on the bf16 MFMA against the float64 oracle on the same
bf16-rounded inputs, the (B, N, H, D) views, and the C ABI.

Bars, stated for bf16 (8 significant bits against fp16's 11, so its rounding
unit is 8x fp16's): forward max-abs <= 2.5e-2 and LSE max-abs <= 1e-3 (LSE is
fp32 from exact products), gradients relative L2 <= 2e-2, and on every output
an elementwise bound max |got - ref| / (|ref| + RMS(ref)) <= 6e-2, which a
wrong or stale tile would exceed by far. The reference's max|err|/RMS(ref)
is not used here: on causal dV the largest elements are ~16x the RMS, so
their bf16 rounding alone reaches its fp16-sized 6e-2. Measured: gradients
relative L2 ~2.5e-3, elementwise ~3e-2 (dQ, where dS = P (dP - Dv) is
rounded to bf16 as an MFMA operand).
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import fa_opts, load_capi
from oracle import attention as ora

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF_FWD_MAX_ABS = 2.5e-2
BF_LSE_MAX_ABS = 1e-3
BF_GRAD_REL_L2 = 2e-2
BF_ELEM_REL = 6e-2


def rel_elem(got, ref):
    rms = float(np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(got - ref) / (np.abs(ref) + rms)))


def bf16_inputs(B, Hq, Hkv, N, D, seed):
    """q, k, v, dO from one CPU generator (N(0,1)), rounded to bf16."""
    g = torch.Generator().manual_seed(seed)
    shapes = ((B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D))
    return [torch.randn(*s, generator=g).to(torch.bfloat16) for s in shapes]


def f64(t):
    return t.detach().float().cpu().double().numpy()


def check(o, grads, lse, q, k, v, do, causal, what):
    qn, kn, vn, dn = (f64(t) for t in (q, k, v, do))
    ref_o, ref_lse = ora.attention_fwd(qn, kn, vn, causal)
    err = ora.max_abs(f64(o), ref_o)
    assert err <= BF_FWD_MAX_ABS and rel_elem(f64(o), ref_o) <= BF_ELEM_REL, (what, err)
    if lse is not None:
        assert ora.max_abs(f64(lse), ref_lse) <= BF_LSE_MAX_ABS, what
    for name, g, r in zip(("dQ", "dK", "dV"), grads, ora.attention_bwd(qn, kn, vn, dn, causal)):
        g = f64(g)
        assert np.isfinite(g).all(), (what, name)
        l2 = ora.rel_l2(g, r)
        assert l2 <= BF_GRAD_REL_L2 and rel_elem(g, r) <= BF_ELEM_REL, (what, name, l2)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 2)])
@pytest.mark.parametrize("N", [7, 129, 333, 1000])
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_flash_attn_matches_oracle(D, Hq, Hkv, N, causal):
    import fa_p100
    q, k, v, do = bf16_inputs(1, Hq, Hkv, N, D, seed=N + D + Hkv + causal)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fa_p100.flash_attn(qg, kg, vg, causal)
    assert o.dtype == torch.bfloat16
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert qg.grad.dtype == kg.grad.dtype == vg.grad.dtype == torch.bfloat16
    _, lse = fa_p100._ext.forward_dt(qg.detach(), kg.detach(), vg.detach(), causal)
    check(o, (qg.grad, kg.grad, vg.grad), lse, q, k, v, do, causal,
          f"bf16 D{D} {Hq}/{Hkv} N{N} causal={causal}")


@pytest.mark.parametrize("D", [64, 128])
def test_bf16_bnhd_views_match_dense_bit_for_bit(D):
    import fa_p100
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(2, 8, 2, 300, D, seed=D))
    as_bnhd = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    dense = [t.clone().requires_grad_(True) for t in (q, k, v)]
    views = [as_bnhd(t).detach().requires_grad_(True) for t in (q, k, v)]
    o1 = fa_p100.flash_attn(*dense, True)
    o2 = fa_p100.flash_attn(*views, True)
    o1.backward(do)
    o2.backward(as_bnhd(do))
    torch.cuda.synchronize()
    assert o2.dtype == torch.bfloat16 and torch.equal(o1, o2)
    for a, b in zip(dense, views):
        assert torch.equal(a.grad, b.grad)


def test_bf16_capi_matches_op():
    """fa_fwd_ex / fa_bwd_ex with options {FA_DTYPE_BF16, FA_LAYOUT_BHND} on
    caller-owned buffers give the op's results bit for bit, and the wrong
    format is rejected by the binding with a message."""
    import fa_p100
    lib = load_capi()
    B, Hq, Hkv, N, D, causal = 1, 4, 2, 257, 128, 1
    q, k, v, do = (t.to(DEV) for t in bf16_inputs(B, Hq, Hkv, N, D, seed=3))
    o_op, lse_op = fa_p100._ext.forward_dt(q, k, v, True)
    dq_op, dk_op, dv_op = fa_p100._ext.backward_dt(q, k, v, do, o_op, lse_op, True)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    o, lse = torch.empty_like(q), torch.empty(B, Hq, N, device=DEV)
    opts = fa_opts(dtype=1, layout=0)
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
    with pytest.raises(RuntimeError, match="q, k and v must have one dtype"):
        fa_p100._ext.forward_dt(q, k.half(), v, True)
    with pytest.raises(RuntimeError, match="q must be fp16"):
        fa_p100._ext.forward(q, k, v, True, False)  # the reference's entry stays fp16-only
